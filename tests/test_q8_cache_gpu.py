"""GPU parity of KQKV over an 8-bit (Q8_0) latent cache (kqkv_decode_q8.hip).

The reference has no such cache type, so parity is split in two:
  * kernel error: the kernel against the CPU oracle (the unfused ggml graph) run on the f16 values
    the kernel computes with, f16(q * d) (oracle.q8_0_dequant_f16), at the f16-cache bars of
    test_kqkv_gpu.py (max abs <= 1e-2, relative to max|ref| <= 3e-3) and against a float64 brute
    force on the same values (relative <= 1e-3);
  * quantisation error: the oracle on those values against the oracle on the original cache, which
    must stay within the bound the score perturbation fixes: with ds = kq_scale max|q . dk| over
    heads and keys (dk = dequantised - original, computed in float64), softmax weights move by at
    most a factor e^(2 ds), so |do| <= max|v| (e^(2 ds) - 1) + max|dv|.
The cache is quantised by ggml's quantize_row_q8_0_ref (oracle.q8_0_quantize, pinned in
test_oracle_q8.py).  Cases: config 3's 32K-key step, the single-split direct path, ragged windows
with masked holes and a masked tail, long splits (the int8 ring cycling over many tiles), the
reference's (320, 256) geometry, several rows, and sharp scores that move the lazy reference max.
From 16 tokens (chunked prefill) the op runs the f16 prefill kernel on an f16 copy of the cache
that it writes into its workspace: those results must equal the op over an F16 cache holding the
same values bit for bit.
"""
import numpy as np
import pytest
import torch

import aubier_amd as A
from aubier_amd import inputs as I
from oracle import oracle as orc

from conftest import errs, say

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0 / np.sqrt(192.0)))


def q8_cache(kc_f16, dev):
    dk = kc_f16.shape[1]
    wq = orc.q8_0_quantize(kc_f16.astype(np.float32))
    return wq, orc.q8_0_dequant_f16(wq, dk), A.Q8_0(torch.from_numpy(wq).to(dev), dk)


def run(kq, q_d, m_d, n_split, dv):
    if n_split is None:
        out = A.ggml_m4_kqkv(kq, q_d, m_d, SCALE)
    else:
        part = A.ggml_m4_kqkv_partial(kq, q_d, m_d, SCALE, n_split, d_v=dv)
        out = A.ggml_m4_phase_merge(part, n_head=q_d.shape[1], d_v=dv)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(name, got, ref, abs_tol, rel_tol):
    ea, er, rr = errs(got, ref)
    say(f"{name}: max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}")
    assert np.isfinite(got).all(), name
    assert ea <= abs_tol and er <= rel_tol, (name, ea, er)
    return ea


def quant_bound(kc, deq, q, dv):
    """max |do| the quantisation can cause (module docstring), in float64."""
    dk = deq.astype(np.float64) - kc.astype(np.float64)
    ds = SCALE * np.abs(q.reshape(-1, q.shape[-1]).astype(np.float64) @ dk.T).max()
    return float(np.abs(kc[:, :dv].astype(np.float64)).max() * np.expm1(2.0 * ds) + np.abs(dk[:, :dv]).max()), ds


def test_config3_q8_cache(dev):
    """Config 3 (32,768 keys, 32 heads, one token) with its cache in Q8_0, the library's split count."""
    inp = I.make_config(3)
    dv = I.D_V
    wq, deq, kq = q8_cache(inp.kcache, dev)
    # Qcur as the step builds it (WKB on the GPU, then the rope part)
    from gpu_util import upload
    g = upload(inp, dev)
    A.ggml_m4_wkb(g["w_kb"], g["q"][:, :, :I.D_NOPE], out=g["qcur"][:, :, :I.D_V])
    torch.cuda.synchronize()
    q = g["qcur"].cpu().numpy()
    out = run(kq, g["qcur"], g["mask"], None, dv)
    ref_deq = orc.kqkv(deq, q, inp.mask, inp.kq_scale)
    ek = check("cfg3 q8: kernel vs oracle(dequantised)", out, ref_deq, 1e-2, 3e-3)
    ref64 = orc.attn_f64(deq, q[:, :4], inp.mask, inp.kq_scale)
    check("cfg3 q8: kernel vs f64(dequantised), heads 0-3", out[:4], ref64, 1e-2, 1e-3)
    ref_orig = orc.kqkv(inp.kcache, q, inp.mask, inp.kq_scale)
    eq, _, _ = errs(ref_deq, ref_orig)
    bound, ds = quant_bound(inp.kcache, deq, q, dv)
    say(f"cfg3 q8: quantisation error {eq:.3e} (bound {bound:.3e}, max score shift {ds:.3e}); kernel error {ek:.3e}")
    assert eq <= bound
    # bytes per key: 612 of cache + 4 of mask against 1,152 + 4
    assert wq.shape[1] == 612


@pytest.mark.parametrize("dk,dv,n_kv,nt,splits,holes,q_scale", [
    (576, 512, 4197, 1, (None, 1, 3, 64), True, 0.05),      # ragged window, holes + masked tail
    (576, 512, 8192, 1, (2, 5), False, 0.05),               # 64 and 26 tiles per split: the ring cycles
    (320, 256, 3000, 1, (None, 1, 7), True, 0.05),          # the reference geometry
    (576, 512, 2048, 3, (None, 4), True, 0.05),             # several rows
    (576, 512, 6000, 1, (None, 2, 40), True, 300.0),        # sharp: the lazy reference max moves
])
def test_q8_cache_cases(dev, dk, dv, n_kv, nt, splits, holes, q_scale):
    H = 32
    kc = I.randn(7200 + dk, n_kv * dk).astype(np.float16).reshape(n_kv, dk)
    q = I.randn(7201 + nt, nt * H * dk, q_scale).reshape(nt, H, dk)
    mask = np.zeros((nt, n_kv), dtype=np.float32)
    if holes:
        for t in range(nt):
            mask[t, (5 + t)::37] = -np.inf
            mask[t, n_kv - 90 - 7 * t:] = -np.inf
    wq, deq, kq = q8_cache(kc, dev)
    ref = orc.kqkv(deq, q, mask, SCALE, d_v=dv)
    ref64 = orc.attn_f64(deq, q[:, :4], mask, SCALE, d_v=dv)
    q_d, m_d = torch.from_numpy(q).to(dev), torch.from_numpy(mask).to(dev)
    # sharp (q_scale 300) bars at ~2x the MI355X's measured errors: max_rel vs the oracle <= 4.45e-4,
    # vs float64 <= 1.45e-3
    rel = 1e-3 if q_scale > 1 else 3e-3
    for S in splits:
        out = run(kq, q_d, m_d, S, dv)
        tag = f"q8 {dk}/{dv} n_kv={n_kv} nt={nt} S={S} q_scale={q_scale}"
        check(f"{tag} vs oracle(dequantised)", out, ref, 1e-2, rel)
        check(f"{tag} vs f64(dequantised), heads 0-3", out[:4], ref64, 1e-2, 3e-3 if q_scale > 1 else 1e-3)
    if q_scale <= 1:
        eq, _, _ = errs(ref, orc.kqkv(kc, q, mask, SCALE, d_v=dv))
        bound, ds = quant_bound(kc, deq, q, dv)
        say(f"quantisation error {eq:.3e} (bound {bound:.3e})")
        assert eq <= bound


def test_q8_cache_max_context(dev):
    """Config 4's window (262,144 keys, 16 tiles per split, its masked tail of 1000-valued rows)
    quantised to Q8_0: all 32 heads against the float64 brute force on the dequantised values at
    the f16-cache relative bar (1e-3), and against the F16-cache op over those same values."""
    inp = I.make_config(4)
    _, deq, kq = q8_cache(inp.kcache, dev)
    q = I.randn(7800, 32 * 576, 0.05).reshape(1, 32, 576)
    q_d, m_d = torch.from_numpy(q).to(dev), torch.from_numpy(inp.mask).to(dev)
    out = run(kq, q_d, m_d, None, 512)
    ref64 = orc.attn_f64(deq, q, inp.mask, SCALE)
    ea, er, rr = errs(out, ref64)
    say(f"q8 262,144 keys vs f64(dequantised): max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}")
    assert np.isfinite(out).all() and er <= 1e-3
    via_f16 = run(torch.from_numpy(deq).to(dev), q_d, m_d, None, 512)
    check("q8 262,144 keys vs the F16 op on the same values", out, via_f16, 1e-2, 1e-3)


def causal_chunk(n_kv, nt, dk, H, seed):
    kc = I.randn(seed, n_kv * dk).astype(np.float16).reshape(n_kv, dk)
    q = I.randn(seed + 1, nt * H * dk, 0.05).reshape(nt, H, dk)
    mask = np.zeros((nt, n_kv), dtype=np.float32)
    for t in range(nt):
        mask[t, n_kv - nt + t + 1:] = -np.inf
    return kc, q, mask


@pytest.mark.parametrize("n_seq,region,splits", [(4, 2048, (None, 3)), (8, 1536, (None, 64))])
def test_q8_cache_batch_decode(dev, n_seq, region, splits):
    """Batch-of-N decode over per-sequence regions (inputs.make_batch) of a Q8_0 cache: each row's
    splits outside its region record empty splits; against the oracle on the dequantised cache."""
    inp = I.make_batch(n_seq, region)
    _, deq, kq = q8_cache(inp.kcache, dev)
    q = I.randn(7700 + n_seq, n_seq * 32 * 576, 0.05).reshape(n_seq, 32, 576)
    q_d, m_d = torch.from_numpy(q).to(dev), torch.from_numpy(inp.mask).to(dev)
    ref = orc.kqkv(deq, q, inp.mask, SCALE)
    for S in splits:
        out = run(kq, q_d, m_d, S, 512)
        check(f"q8 batch N={n_seq} x {region} S={S} vs oracle(dequantised)", out, ref, 1e-2, 3e-3)


@pytest.mark.parametrize("dk,dv", [(576, 512), (320, 256)])
def test_q8_cache_chunked_prefill(dev, dk, dv):
    """A chunk of 20 tokens over a Q8_0 cache with a causal mask (token i sees the cached keys and
    new keys up to its own).  From 16 tokens the op writes the cache's f16 values into its
    workspace and runs the f16 prefill kernel on them: the result is bit-identical to the op over
    an F16 cache holding those values, and within the f16 bars of the oracle."""
    n_kv, nt, H = 1500, 20, 32
    kc, q, mask = causal_chunk(n_kv, nt, dk, H, 7400)
    _, deq, kq = q8_cache(kc, dev)
    q_d, m_d = torch.from_numpy(q).to(dev), torch.from_numpy(mask).to(dev)
    ref = orc.kqkv(deq, q, mask, SCALE, d_v=dv)
    out = run(kq, q_d, m_d, None, dv)
    check(f"q8 chunked prefill {dk}/{dv} nt=20 vs oracle(dequantised)", out, ref, 1e-2, 3e-3)
    via_f16 = run(torch.from_numpy(deq).to(dev), q_d, m_d, None, dv)
    assert np.array_equal(out, via_f16)
    # the explicit-split entry point keeps the per-token 8-bit kernel (include/mla_m4.h says so):
    # the same bars against the oracle, and against the op's f16-copy path on the same operands
    out_p = run(kq, q_d, m_d, 7, dv)
    check(f"q8 chunked prefill {dk}/{dv} nt=20 S=7 (8-bit kernel) vs oracle(dequantised)", out_p, ref, 1e-2, 3e-3)
    check(f"q8 chunked prefill {dk}/{dv} nt=20 S=7 (8-bit kernel) vs mla_m4_kqkv (f16 copy)", out_p, out, 1e-2, 3e-3)


def test_q8_cache_prefill_config5_shape(dev):
    """Config 5's shape (512 tokens x 8,192 keys, causal) over a Q8_0 cache: bit-identical to the
    op over the dequantised F16 cache, and the first and last 8 tokens against the oracle."""
    n_kv, nt, dk, dv, H = 8192, 512, 576, 512, 32
    kc, q, mask = causal_chunk(n_kv, nt, dk, H, 7500)
    _, deq, kq = q8_cache(kc, dev)
    q_d, m_d = torch.from_numpy(q).to(dev), torch.from_numpy(mask).to(dev)
    out = run(kq, q_d, m_d, None, dv)
    via_f16 = run(torch.from_numpy(deq).to(dev), q_d, m_d, None, dv)
    assert np.array_equal(out, via_f16)
    for sl in (slice(0, 8), slice(nt - 8, nt)):
        ref = orc.kqkv(deq, np.ascontiguousarray(q[sl]), np.ascontiguousarray(mask[sl]), SCALE, d_v=dv)
        check(f"q8 prefill 512 x 8192, tokens {sl.start}..{sl.stop - 1} vs oracle(dequantised)", out[:, sl], ref, 1e-2, 3e-3)


def test_q8_cache_prefill_noalloc_matches(dev):
    """The no-allocation entry point over a Q8_0 prefill chunk whose f16 copy and partials fit
    its scratch (1.2 MB of copy, 16 splits x 16 tokens of partials): bit-identical with
    ggml_m4_kqkv."""
    n_kv, nt, dk, H = 1024, 16, 576, 32
    kc, q, mask = causal_chunk(n_kv, nt, dk, H, 7600)
    _, _, kq = q8_cache(kc, dev)
    q_d, m_d = torch.from_numpy(q).to(dev), torch.from_numpy(mask).to(dev)
    a = A.ggml_m4_kqkv(kq, q_d, m_d, SCALE)
    b = A.ggml_m4_kqkv_noalloc(kq, q_d, m_d, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_q8_cache_noalloc_matches(dev):
    """The no-allocation entry point runs the same Q8_0 kernels: bit-exact with ggml_m4_kqkv."""
    n_kv, dk = 32768, 576
    kc = I.randn(7300, n_kv * dk).astype(np.float16).reshape(n_kv, dk)
    q = I.randn(7301, 32 * dk, 0.05).reshape(1, 32, dk)
    _, _, kq = q8_cache(kc, dev)
    q_d = torch.from_numpy(q).to(dev)
    a = A.ggml_m4_kqkv_noalloc(kq, q_d, None, SCALE)
    b = A.ggml_m4_kqkv(kq, q_d, None, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(a, b)

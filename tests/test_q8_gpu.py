"""GPU parity of the reference geometry's quantised ops through the C ABI: GGML_OP_M4_WKB with a
Q8_0 W_kb, GGML_OP_M4_PHASE phase 1 (wv_b) and phase 0 (KV-write), against the oracle's
restatements of the reference kernels (patches/ggml-m4/m4-wkb.cu:21-69, m4-phase.cu:52-200;
tests/test_oracle_q8.py pins those).

Bars: WKB and wv_b are integer dots with the reference's f32 accumulation order, so they must be
bit-identical to the oracle.  KV-write's gemv is bit-identical too (seen directly in the rope rows
at pos = 0, where the rotation is the identity); the RMS norm uses the hardware rsqrt (the
reference's rsqrtf; the oracle divides by sqrtf): <= 4 ulp; the rope rows use the device's powf /
sinf / cosf (the oracle the C library's): |err| <= 1e-6 + 4e-7 pos max|x|, the f32 resolution of
an angle of size pos.  The cache row must equal f16(dst) and be the only row written.  With an
8-bit (Q8_0) cache -- an extension, the reference's cache is f16 -- the row must hold exactly
ggml's quantize_row_q8_0_ref of dst (oracle.q8_0_quantize, pinned in test_oracle_q8.py), and dst
must be the f16-cache launch's, bit for bit.
"""
import numpy as np
import pytest
import torch

import aubier_amd as A
from oracle import oracle as orc

from conftest import errs, say

pytestmark = pytest.mark.gpu


def q8_dev(blocks_np: np.ndarray, lead_shape, ne0: int, dev) -> A.Q8_0:
    b = torch.from_numpy(np.ascontiguousarray(blocks_np)).reshape(*lead_shape, ne0 // 32 * 34).to(dev)
    return A.Q8_0(b, ne0)


@pytest.mark.parametrize("d_n,d_v", [(64, 256), (128, 512)])
@pytest.mark.parametrize("nt", [1, 3])
def test_wkb_q8_bit_exact(dev, d_n, d_v, nt):
    """The reference's W_kb form: Q8_0 [d_n, D_v, 32] against q_nope viewed out of q with a
    (d_n + 64)-float head stride (m4-wkb.cu:76 asserts the 128-float stride at d_n = 64)."""
    H = 32
    w = orc.q8_0_random(8100 + d_n, H * d_v, d_n)
    q = np.random.default_rng(8101).standard_normal((nt, H, d_n + 64)).astype(np.float32) * 0.05
    ref = orc.wkb_q8(w, d_n, d_v, H, np.ascontiguousarray(q[:, :, :d_n]))
    qd = torch.from_numpy(q).to(dev)
    out = A.ggml_m4_wkb(q8_dev(w, (H, d_v), d_n, dev), qd[:, :, :d_n])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    say(f"WKB Q8_0 d_n={d_n} D_v={d_v} nt={nt}: max|diff|={np.abs(got - ref).max():.3e}")
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("d_in,d_out", [(256, 128), (512, 128)])
@pytest.mark.parametrize("nt", [1, 5])
def test_wvb_q8_bit_exact(dev, d_in, d_out, nt):
    H = 32
    w = orc.q8_0_random(8200 + d_in, H * d_out, d_in)
    x = np.random.default_rng(8201).standard_normal((H, nt, d_in)).astype(np.float32) * 0.05   # [H][nt][d_in]
    ref = orc.wvb_q8(w, d_in, d_out, H, np.ascontiguousarray(x.transpose(1, 0, 2))).transpose(1, 0, 2)
    out = A.ggml_m4_phase_wvb(q8_dev(w, (H, d_out), d_in, dev), torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    say(f"wv_b Q8_0 d_in={d_in} d_out={d_out} nt={nt}: max|diff|={np.abs(got - ref).max():.3e}")
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(ref).view(np.uint32))


RP_PLAIN = dict(freq_base=10000.0, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
                eps=1e-6, n_ctx_orig=4096)
RP_YARN = dict(freq_base=1e6, freq_scale=0.25, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
               eps=1e-5, n_ctx_orig=8192)


@pytest.mark.parametrize("n_embd,d_lat", [(4096, 256), (7168, 512)])
@pytest.mark.parametrize("pos", [0, 77, 5000])
@pytest.mark.parametrize("yarn", [False, True])
def test_kvwrite(dev, n_embd, d_lat, pos, yarn):
    n_rope, n_kv, row = 64, 300, 123
    n_out = d_lat + n_rope
    rng = np.random.default_rng(8300)
    w = orc.q8_0_random(8301, n_out, n_embd, scale=0.002)
    cur = rng.standard_normal(n_embd).astype(np.float32)
    nw = (1.0 + 0.25 * rng.standard_normal(d_lat)).astype(np.float32)
    kc0 = rng.standard_normal((n_kv, n_out)).astype(np.float16)
    rp = RP_YARN if yarn else RP_PLAIN
    kc_ref = kc0.view(np.uint16).copy()
    ref = orc.kvwrite(cur, w, d_lat, n_rope, nw, kc_ref, row, pos, rp)

    kc_d = torch.from_numpy(kc0.copy()).to(dev)
    out = A.ggml_m4_phase_kvwrite(torch.from_numpy(cur).to(dev), q8_dev(w, (n_out,), n_embd, dev),
                                  torch.from_numpy(nw).to(dev), kc_d, torch.tensor([row], dtype=torch.int64, device=dev),
                                  torch.tensor([pos], dtype=torch.int32, device=dev),
                                  A.rope_params(n_dims=n_rope, **rp))
    torch.cuda.synchronize()
    got, kc = out.cpu().numpy(), kc_d.cpu().numpy()
    lat_ulp = np.abs(got[:d_lat] - ref[:d_lat]) / np.spacing(np.abs(ref[:d_lat]).astype(np.float32))
    rope_err = np.abs(got[d_lat:] - ref[d_lat:]).max()
    say(f"KV-write {n_embd}->{d_lat}+{n_rope} pos={pos} yarn={yarn}: latent max ulp {lat_ulp.max():.1f}, "
        f"rope max|err| {rope_err:.3e}")
    assert lat_ulp.max() <= 4
    if pos == 0 and not yarn:                  # identity rotation: the gemv itself, bit for bit
        assert np.array_equal(got[d_lat:].view(np.uint32), ref[d_lat:].view(np.uint32))
    assert rope_err <= 1e-6 + 4e-7 * pos * np.abs(ref[d_lat:]).max() * (1.0 + 0.1 * np.log(4.0) if yarn else 1.0)
    # the cache: row `row` is f16(dst), every other row untouched
    assert np.array_equal(kc[row].view(np.uint16), got.astype(np.float16).view(np.uint16))
    others = np.ones(n_kv, bool)
    others[row] = False
    assert np.array_equal(kc[others].view(np.uint16), kc0[others].view(np.uint16))
    ea, _, _ = errs(kc[row].astype(np.float32), kc_ref[row].view(np.float16).astype(np.float32))
    assert ea <= 1e-3 * max(1.0, np.abs(ref).max())


def test_kvwrite_row_outside_cache_is_not_written(dev):
    n_embd, d_lat, n_rope, n_kv = 4096, 256, 64, 16
    n_out = d_lat + n_rope
    w = orc.q8_0_random(8400, n_out, n_embd, scale=0.002)
    cur = np.random.default_rng(8401).standard_normal(n_embd).astype(np.float32)
    nw = np.ones(d_lat, dtype=np.float32)
    kc0 = np.random.default_rng(8402).standard_normal((n_kv, n_out)).astype(np.float16)
    kc_d = torch.from_numpy(kc0.copy()).to(dev)
    args = (torch.from_numpy(cur).to(dev), q8_dev(w, (n_out,), n_embd, dev), torch.from_numpy(nw).to(dev), kc_d)
    for bad in (n_kv, n_kv + 5, -1):
        out = A.ggml_m4_phase_kvwrite(*args, torch.tensor([bad], dtype=torch.int64, device=dev),
                                      torch.tensor([3], dtype=torch.int32, device=dev), A.rope_params(n_dims=n_rope, **RP_PLAIN))
        torch.cuda.synchronize()
        assert np.isfinite(out.cpu().numpy()).all()
    assert np.array_equal(kc_d.cpu().numpy().view(np.uint16), kc0.view(np.uint16))


@pytest.mark.parametrize("n_embd,d_lat,pos,yarn", [(4096, 256, 77, False), (7168, 512, 5000, True)])
def test_kvwrite_q8_cache(dev, n_embd, d_lat, pos, yarn):
    """KV-write into a Q8_0 cache, then KQKV reads the row back: the stored blocks are the oracle's
    quantisation of the launch's own Kcur, every other row is untouched, and KQKV over the cache
    sees f16(q * d) of that row."""
    n_rope, n_kv, row = 64, 300, 123
    n_out = d_lat + n_rope
    rng = np.random.default_rng(8500 + d_lat)
    w = orc.q8_0_random(8501, n_out, n_embd, scale=0.002)
    cur = rng.standard_normal(n_embd).astype(np.float32)
    nw = (1.0 + 0.25 * rng.standard_normal(d_lat)).astype(np.float32)
    kc0 = orc.q8_0_quantize(rng.standard_normal((n_kv, n_out)).astype(np.float32))
    rp = A.rope_params(n_dims=n_rope, **(RP_YARN if yarn else RP_PLAIN))
    args = (torch.from_numpy(cur).to(dev), q8_dev(w, (n_out,), n_embd, dev), torch.from_numpy(nw).to(dev))
    kidx, pos_d = torch.tensor([row], dtype=torch.int64, device=dev), torch.tensor([pos], dtype=torch.int32, device=dev)
    kc_q = torch.from_numpy(kc0.copy()).to(dev)
    out = A.ggml_m4_phase_kvwrite(*args, A.Q8_0(kc_q, n_out), kidx, pos_d, rp)
    kc_h = torch.zeros((n_kv, n_out), dtype=torch.float16, device=dev)
    out_h = A.ggml_m4_phase_kvwrite(*args, kc_h, kidx, pos_d, rp)
    torch.cuda.synchronize()
    got, kc = out.cpu().numpy(), kc_q.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), out_h.cpu().numpy().view(np.uint32))
    want = orc.q8_0_quantize(got[None, :])[0]
    say(f"KV-write Q8_0 {n_embd}->{d_lat}+{n_rope} pos={pos}: {np.count_nonzero(kc[row] != want)} bytes differ")
    assert np.array_equal(kc[row], want)
    others = np.ones(n_kv, bool)
    others[row] = False
    assert np.array_equal(kc[others], kc0[others])
    # the row as KQKV reads it: one head whose q picks out column j of the cache (a one-key window)
    deq = orc.q8_0_dequant_f16(kc[row:row + 1], n_out)[0]
    assert np.abs(deq.astype(np.float32) - got).max() <= np.abs(got).max() * (0.5 / 127.0 + 2.0 ** -11) * 1.01
    mask = np.full((1, n_kv), -np.inf, dtype=np.float32)
    mask[0, row] = 0.0
    q = np.zeros((1, 32, n_out), dtype=np.float32)
    o = A.ggml_m4_kqkv(A.Q8_0(kc_q, n_out), torch.from_numpy(q).to(dev), torch.from_numpy(mask).to(dev), 1.0)
    torch.cuda.synchronize()
    # with one key unmasked its softmax weight is 1: out = its first d_lat values
    np.testing.assert_allclose(o.cpu().numpy()[0, 0], deq[:d_lat].astype(np.float32), rtol=1e-6, atol=0)


def test_kvwrite_q8_row_outside_cache_is_not_written(dev):
    n_embd, d_lat, n_rope, n_kv = 4096, 256, 64, 16
    n_out = d_lat + n_rope
    w = orc.q8_0_random(8600, n_out, n_embd, scale=0.002)
    cur = np.random.default_rng(8601).standard_normal(n_embd).astype(np.float32)
    kc0 = orc.q8_0_quantize(np.random.default_rng(8602).standard_normal((n_kv, n_out)).astype(np.float32))
    kc_q = torch.from_numpy(kc0.copy()).to(dev)
    args = (torch.from_numpy(cur).to(dev), q8_dev(w, (n_out,), n_embd, dev),
            torch.ones(d_lat, dtype=torch.float32, device=dev), A.Q8_0(kc_q, n_out))
    for bad in (n_kv, n_kv + 5, -1):
        out = A.ggml_m4_phase_kvwrite(*args, torch.tensor([bad], dtype=torch.int64, device=dev),
                                      torch.tensor([3], dtype=torch.int32, device=dev), A.rope_params(n_dims=n_rope, **RP_PLAIN))
        torch.cuda.synchronize()
        assert np.isfinite(out.cpu().numpy()).all()
    assert np.array_equal(kc_q.cpu().numpy(), kc0)

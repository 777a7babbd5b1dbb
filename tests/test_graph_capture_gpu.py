"""The plain-launch contract under graph capture (the engine captures its layer graph after warm-up:
vendor/llama.cpp/ggml/src/ggml-cuda/ggml-cuda.cu:4646-4700).  One attention step of a layer in the
reference geometry -- PHASE KV-write (the new cache row) -> WKB (Q8_0 W_kb) -> the concat of the
rope half into Qcur -> KQKV with its caller-owned workspace (partial + merge) -> PHASE wv_b -- is
captured into one graph with capture_error_mode="global" (any allocation, synchronisation or
host read inside a launcher fails the capture), then replayed three times with new inputs copied
into the captured buffers (q, the KV-write input, the rope position and cache row, the cache
contents, the mask).  After every replay each stage's output is checked against the CPU oracle
chain on the same inputs, and against the same sequence run eagerly.

Bars: KV-write's latent rows within 4 ulp and its rope rows within the angle bound of
tests/test_q8_gpu.py; the cache row = f16(Kcur); WKB bit-identical (integer dots); KQKV within the
f16-cache bar (1e-2 absolute, 3e-3 relative to max); wv_b bit-identical to the oracle's wv_b of
the GPU's own KQKV output; every replay bit-identical to the eager run.
"""
import numpy as np
import pytest
import torch

import aubier_amd as A
from oracle import oracle as orc

from conftest import errs, say

pytestmark = pytest.mark.gpu

H, D_N, D_R, D_LAT = 32, 64, 64, 256
D_K = D_LAT + D_R
N_EMBD, D_OUT = 4096, 128
W = 8192                                  # cache window (split-K: several splits, a workspace)
KQ_SCALE = 1.0 / np.sqrt(D_N + D_R)
RP = dict(freq_base=1e6, freq_scale=0.25, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
          eps=1e-6, n_ctx_orig=8192)


def q8_dev(blocks_np, lead_shape, ne0, dev):
    b = torch.from_numpy(np.ascontiguousarray(blocks_np)).reshape(*lead_shape, ne0 // 32 * 34).to(dev)
    return A.Q8_0(b, ne0)


def step_inputs(seed):
    """Per-step inputs: q (nope + rope), the KV-write input, the cache before the step and the
    position of the new token (its row; keys [0, pos] are live)."""
    r = np.random.default_rng(seed)
    pos = int(r.integers(3000, W - 1))
    return dict(q=(r.standard_normal((1, H, D_N + D_R)) * 0.05).astype(np.float32),
                cur=r.standard_normal(N_EMBD).astype(np.float32),
                kc=(r.standard_normal((W, D_K)) * 0.05).astype(np.float16),
                pos=pos)


def oracle_chain(inp, w_kva, nw, w_kb, w_vb):
    kc_bits = inp["kc"].view(np.uint16).copy()
    kcur = orc.kvwrite(inp["cur"], w_kva, D_LAT, D_R, nw, kc_bits, inp["pos"], inp["pos"], RP)
    q_abs = orc.wkb_q8(w_kb, D_N, D_LAT, H, np.ascontiguousarray(inp["q"][:, :, :D_N]))
    qcur = np.concatenate([q_abs, inp["q"][:, :, D_N:]], axis=2)
    mask = np.full((1, W), -np.inf, dtype=np.float32)
    mask[0, :inp["pos"] + 1] = 0.0
    out = orc.kqkv(kc_bits.view(np.float16), qcur, mask, KQ_SCALE, d_v=D_LAT)          # [H, 1, D_LAT]
    return dict(kcur=kcur, kc_row=kc_bits[inp["pos"]], qcur=qcur, kqv=out, mask=mask)


def test_layer_step_capture_and_replay(dev):
    w_kva = orc.q8_0_random(9500, D_K, N_EMBD, scale=0.002)
    w_kb = orc.q8_0_random(9501, H * D_LAT, D_N)
    w_vb = orc.q8_0_random(9502, H * D_OUT, D_LAT)
    nw = (1.0 + 0.25 * np.random.default_rng(9503).standard_normal(D_LAT)).astype(np.float32)

    # device buffers, allocated once before capture (the graph reads and writes them in place)
    d_wkva, d_wkb, d_wvb = q8_dev(w_kva, (D_K,), N_EMBD, dev), q8_dev(w_kb, (H, D_LAT), D_N, dev), \
        q8_dev(w_vb, (H, D_OUT), D_LAT, dev)
    d_nw = torch.from_numpy(nw).to(dev)
    d_q = torch.zeros((1, H, D_N + D_R), dtype=torch.float32, device=dev)
    d_cur = torch.zeros(N_EMBD, dtype=torch.float32, device=dev)
    d_kc = torch.zeros((W, D_K), dtype=torch.float16, device=dev)
    d_kidx = torch.zeros(1, dtype=torch.int64, device=dev)
    d_pos = torch.zeros(1, dtype=torch.int32, device=dev)
    d_mask = torch.full((1, W), float("-inf"), dtype=torch.float32, device=dev)
    d_kcur = torch.empty(D_K, dtype=torch.float32, device=dev)
    d_qcur = torch.empty((1, H, D_K), dtype=torch.float32, device=dev)
    d_kqv = torch.empty((H, 1, D_LAT), dtype=torch.float32, device=dev)
    d_out = torch.empty((H, 1, D_OUT), dtype=torch.float32, device=dev)
    need = A.kqkv_workspace_bytes(d_kc, d_qcur, d_kqv)
    assert need > 0                                           # the split-K path, with partials
    d_ws = torch.empty(need, dtype=torch.uint8, device=dev)
    rope = A.rope_params(n_dims=D_R, **RP)

    def layer_step():
        A.ggml_m4_phase_kvwrite(d_cur, d_wkva, d_nw, d_kc, d_kidx, d_pos, rope, out=d_kcur)
        A.ggml_m4_wkb(d_wkb, d_q[:, :, :D_N], out=d_qcur[:, :, :D_LAT])
        d_qcur[:, :, D_LAT:].copy_(d_q[:, :, D_N:])          # the concat (a copy kernel)
        A.ggml_m4_kqkv(d_kc, d_qcur, d_mask, KQ_SCALE, out=d_kqv, workspace=d_ws)
        A.ggml_m4_phase_wvb(d_wvb, d_kqv, out=d_out)

    def load(inp):
        d_q.copy_(torch.from_numpy(inp["q"]))
        d_cur.copy_(torch.from_numpy(inp["cur"]))
        d_kc.copy_(torch.from_numpy(inp["kc"]))
        d_kidx.fill_(inp["pos"])
        d_pos.fill_(inp["pos"])
        m = np.full((1, W), -np.inf, dtype=np.float32)
        m[0, :inp["pos"] + 1] = 0.0
        d_mask.copy_(torch.from_numpy(m))
        torch.cuda.synchronize()

    def results():
        torch.cuda.synchronize()
        return dict(kcur=d_kcur.cpu().numpy(), kc_row=None, kc=d_kc.cpu().numpy(), qcur=d_qcur.cpu().numpy(),
                    kqv=d_kqv.cpu().numpy(), out=d_out.cpu().numpy())

    # warm-up on a side stream, then capture (the launchers must neither allocate nor synchronise)
    load(step_inputs(1))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer_step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="global"):
        layer_step()
    torch.cuda.synchronize()

    for rep, seed in enumerate((11, 12, 13)):
        inp = step_inputs(seed)
        ref = oracle_chain(inp, w_kva, nw, w_kb, w_vb)
        load(inp)
        layer_step()                                          # eager
        eager = results()
        load(inp)
        g.replay()                                            # the captured graph on the same inputs
        got = results()
        pos = inp["pos"]
        tag = f"replay {rep} (pos {pos})"
        # every output of the replay equals the eager run bit for bit
        for k in ("kcur", "kc", "qcur", "kqv", "out"):
            assert np.array_equal(np.ascontiguousarray(got[k]).view(np.uint8), np.ascontiguousarray(eager[k]).view(np.uint8)), (tag, k)
        # KV-write: latent rows within 4 ulp, rope rows within the angle bound, the row and only it
        lat_ulp = np.abs(got["kcur"][:D_LAT] - ref["kcur"][:D_LAT]) / np.spacing(np.abs(ref["kcur"][:D_LAT]))
        rope_err = np.abs(got["kcur"][D_LAT:] - ref["kcur"][D_LAT:]).max()
        assert lat_ulp.max() <= 4, tag
        assert rope_err <= (1e-6 + 4e-7 * pos * np.abs(ref["kcur"][D_LAT:]).max()) * (1.0 + 0.1 * np.log(4.0)), tag
        assert np.array_equal(got["kc"][pos].view(np.uint16), got["kcur"].astype(np.float16).view(np.uint16)), tag
        others = np.ones(W, bool)
        others[pos] = False
        assert np.array_equal(got["kc"][others].view(np.uint16), inp["kc"][others].view(np.uint16)), tag
        # WKB: bit-identical; the concat copied the rope half
        assert np.array_equal(got["qcur"].view(np.uint32), ref["qcur"].astype(np.float32).view(np.uint32)), tag
        # KQKV against the oracle on the GPU's own cache (the row KV-write produced) and Qcur
        kq_ref = orc.kqkv(got["kc"], got["qcur"], ref["mask"], KQ_SCALE, d_v=D_LAT)
        ea, er, rr = errs(got["kqv"], kq_ref)
        say(f"{tag}: KQKV vs oracle max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}; "
            f"KV-write rope max|err|={rope_err:.2e}")
        assert np.isfinite(got["kqv"]).all() and ea <= 1e-2 and er <= 3e-3, tag
        # and against the whole oracle chain (its own cache row): the same bar
        ea2, er2, _ = errs(got["kqv"], ref["kqv"])
        assert ea2 <= 1e-2 and er2 <= 3e-3, tag
        # wv_b: bit-identical to the oracle's wv_b of the GPU's KQKV output
        wvb_ref = orc.wvb_q8(w_vb, D_LAT, D_OUT, H, np.ascontiguousarray(got["kqv"].transpose(1, 0, 2))).transpose(1, 0, 2)
        assert np.array_equal(got["out"].view(np.uint32), np.ascontiguousarray(wvb_ref).view(np.uint32)), tag


def test_short_window_one_launch_capture_and_replay(dev):
    """A short window's one-launch KQKV (a workgroup per (32-key split, head), the last workgroup of
    a head merging through a per-head ticket) under graph capture: WKB (f32 W_kb) -> KQKV over a
    256-key f16 cache at the 576 / 512 geometry, captured after an eager warm-up on a side stream
    (which resolves the ticket array), then replayed three times with new q, cache and live length,
    each replay run twice in a row (the tickets must be back at zero after every launch) and checked
    bit for bit against the eager run and against the oracle at the f16-cache bar."""
    Hs, DN, DK, DV, WS = 32, 128, 576, 512, 256
    rng = np.random.default_rng(9600)
    w_kb = (rng.standard_normal((Hs, DV, DN)) * 0.05).astype(np.float32)
    scale = 1.0 / np.sqrt(192.0)
    d_wkb = torch.from_numpy(w_kb).to(dev)
    d_q = torch.zeros((1, Hs, DN + 64), dtype=torch.float32, device=dev)
    d_kc = torch.zeros((WS, DK), dtype=torch.float16, device=dev)
    d_mask = torch.full((1, WS), float("-inf"), dtype=torch.float32, device=dev)
    d_qcur = torch.empty((1, Hs, DK), dtype=torch.float32, device=dev)
    d_out = torch.empty((Hs, 1, DV), dtype=torch.float32, device=dev)
    need = A.kqkv_workspace_bytes(d_kc, d_qcur, d_out)
    assert need > 0                                           # the one-launch kernel's records
    d_ws = torch.empty(need, dtype=torch.uint8, device=dev)

    def step():
        A.ggml_m4_wkb(d_wkb, d_q[:, :, :DN], out=d_qcur[:, :, :DV])
        d_qcur[:, :, DV:].copy_(d_q[:, :, DN:])
        A.ggml_m4_kqkv(d_kc, d_qcur, d_mask, scale, out=d_out, workspace=d_ws)

    def load(seed):
        r = np.random.default_rng(seed)
        live = int(r.integers(40, WS + 1))
        q = (r.standard_normal((1, Hs, DN + 64)) * 0.05).astype(np.float32)
        kc = (r.standard_normal((WS, DK)) * 0.05).astype(np.float16)
        m = np.full((1, WS), -np.inf, dtype=np.float32)
        m[0, :live] = 0.0
        d_q.copy_(torch.from_numpy(q))
        d_kc.copy_(torch.from_numpy(kc))
        d_mask.copy_(torch.from_numpy(m))
        torch.cuda.synchronize()
        return kc, m, live

    load(1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="global"):
        step()
    torch.cuda.synchronize()

    for rep, seed in enumerate((21, 22, 23)):
        kc, m, live = load(seed)
        step()
        torch.cuda.synchronize()
        eager = d_out.cpu().numpy()
        qcur = d_qcur.cpu().numpy()
        for k in range(2):
            g.replay()
            torch.cuda.synchronize()
            got = d_out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), (rep, k)
        ref = orc.kqkv(kc, qcur, m, scale, d_v=DV)
        ea, er, rr = errs(got, ref)
        say(f"one-launch replay {rep} (live {live}): vs oracle max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}")
        assert np.isfinite(got).all() and ea <= 1e-2 and er <= 3e-3, rep

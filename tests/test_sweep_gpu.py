"""Seeded sweeps of GGML_OP_M4_KQKV and GGML_OP_M4_WKB shapes through the C ABI against the CPU oracle.

Every case draws, from a fixed seed: the cache type (f16 / f32) and geometry (the two MFMA
instantiations, BASELINE's 576/512 and the reference's 320/256, plus one outside them that takes
the VALU kernel), n_kv (from 1 key to a few thousand, ragged against the 16-key slices and 64-key
tiles), the token count (decode, batch-of-N rows, prefill), the head count (also partial 32-head
groups), padded row strides of the cache, q and mask (ggml views), the mask pattern (none,
scattered holes, causal, per-row regions with empty rows of a split), the q scale (flat or sharp
softmax) and the split count (the library's own, or an explicit one through the partial + merge
ops).  Tolerances as test_kqkv_gpu.py: f16 cache 1e-2 absolute / 3e-3 relative to max|oracle|
(2e-2 with a sharp softmax), f32 cache 1e-3 / 1e-5.
"""
import os

import numpy as np
import pytest
import torch

import aubier_amd as A
from aubier_amd import inputs as I
from oracle import oracle as orc

from conftest import errs, say

pytestmark = pytest.mark.gpu

GEOMS = [(576, 512), (320, 256), (192, 128)]
N_CASES = int(os.environ.get("MLA_SWEEP_CASES", "40"))   # more cases on request


def draw(i):
    g = np.random.default_rng(9100 + i)
    f16 = bool(g.random() < 0.8)
    dk, dv = GEOMS[g.choice(3, p=[0.6, 0.25, 0.15])]
    n_kv = int(g.choice([1, 15, 17, 63, 65, 200, 1000, 2049, 4095, 6001]))
    nt = int(g.choice([1, 1, 2, 3, 7, 16, 17, 20]))
    H = int(g.choice([32, 32, 1, 7, 33, 48, 64]))
    mask_kind = str(g.choice(["none", "holes", "causal", "regions"]))
    q_scale = float(g.choice([0.05, 0.05, 1.0, 30.0]))
    pad_k = int(g.choice([0, 8, 64]))            # extra elements per cache row (a strided view)
    pad_q = int(g.choice([0, 4]))                # extra floats per head row of q
    n_split = None if g.random() < 0.5 else int(g.integers(1, 300))
    return dict(f16=f16, dk=dk, dv=dv, n_kv=n_kv, nt=nt, H=H, mask_kind=mask_kind, q_scale=q_scale,
                pad_k=pad_k, pad_q=pad_q, n_split=n_split, seed=9200 + i)


def make_mask(c, g):
    nt, n_kv = c["nt"], c["n_kv"]
    kind = c["mask_kind"]
    if kind == "none":
        return None
    m = np.zeros((nt, n_kv), dtype=np.float32)
    if kind == "holes":
        m[g.random((nt, n_kv)) < 0.2] = -np.inf
        m[:, 0] = 0.0                              # every row keeps a live key
    elif kind == "causal":
        for t in range(nt):
            m[t, n_kv - nt + t + 1:] = -np.inf
        m[:, 0] = 0.0
    else:                                          # per-row regions (batch-of-N sequences)
        for t in range(nt):
            a = int(g.integers(0, n_kv))
            b = int(g.integers(a + 1, n_kv + 1))
            m[t, :a] = -np.inf
            m[t, b:] = -np.inf
    return m


@pytest.mark.parametrize("i", range(N_CASES))
def test_kqkv_sweep(dev, i):
    c = draw(i)
    g = np.random.default_rng(c["seed"])
    dk, dv, n_kv, nt, H = c["dk"], c["dv"], c["n_kv"], c["nt"], c["H"]
    kc = (g.standard_normal((n_kv, dk)) * 0.05).astype(np.float16 if c["f16"] else np.float32)
    q = (g.standard_normal((nt, H, dk)) * c["q_scale"]).astype(np.float32)
    mask = make_mask(c, g)
    scale = float(np.float32(1.0 / np.sqrt(192.0)))
    ref = orc.kqkv(kc, q, mask, scale, d_v=dv)

    # device tensors as padded ggml views: cache rows, q head rows and mask rows with a stride
    kc_t = torch.zeros((n_kv, dk + c["pad_k"]), dtype=torch.float16 if c["f16"] else torch.float32)
    kc_t[:, :dk] = torch.from_numpy(kc)
    kc_d = kc_t.to(dev)[:, :dk]
    q_t = torch.zeros((nt, H, dk + c["pad_q"]), dtype=torch.float32)
    q_t[:, :, :dk] = torch.from_numpy(q)
    q_d = q_t.to(dev)[:, :, :dk]
    m_d = None
    if mask is not None:
        m_t = torch.zeros((nt, n_kv + 4), dtype=torch.float32)
        m_t[:, :n_kv] = torch.from_numpy(mask)
        m_d = m_t.to(dev)[:, :n_kv]
    say(f"case {i}: {c}")
    if c["n_split"] is None:
        out = A.ggml_m4_kqkv(kc_d, q_d, m_d, scale, out=torch.empty((H, nt, dv), dtype=torch.float32, device=dev))
    else:
        part = A.ggml_m4_kqkv_partial(kc_d, q_d, m_d, scale, c["n_split"], d_v=dv)
        out = A.ggml_m4_phase_merge(part, n_head=H, d_v=dv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ea, er, rr = errs(got, ref)
    say(f"case {i}: max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}")
    assert np.isfinite(got).all()
    if c["f16"]:
        # the 1,000-case run on the MI355X: f16-cache max_rel 8.4e-4 over flat and sharp draws
        ta, tr = 1e-2, (2e-3 if c["q_scale"] > 1.0 else 3e-3)
    else:
        ta, tr = 1e-3, (1e-4 if c["q_scale"] > 1.0 else 1e-5)
    assert ea <= ta, (i, ea)
    assert er <= tr, (i, er)


def draw_wkb(i):
    g = np.random.default_rng(9500 + i)
    q8 = bool(g.random() < 0.4)
    d_n = int(g.choice([64, 128]))
    d_v = int(g.choice([16, 48, 256, 512, 528]))
    H = int(g.choice([1, 7, 32, 32, 48]))
    nt = int(g.choice([1, 2, 15, 16, 17, 128, 129]))
    pad_q = int(g.choice([0, 4, 64]))           # floats past d_n per head row (the rope part)
    pad_o = int(g.choice([0, 4, 8]))            # floats past D_v per output head row
    return dict(q8=q8, d_n=d_n, d_v=d_v, H=H, nt=nt, pad_q=pad_q, pad_o=pad_o, seed=9600 + i)


@pytest.mark.parametrize("i", range(max(1, N_CASES // 2)))
def test_wkb_sweep(dev, i):
    """GGML_OP_M4_WKB over seeded shapes: f32 W_kb (the GEMV that holds its rows while up to 15
    tokens stream, and the 16-token-and-up MFMA GEMM with partial tiles) at the f32 bar, Q8_0 W_kb bit-exact;
    head counts off 32, q a strided view, the output a strided view whose padding must stay
    untouched."""
    c = draw_wkb(i)
    g = np.random.default_rng(c["seed"])
    d_n, d_v, H, nt = c["d_n"], c["d_v"], c["H"], c["nt"]
    q = (g.standard_normal((nt, H, d_n + c["pad_q"])) * 0.05).astype(np.float32)
    qn = np.ascontiguousarray(q[:, :, :d_n])
    q_d = torch.from_numpy(q).to(dev)[:, :, :d_n]
    if c["q8"]:
        w = orc.q8_0_random(c["seed"] + 1, H * d_v, d_n)
        ref = orc.wkb_q8(w, d_n, d_v, H, qn)
        w_d = A.Q8_0(torch.from_numpy(np.ascontiguousarray(w)).reshape(H, d_v, d_n // 32 * 34).to(dev), d_n)
    else:
        w = (g.standard_normal((H, d_v, d_n)) * 0.05).astype(np.float32)
        ref = orc.wkb(w, qn)
        w_d = torch.from_numpy(w).to(dev)
    sentinel = 12345.0
    o_full = torch.full((nt, H, d_v + c["pad_o"]), sentinel, dtype=torch.float32, device=dev)
    say(f"case {i}: {c}")
    A.ggml_m4_wkb(w_d, q_d, out=o_full[:, :, :d_v])
    torch.cuda.synchronize()
    got_full = o_full.cpu().numpy()
    got = got_full[:, :, :d_v]
    assert (got_full[:, :, d_v:] == sentinel).all(), "write past D_v"
    if c["q8"]:
        say(f"case {i}: max|diff|={np.abs(got - ref).max():.3e}")
        assert np.array_equal(np.ascontiguousarray(got).view(np.uint32), ref.view(np.uint32))
    else:
        ea, er, rr = errs(got, ref)
        say(f"case {i}: max_abs={ea:.3e} max_rel={er:.3e}")
        assert ea <= 1e-3 and er <= 1e-5, (i, ea, er)

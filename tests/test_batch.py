"""Batch-of-N decode: N rows in one KQKV, each over its own region of one cache window (the
engine's per-sequence regions: a row's mask is 0 on [base, base + len) and -inf elsewhere,
engine/m1_layer.h:212-223, engine/m1_session.h:188-201).  N < 4 runs the decode kernels (one
token per workgroup), N >= 4 the 4-token prefill kernel.

CPU: the oracle's row s over the full masked window equals the oracle over the row's own cells
with no mask (a size-independent restatement of what the mask means), and the f64 brute force.
GPU: parity with the oracle and f64 at the f16-cache bars of test_kqkv_gpu.py, default and forced
split counts (a split that holds no live key of its rows contributes nothing)."""
import numpy as np
import pytest
import torch

import aubier_amd as A
from aubier_amd import inputs as I
from oracle import oracle as orc

from conftest import errs, say
from gpu_util import run_step, upload


def region_q(inp):
    """Qcur as WKB would produce it, on the CPU (the oracle's WKB), [nt, H, 576]."""
    q = np.zeros((inp.nt, I.N_HEAD, I.D_K), dtype=np.float32)
    q[:, :, :I.D_V] = orc.wkb(inp.w_kb, inp.q_nope)
    q[:, :, I.D_V:] = inp.q_pe
    return q


def test_batch_mask_means_region():
    region, lens = 200, [1, 137, 200]
    inp = I.make_batch(3, region, lens=lens)
    q = region_q(inp)
    full = orc.kqkv(inp.kcache, q, inp.mask, inp.kq_scale)                 # [H, nt, 512]
    for s, l in enumerate(lens):
        kc = np.ascontiguousarray(inp.kcache[s * region:s * region + l])
        own = orc.kqkv(kc, np.ascontiguousarray(q[s:s + 1]), None, inp.kq_scale)
        ea, er, _ = errs(full[:, s:s + 1], own)
        say(f"row {s} (len {l}): full window vs own cells max_abs={ea:.2e}")
        assert np.array_equal(full[:, s:s + 1], own)
        ref64 = orc.attn_f64(kc, np.ascontiguousarray(q[s:s + 1]), None, inp.kq_scale)
        assert errs(own, ref64)[1] <= 3e-3
    if lens[0] == 1:      # one live key: the output is that key's V row (f16 -> f32)
        v = inp.kcache[0, :I.D_V].astype(np.float32)
        assert np.allclose(full[:, 0], v[None, :], rtol=0, atol=2e-3 * np.abs(v).max())


@pytest.mark.gpu
@pytest.mark.parametrize("n_seq,region", [(2, 4096), (3, 3000), (4, 2048), (8, 2048)])
def test_batch_decode_matches_oracle(dev, n_seq, region):
    inp = I.make_batch(n_seq, region)
    say(f"batch {inp.notes}")
    g = upload(inp, dev)
    qcur, out = run_step(g, inp.kq_scale)
    ref = orc.kqkv(inp.kcache, qcur, inp.mask, inp.kq_scale)
    ea, er, rr = errs(out, ref)
    say(f"batch N={n_seq}: vs oracle max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}")
    assert np.isfinite(out).all()
    assert ea <= 1e-2 and er <= 3e-3
    ref64 = orc.attn_f64(inp.kcache, qcur, inp.mask, inp.kq_scale)
    assert errs(out, ref64)[1] <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("n_seq", [3, 8])
@pytest.mark.parametrize("n_split", [1, 7, 64, 256])
def test_batch_split_counts(dev, n_seq, n_split):
    inp = I.make_batch(n_seq, 1536, lens=[1] + [1536] * (n_seq - 2) + [700])
    g = upload(inp, dev)
    qcur, out = run_step(g, inp.kq_scale, n_split=n_split)
    ref = orc.kqkv(inp.kcache, qcur, inp.mask, inp.kq_scale)
    ea, er, _ = errs(out, ref)
    say(f"batch N={n_seq} S={n_split}: max_abs={ea:.3e} max_rel={er:.3e}")
    assert np.isfinite(out).all()
    assert ea <= 1e-2 and er <= 3e-3

"""mla_m4_kqkv_noalloc (include/mla_m4.h): the KQKV entry point whose split-K partials live in the
library's static device scratch instead of a caller workspace.  It has no counterpart in the
reference's interface; it must give exactly what mla_m4_kqkv gives on the same operands (same
kernels, same split counts: bit for bit), on consecutive calls that reuse the one scratch array
with a smaller input each time, and reject shapes whose partials exceed the scratch.

Bars: bit-exact against mla_m4_kqkv; against the CPU oracle (the unfused ggml graph) the
north-star bar, max abs <= 1e-2 with an f16 cache and <= 1e-3 with an f32 one, plus the
relative-to-max bars of the other decode parity tests (3e-3 f16, 1e-5 f32).
"""
import numpy as np
import pytest
import torch

import aubier_amd as A
from aubier_amd import inputs as I
from oracle import oracle as orc

from conftest import errs, say
from gpu_util import upload

pytestmark = pytest.mark.gpu

TOL = {False: (1e-3, 1e-5), True: (1e-2, 3e-3)}   # kc_f16 -> (abs, rel-to-max) vs the oracle

# consecutive calls on one scratch array, each smaller than the one before:
# (config, n_kv, nt) -> 25.4 MB of partials (3 tokens, 256 splits), 8.45 MB, 0.54 MB (64 splits),
# the f32-cache VALU kernel (8 splits of 16-key granules)
CALLS = [(3, 32768, 3), (3, 32768, 1), (2, 4096, 1), (1, 256, 1)]


def _inputs(dev, cfg, n_kv, nt):
    inp = I.make_config(cfg, n_kv=n_kv, nt=nt)
    g = upload(inp, dev)
    A.ggml_m4_wkb(g["w_kb"], g["q"][:, :, :I.D_NOPE], out=g["qcur"][:, :, :I.D_V])
    torch.cuda.synchronize()
    return inp, g


def test_noalloc_matches_kqkv_on_consecutive_calls(dev):
    prev = None
    for cfg, n_kv, nt in CALLS:
        inp, g = _inputs(dev, cfg, n_kv, nt)
        out_na = torch.empty((I.N_HEAD, nt, I.D_V), dtype=torch.float32, device=dev)
        need = A.kqkv_workspace_bytes(g["kcache"], g["qcur"], out_na)
        say(f"noalloc call: cfg{cfg} n_kv={n_kv} nt={nt} f16={inp.kc_f16} partial bytes={need}")
        assert 0 < need <= A.ops.NOALLOC_SCRATCH_BYTES
        if prev is not None:
            assert need < prev
        prev = need
        A.ggml_m4_kqkv_noalloc(g["kcache"], g["qcur"], g["mask"], inp.kq_scale, out=out_na)
        torch.cuda.synchronize()
        out_ws = A.ggml_m4_kqkv(g["kcache"], g["qcur"], g["mask"], inp.kq_scale)
        torch.cuda.synchronize()
        got, ws = out_na.cpu().numpy(), out_ws.cpu().numpy()
        assert np.isfinite(got).all()
        nbad = int(np.count_nonzero(got.view(np.uint32) != ws.view(np.uint32)))
        say(f"  vs mla_m4_kqkv: {nbad} differing words of {got.size}")
        assert nbad == 0
        ref = orc.kqkv(inp.kcache, g["qcur"].cpu().numpy(), inp.mask, inp.kq_scale)
        ea, er, rr = errs(got, ref)
        say(f"  vs oracle: max_abs={ea:.3e} max_rel={er:.3e} rms_rel={rr:.3e}")
        ta, tr = TOL[inp.kc_f16]
        assert ea <= ta and er <= tr, (cfg, n_kv, nt, ea, er)


def test_noalloc_rejects_partials_beyond_scratch(dev):
    # 4 tokens at 256 splits need 33.8 MB > 32 MiB; nothing is launched
    inp, g = _inputs(dev, 3, 32768, 4)
    out = torch.full((I.N_HEAD, 4, I.D_V), 7.0, dtype=torch.float32, device=dev)
    need = A.kqkv_workspace_bytes(g["kcache"], g["qcur"], out)
    say(f"noalloc oversize: partial bytes={need} scratch={A.ops.NOALLOC_SCRATCH_BYTES}")
    assert need > A.ops.NOALLOC_SCRATCH_BYTES
    with pytest.raises(A.MlaM4Error, match="static scratch"):
        A.ggml_m4_kqkv_noalloc(g["kcache"], g["qcur"], g["mask"], inp.kq_scale, out=out)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    # the entry point still works after a rejection
    inp, g = _inputs(dev, 2, 4096, 1)
    got = A.ggml_m4_kqkv_noalloc(g["kcache"], g["qcur"], g["mask"], inp.kq_scale)
    ws = A.ggml_m4_kqkv(g["kcache"], g["qcur"], g["mask"], inp.kq_scale)
    torch.cuda.synchronize()
    assert torch.equal(got, ws)


def test_noalloc_under_graph_capture(dev):
    """The callers the entry point is for: code under hipGraph capture.  One eager call first (it
    resolves the scratch array's address on this device), then the call captured with
    capture_error_mode="global" (an allocation, synchronisation or host read inside it would fail
    the capture).  Three replays, each after new q values are copied into the captured buffer and
    followed by eager work and a synchronisation, must each be bit-identical to mla_m4_kqkv (with
    its own workspace) on the same operands."""
    inp, g = _inputs(dev, 3, 32768, 1)
    out = torch.empty((I.N_HEAD, 1, I.D_V), dtype=torch.float32, device=dev)
    A.ggml_m4_kqkv_noalloc(g["kcache"], g["qcur"], g["mask"], inp.kq_scale, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="global"):
        A.ggml_m4_kqkv_noalloc(g["kcache"], g["qcur"], g["mask"], inp.kq_scale, out=out)
    for rep in range(3):
        qn = I.randn(9300 + rep, 32 * I.D_K, 0.05).reshape(1, 32, I.D_K)
        g["qcur"].copy_(torch.from_numpy(qn).to(dev))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ws = A.ggml_m4_kqkv(g["kcache"], g["qcur"], g["mask"], inp.kq_scale)
        torch.cuda.synchronize()
        got, ref = out.cpu().numpy(), ws.cpu().numpy()
        nbad = int(np.count_nonzero(got.view(np.uint32) != ref.view(np.uint32)))
        say(f"noalloc graph replay {rep}: {nbad} differing words of {got.size}")
        assert np.isfinite(got).all() and nbad == 0

"""The short-window KQKV (one launch, the splits merged inside it through per-head tickets) on two
streams at once.  The tickets live in a static device array, one slot per (device, stream), so
launches that overlap on one GPU never count each other's workgroups; with a shared slot a head's
merge would run early or not at all.  Each stream works on its own inputs (different windows and
values) with its own workspace, launching back to back while the other stream does the same, and
every output must equal that stream's own earlier result bit for bit (the merge reads the records
in split order, whichever workgroup draws the last ticket), which itself matches the oracle."""
import numpy as np
import pytest
import torch

import aubier_amd as A
from aubier_amd import inputs as I
from oracle import oracle as orc

from conftest import errs, say

pytestmark = pytest.mark.gpu

H, DK, DV = 32, 576, 512
SCALE = float(np.float32(1.0 / np.sqrt(192.0)))
BARS = {False: (1e-3, 1e-5), True: (1e-2, 3e-3)}     # f16 cache -> (abs, rel to max) vs the oracle


@pytest.mark.parametrize("f16,n_kv", [(False, 256), (False, 512), (True, 256)])
def test_short_window_on_two_streams(dev, f16, n_kv):
    iters = 64
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    runs = []
    for k, s in enumerate(streams):
        kc = I.randn(9100 + 2 * k + int(f16), n_kv * DK).reshape(n_kv, DK)
        kc = kc.astype(np.float16) if f16 else kc.astype(np.float32)
        q = I.randn(9110 + k, H * DK).reshape(1, H, DK).astype(np.float32)
        mask = np.zeros((1, n_kv), dtype=np.float32)
        mask[0, n_kv - 40 - 25 * k:] = -np.inf                  # a different live window per stream
        ref = orc.kqkv(kc, q, mask, SCALE, d_v=DV)
        d_kc, d_q, d_m = (torch.from_numpy(x).to(dev) for x in (kc, q, mask))
        first = torch.empty((H, 1, DV), dtype=torch.float32, device=dev)
        ws = torch.empty(max(A.kqkv_workspace_bytes(d_kc, d_q, first), 16), dtype=torch.uint8, device=dev)
        outs = torch.empty((iters, H, 1, DV), dtype=torch.float32, device=dev)
        runs.append(dict(s=s, kc=d_kc, q=d_q, m=d_m, ws=ws, first=first, outs=outs, ref=ref))
    torch.cuda.synchronize()
    # each stream's own result first, alone
    for r in runs:
        with torch.cuda.stream(r["s"]):
            A.ggml_m4_kqkv(r["kc"], r["q"], r["m"], SCALE, out=r["first"], workspace=r["ws"])
        torch.cuda.synchronize()
        first = r["first"].cpu().numpy()
        ea, er, _ = errs(first, r["ref"])
        say(f"f16={f16} n_kv={n_kv}: alone vs oracle max_abs={ea:.3e} max_rel={er:.3e}")
        ta, tr = BARS[f16]
        assert np.isfinite(first).all() and ea <= ta and er <= tr
    # then both streams launching back to back, with no synchronisation between them
    for it in range(iters):
        for r in runs:
            with torch.cuda.stream(r["s"]):
                A.ggml_m4_kqkv(r["kc"], r["q"], r["m"], SCALE, out=r["outs"][it], workspace=r["ws"])
    torch.cuda.synchronize()
    for k, r in enumerate(runs):
        first = r["first"].cpu().numpy().view(np.uint32)
        outs = r["outs"].cpu().numpy().view(np.uint32)
        bad = [it for it in range(iters) if not np.array_equal(outs[it], first)]
        say(f"stream {k}: {iters - len(bad)} of {iters} concurrent launches equal to its own result")
        assert not bad, (k, bad[:8])

"""Helpers for the GPU tests: upload a config's inputs and run the decode/prefill step through the
C ABI (WKB into the Qcur buffer, then KQKV)."""
import numpy as np
import torch

import aubier_amd as A
from aubier_amd import inputs as I


def upload(inp, dev):
    g = {}
    g["kcache"] = torch.from_numpy(np.ascontiguousarray(inp.kcache)).to(dev)
    g["w_kb"] = torch.from_numpy(inp.w_kb).to(dev)
    q = np.zeros((inp.nt, I.N_HEAD, I.D_NOPE + I.D_ROPE), dtype=np.float32)
    q[:, :, :I.D_NOPE] = inp.q_nope
    q[:, :, I.D_NOPE:] = inp.q_pe
    g["q"] = torch.from_numpy(q).to(dev)                       # the q_b output, head stride 192
    qcur = torch.zeros((inp.nt, I.N_HEAD, I.D_K), dtype=torch.float32, device=dev)
    qcur[:, :, I.D_V:] = g["q"][:, :, I.D_NOPE:]                # rope part (given)
    g["qcur"] = qcur
    g["mask"] = torch.from_numpy(inp.mask).to(dev)
    return g


def run_step(g, kq_scale, n_split=None):
    """WKB writes the absorbed nope part straight into Qcur[..., :512]; KQKV reads Qcur."""
    A.ggml_m4_wkb(g["w_kb"], g["q"][:, :, :I.D_NOPE], out=g["qcur"][:, :, :I.D_V])
    if n_split is None:
        out = A.ggml_m4_kqkv(g["kcache"], g["qcur"], g["mask"], kq_scale)
    else:
        part = A.ggml_m4_kqkv_partial(g["kcache"], g["qcur"], g["mask"], kq_scale, n_split)
        out = A.ggml_m4_phase_merge(part, n_head=g["q"].shape[1])
    torch.cuda.synchronize()
    return g["qcur"].cpu().numpy(), out.cpu().numpy()

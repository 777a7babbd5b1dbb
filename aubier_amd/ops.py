"""Python mirror of aubier's three custom ggml ops, calling the gfx950 kernels through the C ABI
of include/mla_m4.h (aubier_amd/libmla_m4.so).

Names and argument meaning follow the reference's op builders (vendor/llama.cpp/ggml/include/
ggml.h:1524-1586, ggml.c:3405-3539): ``ggml_m4_wkb(w_kb, q_nope)``, ``ggml_m4_kqkv(kcache, q,
mask, kq_scale)`` and the PHASE op's split-K merge ``ggml_m4_phase_merge(part)``.  A contract
violation raises :class:`MlaM4Error` (the ggml glue aborts instead, keeping the FATAL semantics).
There is no CPU path: without the built library every call raises.

Tensors are torch CUDA tensors in row-major order, i.e. with the ggml ``ne[]`` axes reversed:

=============  =========================  ==============================
op / operand   ggml ne (fastest first)    torch shape
=============  =========================  ==============================
W_kb           [d_n, D_v, H]              [H, D_v, d_n]
q_nope         [d_n, H, nt]               [nt, H, d_n] (a strided view is fine)
WKB dst        [D_v, H, nt]               [nt, H, D_v] (a view into Qcur is fine)
kcache         [D_k, n_kv]                [n_kv, D_k]  (f16 or f32)
q (Qcur)       [D_k, H, nt]               [nt, H, D_k]
mask           [n_kv, >= nt]              [>= nt, n_kv]
KQKV dst       [D_v, nt, H]               [H, nt, D_v]
partials       [64 + 16 D_v, S, nt, G]    [G, nt, S, 64 + 16 D_v]   (G = ceil(H / 32) head groups)
=============  =========================  ==============================
"""
from __future__ import annotations

import ctypes
import math
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmla_m4.so"

TYPE_F32, TYPE_F16 = 0, 1
PART_HEADS = 32
MAX_SPLITS = 1024


def part_floats(d_v: int, kc_f16: bool = True) -> int:
    """4-byte words per split-K partial block (include/mla_m4.h MLA_M4_PART_FLOATS[_F32])."""
    return 64 + (16 if kc_f16 else 32) * d_v


PHASE_KVWRITE, PHASE_WVB, PHASE_MERGE = 0, 1, 2

STATUS = {
    0: "ok", -1: "null tensor or data pointer", -2: "unsupported element type",
    -3: "shape violates the op contract", -4: "strides/alignment violate the op contract",
    -5: "workspace missing or too small", -6: "scalar argument out of range",
    -7: "HIP launch failed", -8: "shape not implemented by these kernels",
    -9: "needs more than the static scratch holds (or its address is unavailable)",
}


class MlaM4Error(RuntimeError):
    def __init__(self, op: str, status: int):
        self.status = status
        super().__init__(f"{op}: {STATUS.get(status, 'unknown status')} ({status})")


class MlaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


class RopeParams(ctypes.Structure):
    """mla_m4_rope_params: op_params[1..9] of ggml_m4_phase_kvwrite."""
    _fields_ = [(n, ctypes.c_float) for n in ("freq_base", "freq_scale", "ext_factor", "attn_factor", "beta_fast",
                                               "beta_slow", "eps")] + [("n_dims", ctypes.c_int32), ("n_ctx_orig", ctypes.c_int32)]


_lib: Optional[ctypes.CDLL] = None

_EXPORTS = {
    "mla_m4_version": (ctypes.c_char_p, []),
    "mla_m4_status_str": (ctypes.c_char_p, [ctypes.c_int]),
    "mla_m4_wkb": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3 + [ctypes.c_void_p]),
    "mla_m4_kqkv": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3 + [ctypes.c_float, ctypes.POINTER(MlaTensor),
                                                                      ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mla_m4_kqkv_noalloc": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3 + [ctypes.c_float, ctypes.POINTER(MlaTensor),
                                                                              ctypes.c_void_p]),
    "mla_m4_kqkv_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(MlaTensor)] * 3),
    "mla_m4_kqkv_default_splits": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]),
    "mla_m4_kqkv_partial": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3 + [ctypes.c_float, ctypes.c_int, ctypes.c_int64,
                                                                              ctypes.POINTER(MlaTensor), ctypes.c_void_p]),
    "mla_m4_phase_merge": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 2 + [ctypes.c_void_p]),
    "mla_m4_supports_wkb": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3),
    "mla_m4_supports_kqkv": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 4),
    "mla_m4_supports_phase": (ctypes.c_int, [ctypes.c_int32, ctypes.POINTER(MlaTensor), ctypes.POINTER(MlaTensor)]),
    "mla_m4_resolve_flag": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "mla_m4_phase_wvb": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3 + [ctypes.c_void_p]),
    "mla_m4_supports_phase_wvb": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 3),
    "mla_m4_phase_kvwrite": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 6 + [ctypes.POINTER(RopeParams),
                                                                              ctypes.POINTER(MlaTensor), ctypes.c_void_p]),
    "mla_m4_supports_phase_kvwrite": (ctypes.c_int, [ctypes.POINTER(MlaTensor)] * 6 + [ctypes.POINTER(RopeParams),
                                                                                       ctypes.POINTER(MlaTensor)]),
}


def load_library() -> ctypes.CDLL:
    """Load libmla_m4.so (raises if it has not been built: there is no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built (python -m aubier_amd.build); the MLA ops have no CPU path")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_EXPORTS)


# ------------------------------------------------------------------------------------ views
TYPE_Q8_0, TYPE_I32, TYPE_I64 = 8, 26, 27
_DT = {torch.float32: (TYPE_F32, 4), torch.float16: (TYPE_F16, 2), torch.int32: (TYPE_I32, 4),
       torch.int64: (TYPE_I64, 8)}


class Q8_0:
    """A Q8_0 tensor (ggml block_q8_0: f16 scale + 32 int8 = 34 bytes per 32 elements): `blocks`
    is a uint8 tensor [..., ne0 / 32 * 34] of packed rows; the ggml shape is (ne0, reversed leading
    dims of `blocks`)."""

    def __init__(self, blocks: torch.Tensor, ne0: int):
        assert blocks.dtype == torch.uint8 and blocks.is_contiguous() and ne0 % 32 == 0
        assert blocks.shape[-1] == ne0 // 32 * 34
        self.blocks, self.ne0 = blocks, ne0

    @property
    def device(self):
        return self.blocks.device


def _view_q8(t: Q8_0) -> MlaTensor:
    v = MlaTensor()
    v.data = t.blocks.data_ptr()
    v.type = TYPE_Q8_0
    rows = list(reversed(t.blocks.shape[:-1]))
    shape = [t.ne0] + rows
    nb = [34, t.blocks.shape[-1]]
    for r in rows[:-1] if rows else []:
        nb.append(nb[-1] * r)
    while len(shape) < 4:
        shape.append(1)
    while len(nb) < 4:
        nb.append(nb[-1] * shape[len(nb) - 1])
    for i in range(4):
        v.ne[i] = int(shape[i])
        v.nb[i] = int(nb[i])
    return v


def view(t) -> Optional[MlaTensor]:
    """ggml-style view of a torch tensor: ne/nb are the reversed shape/strides (bytes)."""
    if t is None:
        return None
    if isinstance(t, Q8_0):
        return _view_q8(t)
    if t.dtype not in _DT:
        raise MlaM4Error("view", -2)
    if t.dim() > 4:
        raise MlaM4Error("view", -3)
    ty, es = _DT[t.dtype]
    v = MlaTensor()
    v.data = t.data_ptr()
    v.type = ty
    shape = list(reversed(t.shape))
    strides = [s * es for s in reversed(t.stride())]
    while len(shape) < 4:
        shape.append(1)
        strides.append(strides[-1] * shape[-2] if strides else es)
    for i in range(4):
        v.ne[i] = int(shape[i])
        v.nb[i] = int(strides[i])
    return v


def _ptr(v: Optional[MlaTensor]):
    return ctypes.byref(v) if v is not None else None


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(op: str, rc: int) -> None:
    if rc != 0:
        raise MlaM4Error(op, rc)


# ------------------------------------------------------------------------------------ ops
def ggml_m4_wkb(w_kb, q_nope: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GGML_OP_M4_WKB: out[t, h, c] = sum_d w_kb[h, c, d] * q_nope[t, h, d].

    w_kb f32 [H, D_v, d_n] contiguous, or a Q8_0 with blocks [H, D_v, d_n / 32 * 34] (the
    reference's form: Q8_1 activation numerics); q_nope [nt, H, d_n] (strided view ok);
    out [nt, H, D_v] (a view into the Qcur buffer ok)."""
    lib = load_library()
    if out is None:
        H, D_v = (w_kb.blocks.shape[0], w_kb.blocks.shape[1]) if isinstance(w_kb, Q8_0) else (w_kb.shape[0], w_kb.shape[1])
        out = torch.empty((q_nope.shape[0], H, D_v), dtype=torch.float32, device=q_nope.device)
    vw, vq, vo = view(w_kb), view(q_nope), view(out)
    _check("ggml_m4_wkb", lib.mla_m4_wkb(_ptr(vw), _ptr(vq), _ptr(vo), _stream(q_nope)))
    return out


def kqkv_workspace_bytes(kcache: torch.Tensor, q: torch.Tensor, out: torch.Tensor) -> int:
    lib = load_library()
    return int(lib.mla_m4_kqkv_workspace_bytes(_ptr(view(kcache)), _ptr(view(q)), _ptr(view(out))))


def _kc_width(kcache) -> int:
    """D_k of a cache: a torch tensor [n_kv, D_k] or a Q8_0 one (ne0)."""
    return kcache.ne0 if isinstance(kcache, Q8_0) else kcache.shape[1]


def _dv_of(kcache) -> int:
    """D_v of the op's output for a cache of width D_k: 512 for the 576-wide cache, 256 for the
    reference's 320-wide one, else D_k."""
    dk = _kc_width(kcache)
    return 512 if dk == 576 else (256 if dk == 320 else dk)


def _kc_f16_partials(kcache) -> bool:
    """Whether the partial records hold f16 o (F16 and Q8_0 caches) or f32 (F32 cache)."""
    return isinstance(kcache, Q8_0) or kcache.dtype == torch.float16


def ggml_m4_kqkv(kcache: torch.Tensor, q: torch.Tensor, mask: Optional[torch.Tensor], kq_scale: float,
                 out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GGML_OP_M4_KQKV: out[h, t, :] = softmax_j(kq_scale * q[t, h] . K[j] + mask[t, j]) . V[j, :D_v].

    kcache [n_kv, D_k] f16/f32, or Q8_0 (ne0 = D_k); q [nt, H, D_k] f32; mask [>= nt, n_kv] f32 or None;
    out [H, nt, D_v] f32 (D_v = 512 unless out is given).  workspace: optional uint8 device
    buffer (allocated here when None and the shape needs one)."""
    lib = load_library()
    if out is None:
        out = torch.empty((q.shape[1], q.shape[0], _dv_of(kcache)), dtype=torch.float32, device=q.device)
    vk, vq, vm, vo = view(kcache), view(q), view(mask), view(out)
    need = int(lib.mla_m4_kqkv_workspace_bytes(_ptr(vk), _ptr(vq), _ptr(vo)))
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("ggml_m4_kqkv", lib.mla_m4_kqkv(_ptr(vk), _ptr(vq), _ptr(vm), ctypes.c_float(kq_scale), _ptr(vo),
                                           ws_ptr, ws_bytes, _stream(q)))
    return out


NOALLOC_SCRATCH_BYTES = 32 << 20


def ggml_m4_kqkv_noalloc(kcache: torch.Tensor, q: torch.Tensor, mask: Optional[torch.Tensor], kq_scale: float,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """ggml_m4_kqkv without a workspace: the library's static scratch holds the split-K partials
    (include/mla_m4.h mla_m4_kqkv_noalloc; calls that overlap on one GPU race)."""
    lib = load_library()
    if out is None:
        out = torch.empty((q.shape[1], q.shape[0], _dv_of(kcache)), dtype=torch.float32, device=q.device)
    _check("ggml_m4_kqkv_noalloc", lib.mla_m4_kqkv_noalloc(_ptr(view(kcache)), _ptr(view(q)), _ptr(view(mask)),
                                                           ctypes.c_float(kq_scale), _ptr(view(out)), _stream(q)))
    return out


def ggml_m4_kqkv_partial(kcache: torch.Tensor, q: torch.Tensor, mask: Optional[torch.Tensor], kq_scale: float,
                         n_split: int, part: Optional[torch.Tensor] = None, d_v: int = 512) -> torch.Tensor:
    """Split-K pass 1 with an explicit split count: part [G, nt, n_split, 64 + 16 D_v] (f32 words)."""
    lib = load_library()
    if part is None:
        G = (q.shape[1] + PART_HEADS - 1) // PART_HEADS
        part = torch.empty((G, q.shape[0], n_split, part_floats(d_v, _kc_f16_partials(kcache))),
                           dtype=torch.float32, device=q.device)
    _check("ggml_m4_kqkv_partial", lib.mla_m4_kqkv_partial(_ptr(view(kcache)), _ptr(view(q)), _ptr(view(mask)),
                                                           ctypes.c_float(kq_scale), int(n_split), int(d_v),
                                                           _ptr(view(part)), _stream(q)))
    return part


def ggml_m4_phase_merge(part: torch.Tensor, out: Optional[torch.Tensor] = None, n_head: Optional[int] = None,
                        d_v: int = 512) -> torch.Tensor:
    """GGML_OP_M4_PHASE phase 2: the split-K merge.  part [G, nt, S, 64 + 16 D_v] -> out [H, nt, D_v]."""
    lib = load_library()
    if out is None:
        H = n_head if n_head is not None else part.shape[0] * PART_HEADS
        out = torch.empty((H, part.shape[1], d_v), dtype=torch.float32, device=part.device)
    _check("ggml_m4_phase_merge", lib.mla_m4_phase_merge(_ptr(view(part)), _ptr(view(out)), _stream(part)))
    return out


def decode_partials(part, n_head: int, d_v: int = 512):
    """Split a partial buffer (numpy/torch, [G, nt, S, 64 + 16 D_v] f32 words; per (group, token)
    one record: the (m, l) pairs [32 heads][S], then the o / l blocks [S][32 heads][D_v]) into
    m [H, nt, S], l [H, nt, S] and o_norm [H, nt, S, D_v] (float32 numpy arrays)."""
    import numpy as np
    p = part.detach().cpu().numpy() if isinstance(part, torch.Tensor) else np.asarray(part)
    G, nt, S, W = p.shape
    rec = np.ascontiguousarray(p).reshape(G, nt, S * W)
    ml = rec[..., :2 * PART_HEADS * S].reshape(G, nt, PART_HEADS, S, 2)
    o = np.ascontiguousarray(rec[..., 2 * PART_HEADS * S:])
    if W == part_floats(d_v, True):
        o = o.view(np.float16)
    o = o.reshape(G, nt, S, PART_HEADS, d_v)
    m = np.moveaxis(ml[..., 0], 2, 1).reshape(G * PART_HEADS, nt, S)[:n_head]
    l = np.moveaxis(ml[..., 1], 2, 1).reshape(G * PART_HEADS, nt, S)[:n_head]
    o = np.moveaxis(o, 3, 1).reshape(G * PART_HEADS, nt, S, d_v)[:n_head].astype(np.float32)
    return m, l, o


def default_splits(n_kv: int, n_head: int = 32, kcache_type: int = TYPE_F16) -> int:
    return int(load_library().mla_m4_kqkv_default_splits(n_kv, n_head, kcache_type))


def supports_kqkv(kcache, q, mask, out) -> bool:
    lib = load_library()
    return bool(lib.mla_m4_supports_kqkv(_ptr(view(kcache)), _ptr(view(q)), _ptr(view(mask)), _ptr(view(out))))


def supports_wkb(w_kb, q_nope, out) -> bool:
    lib = load_library()
    return bool(lib.mla_m4_supports_wkb(_ptr(view(w_kb)), _ptr(view(q_nope)), _ptr(view(out))))


def supports_phase(phase: int, src0, dst) -> bool:
    lib = load_library()
    return bool(lib.mla_m4_supports_phase(int(phase), _ptr(view(src0)), _ptr(view(dst))))


def resolve_flag(flag: int, gpu_core: bool) -> bool:
    """The tri-state enable flag (-1 AUTO, 0 off, 1 explicit); explicit without gpu_core raises."""
    rc = int(load_library().mla_m4_resolve_flag(int(flag), int(bool(gpu_core))))
    if rc < 0:
        raise MlaM4Error("resolve_flag", rc)
    return bool(rc)


def kq_scale_default(d_k_nope: int = 128, d_rope: int = 64) -> float:
    return 1.0 / math.sqrt(d_k_nope + d_rope)


# ---------------------------------------------------------------- PHASE 0 / 1 (reference geometry)
def ggml_m4_phase_wvb(w: Q8_0, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GGML_OP_M4_PHASE phase 1 (wv_b): w Q8_0 blocks [H, d_out, d_in / 32 * 34]; x f32 [H, nt, d_in]
    (the KQKV output layout) -> out [H, nt, d_out]."""
    lib = load_library()
    if out is None:
        out = torch.empty((x.shape[0], x.shape[1], w.blocks.shape[1]), dtype=torch.float32, device=x.device)
    _check("ggml_m4_phase_wvb", lib.mla_m4_phase_wvb(_ptr(view(w)), _ptr(view(x)), _ptr(view(out)), _stream(x)))
    return out


def rope_params(**kw) -> RopeParams:
    rp = RopeParams()
    for k, v in kw.items():
        setattr(rp, k, v)
    return rp


def ggml_m4_phase_kvwrite(cur: torch.Tensor, wkv_a: Q8_0, kv_norm: torch.Tensor, kcache: torch.Tensor,
                          kidx: torch.Tensor, pos: torch.Tensor, rope: RopeParams,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GGML_OP_M4_PHASE phase 0 (KV-write): cur f32 [n_embd]; wkv_a Q8_0 blocks [n_out, n_embd/32*34];
    kv_norm f32 [d_lat]; kcache f16 [n_kv, n_out] or Q8_0 (rows of n_out / 32 blocks; row kidx[0]
    written in place, quantised as ggml's f32 -> q8_0 copy); kidx int64 [1]; pos int32 [1] -> Kcur
    f32 [n_out]."""
    lib = load_library()
    if out is None:
        out = torch.empty((wkv_a.blocks.shape[0],), dtype=torch.float32, device=cur.device)
    _check("ggml_m4_phase_kvwrite",
           lib.mla_m4_phase_kvwrite(_ptr(view(cur)), _ptr(view(wkv_a)), _ptr(view(kv_norm)), _ptr(view(kcache)),
                                    _ptr(view(kidx)), _ptr(view(pos)), ctypes.byref(rope), _ptr(view(out)),
                                    _stream(cur)))
    return out


def supports_phase_wvb(w, x, out) -> bool:
    return bool(load_library().mla_m4_supports_phase_wvb(_ptr(view(w)), _ptr(view(x)), _ptr(view(out))))


def supports_phase_kvwrite(cur, wkv_a, kv_norm, kcache, kidx, pos, rope: RopeParams, out) -> bool:
    return bool(load_library().mla_m4_supports_phase_kvwrite(_ptr(view(cur)), _ptr(view(wkv_a)), _ptr(view(kv_norm)),
                                                             _ptr(view(kcache)), _ptr(view(kidx)), _ptr(view(pos)),
                                                             ctypes.byref(rope), _ptr(view(out))))

"""TEST INFRASTRUCTURE ONLY: numpy-facing wrapper of oracle/libmla_oracle.so, the C restatement of
the reference's unfused ggml CPU graph (see mla_oracle.c for what it restates, with file:line).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, as the
checker or as the timed CPU baseline -- never as the product path.

Array conventions are the torch/numpy (row-major, reversed ggml ne) shapes of aubier_amd.ops:
kcache [n_kv, D_k] (float16 or float32), q [nt, H, D_k] f32, mask [nt, n_kv] f32 or None,
KQKV out [H, nt, D_v], W_kb [H, D_v, d_n], q_nope [nt, H, d_n], WKB out [nt, H, D_v],
partials [H, nt, S, 4 + D_v].
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libmla_oracle.so"
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} not built (python -m aubier_amd.build --oracle)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_randn.argtypes = [ctypes.c_uint64, _I64, ctypes.c_float, _P]
        L.orc_f32_to_f16.argtypes = [_P, _P, _I64]
        L.orc_f16_to_f32.argtypes = [_P, _P, _I64]
        L.orc_kqkv.argtypes = [_P, _I32, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, ctypes.c_float,
                               _I64, _P, ctypes.c_int, ctypes.c_int]
        L.orc_kqkv.restype = ctypes.c_int
        L.orc_attn_f64.argtypes = [_P, _I32, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, ctypes.c_float,
                                   _I64, _P, ctypes.c_int]
        L.orc_attn_f64.restype = ctypes.c_int
        L.orc_partials.argtypes = [_P, _I32, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, ctypes.c_float,
                                   _I64, _P, _I64, _P]
        L.orc_partials.restype = ctypes.c_int
        L.orc_merge.argtypes = [_P, _I64, _I64, _I64, _I64, _P, ctypes.c_int]
        L.orc_merge.restype = ctypes.c_int
        L.orc_wkb.argtypes = [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, ctypes.c_int, ctypes.c_int]
        L.orc_wkb.restype = ctypes.c_int
        L.orc_kqkv_bench_pattern.argtypes = [_I64, _P, _I64, _P]
        L.orc_wkb_q8.argtypes = [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, ctypes.c_int]
        L.orc_wkb_q8.restype = ctypes.c_int
        L.orc_wvb_q8.argtypes = [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, ctypes.c_int]
        L.orc_wvb_q8.restype = ctypes.c_int
        L.orc_rope_yarn_corr_dims.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                              ctypes.c_float, _P]
        L.orc_kvwrite.argtypes = [_P, _I64, _P, _I64, _I64, _P, _P, _I64, _I64, _I32] + [ctypes.c_float] * 7 + \
            [_I32, _P, ctypes.c_int]
        L.orc_kvwrite.restype = ctypes.c_int
        L.orc_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def max_threads() -> int:
    return int(lib().orc_max_threads())


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(_P)


def _kc(kcache: np.ndarray):
    if kcache.dtype == np.float16:
        return 1, 2
    if kcache.dtype == np.float32:
        return 0, 4
    raise TypeError(kcache.dtype)


def randn(seed: int, n: int, scale: float = 0.05) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_randn(seed, n, scale, _ptr(out))
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32(_ptr(h), _ptr(out), h.size)
    return out


def kqkv(kcache: np.ndarray, q: np.ndarray, mask: Optional[np.ndarray], kq_scale: float, d_v: int = 512,
         threads: Optional[int] = None, mutant: int = 0) -> np.ndarray:
    """The unfused ggml graph kq -> soft_max_ext -> kqv (engine/m1_layer.cpp:477-495) on the CPU."""
    kcache = np.ascontiguousarray(kcache)
    q = np.ascontiguousarray(q, dtype=np.float32)
    ty, es = _kc(kcache)
    n_kv, d_k = kcache.shape
    nt, H, _ = q.shape
    out = np.empty((H, nt, d_v), dtype=np.float32)
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float32)
    rc = lib().orc_kqkv(_ptr(kcache), ty, d_k, n_kv, d_k * es, _ptr(q), H, nt, d_k * 4, H * d_k * 4,
                        _ptr(mask), n_kv * 4, kq_scale, d_v, _ptr(out), threads or max_threads(), mutant)
    assert rc == 0
    return out


def attn_f64(kcache: np.ndarray, q: np.ndarray, mask: Optional[np.ndarray], kq_scale: float, d_v: int = 512,
             threads: Optional[int] = None) -> np.ndarray:
    """Double-precision brute force (no f16 rounding of q or P)."""
    kcache = np.ascontiguousarray(kcache)
    q = np.ascontiguousarray(q, dtype=np.float32)
    ty, es = _kc(kcache)
    n_kv, d_k = kcache.shape
    nt, H, _ = q.shape
    out = np.empty((H, nt, d_v), dtype=np.float64)
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float32)
    rc = lib().orc_attn_f64(_ptr(kcache), ty, d_k, n_kv, d_k * es, _ptr(q), H, nt, d_k * 4, H * d_k * 4,
                            _ptr(mask), n_kv * 4, kq_scale, d_v, _ptr(out), threads or max_threads())
    assert rc == 0
    return out


def split_bounds(n_kv: int, n_split: int, tile: int = 64) -> np.ndarray:
    """Key boundaries of the balanced whole-tile partition used by the split-K kernels."""
    n_tiles = (n_kv + tile - 1) // tile
    base, rem = divmod(n_tiles, n_split)
    b = [0]
    for s in range(n_split):
        b.append(b[-1] + base + (1 if s < rem else 0))
    return np.minimum(np.array(b, dtype=np.int64) * tile, n_kv)


def partials(kcache: np.ndarray, q: np.ndarray, mask: Optional[np.ndarray], kq_scale: float, bounds: Sequence[int],
             d_v: int = 512) -> np.ndarray:
    kcache = np.ascontiguousarray(kcache)
    q = np.ascontiguousarray(q, dtype=np.float32)
    ty, es = _kc(kcache)
    n_kv, d_k = kcache.shape
    nt, H, _ = q.shape
    b = np.ascontiguousarray(bounds, dtype=np.int64)
    S = len(b) - 1
    part = np.empty((H, nt, S, 4 + d_v), dtype=np.float32)
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float32)
    rc = lib().orc_partials(_ptr(kcache), ty, d_k, n_kv, d_k * es, _ptr(q), H, nt, d_k * 4, H * d_k * 4,
                            _ptr(mask), n_kv * 4, kq_scale, d_v, _ptr(b), S, _ptr(part))
    assert rc == 0
    return part


def merge(part: np.ndarray, mutant: int = 0) -> np.ndarray:
    part = np.ascontiguousarray(part, dtype=np.float32)
    H, nt, S, rs = part.shape
    out = np.empty((H, nt, rs - 4), dtype=np.float32)
    rc = lib().orc_merge(_ptr(part), rs - 4, S, nt, H, _ptr(out), mutant)
    assert rc == 0
    return out


def wkb(w_kb: np.ndarray, q_nope: np.ndarray, threads: Optional[int] = None, mutant: int = 0) -> np.ndarray:
    """The unfused WKB: permute(mul_mat(W_kb, permute(q_nope))) (engine/m1_layer.cpp:444-446)."""
    w_kb = np.ascontiguousarray(w_kb, dtype=np.float32)
    H, d_v, d_n = w_kb.shape
    nt = q_nope.shape[0]
    qn = np.ascontiguousarray(q_nope, dtype=np.float32)
    out = np.empty((nt, H, d_v), dtype=np.float32)
    rc = lib().orc_wkb(_ptr(w_kb), d_n, d_v, H, _ptr(qn), nt, d_n * 4, H * d_n * 4, _ptr(out), d_v * 4,
                       H * d_v * 4, threads or max_threads(), mutant)
    assert rc == 0
    return out


def kqkv_bench_pattern(n_kv: int, d_k: int = 320, n_head: int = 32):
    """Known-answer inputs of engine/m1_kqkv_bench.hip:148-165 (kcache f16 [n_kv, d_k], q f32 [1, H, d_k])."""
    kc = np.empty(n_kv * d_k, dtype=np.uint16)
    q = np.empty(n_head * d_k, dtype=np.float32)
    lib().orc_kqkv_bench_pattern(kc.size, _ptr(kc), q.size, _ptr(q))
    return kc.view(np.float16).reshape(n_kv, d_k), q.reshape(1, n_head, d_k)


def mla_step(inp, threads: Optional[int] = None) -> tuple[np.ndarray, np.ndarray]:
    """The whole unfused decode/prefill step of a config: WKB, concat -> Qcur, KQKV.
    Returns (qcur [nt, H, 576], out [H, nt, 512])."""
    q_abs = wkb(inp.w_kb, inp.q_nope, threads=threads)
    qcur = np.concatenate([q_abs, inp.q_pe], axis=2).astype(np.float32)
    out = kqkv(inp.kcache, qcur, inp.mask, inp.kq_scale, d_v=inp.w_kb.shape[1], threads=threads)
    return qcur, out


os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")


# ---------------------------------------------------------------- Q8_0 x Q8_1 (reference geometry)
def q8_0_random(seed: int, rows: int, ne0: int, scale: float = 0.01) -> np.ndarray:
    """Random Q8_0 rows as raw bytes [rows, ne0 / 32 * 34]: int8 qs in [-127, 127] and positive f16
    scales (any valid Q8_0 bytes do; ggml's own quantiser is not needed to test the dot)."""
    nb = ne0 // 32
    r = np.random.default_rng(seed)
    qs = r.integers(-127, 128, size=(rows, nb, 32), dtype=np.int64).astype(np.int8)
    d = (np.abs(r.standard_normal((rows, nb))) * scale + scale / 8).astype(np.float16)
    out = np.empty((rows, nb, 34), dtype=np.uint8)
    out[:, :, :2] = d.view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.view(np.uint8)
    return out.reshape(rows, nb * 34)


def q8_0_dequant(w: np.ndarray, ne0: int) -> np.ndarray:
    """Q8_0 bytes [rows, ne0/32*34] -> f32 [rows, ne0] (d * qs): ggml's dequantize_row_q8_0
    (vendor/llama.cpp/ggml/src/ggml-quants.c:553-567; the f32 product is exact)."""
    rows = w.shape[0]
    nb = ne0 // 32
    b = np.ascontiguousarray(w).reshape(rows, nb, 34)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float32).reshape(rows, nb, 1)
    qs = b[:, :, 2:].copy().view(np.int8).astype(np.float32)
    return (d * qs).reshape(rows, ne0)


def q8_0_quantize(x: np.ndarray, mutant: int = 0) -> np.ndarray:
    """f32 rows [rows, ne0] -> Q8_0 bytes [rows, ne0/32*34]: ggml's reference quantiser
    quantize_row_q8_0_ref (vendor/llama.cpp/ggml/src/ggml-quants.c:276-299), per 32-value block:
    amax = max |x|, d = amax / 127 in f32, id = 1 / d in f32 (0 when d = 0), the stored scale
    f16(d) (round to nearest even), q = roundf(x * id) with the product in f32 and roundf's half
    away from zero.  (The 8-bit latent cache of the Q8_0 KQKV kernel is ggml's block_q8_0.)
    Test mutants (never used by the library): 1 rounds half to even, 2 takes id from the stored f16
    scale, 3 stores a scale one f16 ulp off the nearest."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, ne0 = x.shape
    assert ne0 % 32 == 0
    b = x.reshape(rows, ne0 // 32, 32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    d16 = d.astype(np.float16)
    dd = d16.astype(np.float32) if mutant == 2 else d
    with np.errstate(divide="ignore"):
        idv = np.where(dd != 0, np.float32(1.0) / dd, np.float32(0.0)).astype(np.float32)
    x0 = (b * idv[:, :, None]).astype(np.float32).astype(np.float64)     # the f32 product, exact in f64
    q = np.round(x0) if mutant == 1 else np.sign(x0) * np.floor(np.abs(x0) + 0.5)
    out = np.empty((rows, ne0 // 32, 34), dtype=np.uint8)
    if mutant == 3:
        d16 = (d16.view(np.uint16) ^ np.uint16(1)).view(np.float16)
    out[:, :, :2] = d16.view(np.uint8).reshape(rows, ne0 // 32, 2)
    out[:, :, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(rows, ne0 // 32 * 34)


def q8_0_dequant_f16(w: np.ndarray, ne0: int) -> np.ndarray:
    """Q8_0 bytes -> the f16 values the Q8_0 KQKV kernel computes with: f16(q * d), the product exact
    in f32 and rounded once (= an f32 dequantisation followed by a conversion to f16)."""
    return q8_0_dequant(w, ne0).astype(np.float16)


def wkb_q8(w: np.ndarray, d_n: int, d_v: int, n_head: int, q_nope: np.ndarray, mutant: int = 0) -> np.ndarray:
    """GGML_OP_M4_WKB with a Q8_0 W_kb (m4-wkb.cu:21-69): w bytes [H * d_v, d_n/32*34];
    q_nope f32 [nt, H, d_n] -> out [nt, H, d_v]."""
    q = np.ascontiguousarray(q_nope, dtype=np.float32)
    nt = q.shape[0]
    out = np.empty((nt, n_head, d_v), dtype=np.float32)
    rc = lib().orc_wkb_q8(_ptr(np.ascontiguousarray(w)), d_n, d_v, n_head, _ptr(q), nt, d_n * 4, n_head * d_n * 4,
                          _ptr(out), d_v * 4, n_head * d_v * 4, mutant)
    assert rc == 0
    return out


def wvb_q8(w: np.ndarray, d_in: int, d_out: int, n_head: int, x: np.ndarray, mutant: int = 0) -> np.ndarray:
    """GGML_OP_M4_PHASE phase 1 (m4-phase.cu:52-88): w bytes [H * d_out, d_in/32*34]; x f32
    [nt, H, d_in] -> out [nt, H, d_out]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nt = x.shape[0]
    out = np.empty((nt, n_head, d_out), dtype=np.float32)
    rc = lib().orc_wvb_q8(_ptr(np.ascontiguousarray(w)), d_in, d_out, n_head, _ptr(x), nt, d_in * 4,
                          n_head * d_in * 4, _ptr(out), d_out * 4, n_head * d_out * 4, mutant)
    assert rc == 0
    return out


def rope_yarn_corr_dims(n_dims: int, n_ctx_orig: int, freq_base: float, beta_fast: float, beta_slow: float):
    d = np.zeros(2, dtype=np.float32)
    lib().orc_rope_yarn_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, _ptr(d))
    return float(d[0]), float(d[1])


def kvwrite(cur: np.ndarray, w: np.ndarray, d_lat: int, n_rope: int, nw: np.ndarray, kcache_bits: np.ndarray,
            kidx: int, pos: int, rp: dict, mutant: int = 0) -> np.ndarray:
    """GGML_OP_M4_PHASE phase 0 (m4-phase.cu:95-200).  kcache_bits (uint16 [n_kv, >= d_lat + n_rope])
    is written in place (row kidx); returns dst = Kcur (f32 [d_lat + n_rope])."""
    cur = np.ascontiguousarray(cur, dtype=np.float32)
    assert kcache_bits.dtype == np.uint16 and kcache_bits.flags["C_CONTIGUOUS"]
    dst = np.empty(d_lat + n_rope, dtype=np.float32)
    rc = lib().orc_kvwrite(_ptr(cur), cur.shape[0], _ptr(np.ascontiguousarray(w)), d_lat, n_rope,
                           _ptr(np.ascontiguousarray(nw, dtype=np.float32)), _ptr(kcache_bits),
                           kcache_bits.shape[1] * 2, kidx, pos, rp["freq_base"], rp["freq_scale"],
                           rp["ext_factor"], rp["attn_factor"], rp["beta_fast"], rp["beta_slow"], rp["eps"],
                           rp["n_ctx_orig"], _ptr(dst), mutant)
    assert rc == 0
    return dst

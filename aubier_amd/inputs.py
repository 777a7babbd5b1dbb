"""Seeded synthetic inputs for the five MLA attention configurations (CPU, numpy).

Values are N(0,1)*0.05 from splitmix64 + Box-Muller, so they are identical on every platform
(std::normal_distribution and numpy's default generator are not portable across libraries).
Value i of a stream depends only on (seed, i): pair p = i // 2 seeds its own splitmix64 state
with seed ^ (0xD1B54A32D192ED03 * (p + 1)) and draws two uniforms u1, u2 in (0, 1];
z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2), computed in double and rounded
once to f32 after scaling by the f32 scale.  An f16 cache is cast with round-to-nearest-even after scaling.

Geometry (all configs): 32 heads, q = 128 nope + 64 rope per head, KV row = 512 latent + 64 rope,
W_kb [H][D_v][d_n] = ggml ne [128, 512, 32] f32, kq_scale = 1/sqrt(192), mask 0 / -inf.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import Optional

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
PAIR_MUL = np.uint64(0xD1B54A32D192ED03)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

SEED_BASE = 0x4D4C4134   # "MLA4"

N_HEAD, D_NOPE, D_ROPE, D_V = 32, 128, 64, 512
D_K = D_V + D_ROPE
KQ_SCALE = 1.0 / math.sqrt(D_NOPE + D_ROPE)
SENTINEL = 1000.0        # finite fill for masked tail keys (0 * sentinel = 0, never NaN)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def randn(seed: int, n: int, scale: float = 0.05) -> np.ndarray:
    """n f32 values N(0,1)*scale from the counter-based splitmix64/Box-Muller stream `seed`."""
    npairs = (n + 1) // 2
    scale = float(np.float32(scale))     # the scale is an f32 parameter (as in the C generator)
    out = np.empty(2 * npairs, dtype=np.float32)
    chunk = 1 << 22
    with np.errstate(over="ignore"):
        for p0 in range(0, npairs, chunk):
            p = np.arange(p0, min(npairs, p0 + chunk), dtype=np.uint64)
            s = np.uint64(seed) ^ (PAIR_MUL * (p + np.uint64(1)))
            s1 = s + GOLDEN
            s2 = s1 + GOLDEN
            u1 = ((_mix(s1) >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
            u2 = ((_mix(s2) >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
            r = np.sqrt(-2.0 * np.log(u1))
            th = 2.0 * math.pi * u2
            out[2 * p0:2 * p0 + 2 * len(p):2] = (r * np.cos(th) * scale).astype(np.float32)
            out[2 * p0 + 1:2 * p0 + 2 * len(p):2] = (r * np.sin(th) * scale).astype(np.float32)
    return out[:n]


def splitmix_u64(seed: int, n: int) -> np.ndarray:
    """n raw splitmix64 outputs of the sequential stream started at `seed` (for small draws)."""
    with np.errstate(over="ignore"):
        s = np.uint64(seed) + GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        return _mix(s)


def seed_of(cfg: int, stream: int) -> int:
    return SEED_BASE + 16 * cfg + stream


@dataclass
class MlaInputs:
    cfg: int
    n_kv: int                 # cache width W
    n_live: int               # L (keys not masked for the last token)
    nt: int
    kc_f16: bool
    kcache: np.ndarray        # [W, 576] float16 or float32
    q_nope: np.ndarray        # [nt, H, 128] f32
    q_pe: np.ndarray          # [nt, H, 64] f32
    w_kb: np.ndarray          # [H, 512, 128] f32
    mask: np.ndarray          # [nt, W] f32 (0 / -inf)
    kq_scale: float = KQ_SCALE
    seeds: dict = field(default_factory=dict)
    notes: str = ""
    kcache_q8: Optional[np.ndarray] = None   # [W, 612] uint8: the cache in ggml block_q8_0 (with_q8_cache)


def q8_0_rows(x: np.ndarray) -> np.ndarray:
    """f32 rows [rows, ne0] -> ggml block_q8_0 bytes [rows, ne0 / 32 * 34] (the algorithm of ggml's
    quantize_row_q8_0_ref: per 32 values d = amax / 127, the stored scale f16(d), q = roundf(x / d)
    computed as x * (1 / d) in f32, half away from zero): the 8-bit latent cache of the Q8_0 KQKV
    kernel, for synthetic caches."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, ne0 = x.shape
    b = x.reshape(rows, ne0 // 32, 32)
    d = (np.abs(b).max(axis=2) / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    x0 = (b * idv[:, :, None]).astype(np.float32).astype(np.float64)
    q = np.sign(x0) * np.floor(np.abs(x0) + 0.5)
    out = np.empty((rows, ne0 // 32, 34), dtype=np.uint8)
    out[:, :, :2] = d.astype(np.float16).view(np.uint8).reshape(rows, ne0 // 32, 2)
    out[:, :, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(rows, ne0 // 32 * 34)


def q8_0_rows_f16(w: np.ndarray, ne0: int) -> np.ndarray:
    """block_q8_0 bytes -> the f16 values a Q8_0 kernel computes with, f16(q * d)."""
    b = np.ascontiguousarray(w).reshape(w.shape[0], ne0 // 32, 34)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float32).reshape(w.shape[0], ne0 // 32, 1)
    return (d * b[:, :, 2:].copy().view(np.int8).astype(np.float32)).reshape(w.shape[0], ne0).astype(np.float16)


def with_q8_cache(inp: MlaInputs) -> MlaInputs:
    """The same inputs with the cache quantised to ggml block_q8_0: kcache_q8 holds the bytes and
    kcache the f16 values they stand for (so any f16-cache reference on kcache is the reference of
    a Q8_0 kernel on kcache_q8)."""
    wq = q8_0_rows(inp.kcache.astype(np.float32))
    return replace(inp, kcache_q8=wq, kcache=q8_0_rows_f16(wq, inp.kcache.shape[1]), kc_f16=True,
                   notes=(inp.notes + "; " if inp.notes else "") + "cache in Q8_0")


def make_config(cfg: int, n_kv: Optional[int] = None, nt: Optional[int] = None) -> MlaInputs:
    """Inputs of BASELINE config `cfg` (1..5).  n_kv / nt override the sizes (tests use smaller
    windows with the same construction)."""
    sd = {k: seed_of(cfg, i) for i, k in enumerate(["kcache", "q_nope", "q_pe", "w_kb", "aux"])}
    notes = ""
    if cfg == 1:
        W, T, f16 = 256, 1, False
    elif cfg == 2:
        W, T, f16 = 4096, 1, True
    elif cfg == 3:
        W, T, f16 = 32768, 1, True
    elif cfg == 4:
        W, T, f16 = 262144, 1, True
    elif cfg == 5:
        W, T, f16 = 8192, 512, True
    else:
        raise ValueError(cfg)
    if n_kv is not None:
        W = n_kv
    if nt is not None:
        T = nt
    kc = randn(sd["kcache"], W * D_K).reshape(W, D_K)
    aux = splitmix_u64(sd["aux"], 4)
    mask = np.zeros((T, W), dtype=np.float32)
    L = W
    if cfg == 3:
        # 16 consecutive keys at a seeded offset get their rope columns scaled x8 (before the cast)
        off = int(aux[0] % np.uint64(max(1, W - 16)))
        kc[off:off + 16, D_V:] *= 8.0
        notes = f"rope x8 on keys [{off}, {off + 16})"
    if cfg == 4:
        r = 1 + int(aux[1] % np.uint64(255))
        L = W - r
        kc[L:, :] = SENTINEL
        mask[:, L:] = -np.inf
        notes = f"{r} masked tail keys filled with {SENTINEL}"
    if cfg == 5:
        # causal chunked prefill: token t sees keys [0, W - T + t]
        cached = W - T
        j = np.arange(W)[None, :]
        t = np.arange(T)[:, None]
        mask[j > cached + t] = -np.inf
        L = W
        notes = f"causal, {cached} cached + {T} new"
    kcache = kc.astype(np.float16) if f16 else kc
    q_nope = randn(sd["q_nope"], T * N_HEAD * D_NOPE).reshape(T, N_HEAD, D_NOPE)
    q_pe = randn(sd["q_pe"], T * N_HEAD * D_ROPE).reshape(T, N_HEAD, D_ROPE)
    w_kb = randn(sd["w_kb"], N_HEAD * D_V * D_NOPE).reshape(N_HEAD, D_V, D_NOPE)
    return MlaInputs(cfg=cfg, n_kv=W, n_live=L, nt=T, kc_f16=f16, kcache=kcache, q_nope=q_nope, q_pe=q_pe,
                     w_kb=w_kb, mask=mask, seeds=sd, notes=notes)


def make_batch(n_seq: int, region: int, lens: Optional[list] = None, seed_cfg: int = 6) -> MlaInputs:
    """Batch-of-N decode (the engine's per-sequence regions, m1_layer.h:212-223 / m1_session.h:188-201):
    one cache window of width n_seq * region, sequence s owning cells [s * region, (s + 1) * region);
    row s's mask is 0 on [s * region, s * region + len_s) and -inf elsewhere.  len_s is seeded in
    [1, region] unless given.  Cache values, q and W_kb as config 2 (f16 cache, N(0,1) * 0.05)."""
    W = n_seq * region
    sd = {k: seed_of(seed_cfg, i) for i, k in enumerate(["kcache", "q_nope", "q_pe", "w_kb", "aux"])}
    if lens is None:
        r = splitmix_u64(sd["aux"], n_seq)
        lens = [1 + int(r[i] % np.uint64(region)) for i in range(n_seq)]
    assert len(lens) == n_seq and all(1 <= l <= region for l in lens)
    mask = np.full((n_seq, W), -np.inf, dtype=np.float32)
    for i, l in enumerate(lens):
        mask[i, i * region:i * region + l] = 0.0
    kcache = randn(sd["kcache"], W * D_K).reshape(W, D_K).astype(np.float16)
    q_nope = randn(sd["q_nope"], n_seq * N_HEAD * D_NOPE).reshape(n_seq, N_HEAD, D_NOPE)
    q_pe = randn(sd["q_pe"], n_seq * N_HEAD * D_ROPE).reshape(n_seq, N_HEAD, D_ROPE)
    w_kb = randn(sd["w_kb"], N_HEAD * D_V * D_NOPE).reshape(N_HEAD, D_V, D_NOPE)
    return MlaInputs(cfg=seed_cfg, n_kv=W, n_live=max(lens), nt=n_seq, kc_f16=True, kcache=kcache, q_nope=q_nope,
                     q_pe=q_pe, w_kb=w_kb, mask=mask, seeds=sd, notes=f"{n_seq} sequences x {region} cells, lens {lens}")

"""Writes tests/golden/kqkv_bench_pattern.npz: the known-answer inputs of the reference's
standalone KQKV bench (engine/m1_kqkv_bench.hip:148-165) at a small size, with the expected
output computed here in float64 by numpy alone (no oracle, no reference code):

    K[i] = ((i * 7919) % 1000) / 1000 - 0.5, stored as f16 by the bench's own conversion
           (mantissa truncated, f16 subnormals flushed to zero);
    q[i] = ((i * 3571) % 1000) / 1000 - 0.5 in f32;   kq_scale = 1/sqrt(320) (the bench's).
    out_f64          = softmax(kq_scale * q.K^T) . V        (no f16 rounding)
    out_f64_rounded  = the same with q and P rounded to f16 (ggml-cpu's F16 mul_mat)

Geometry: the reference's (D_k, D_v) = (320, 256), n_kv = 300 keys, 4 heads, one token.
Run:  python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

N_KV, N_HEAD, D_K, D_V = 300, 4, 320, 256


def bench_f16_bits(v: np.ndarray) -> np.ndarray:
    bits = v.astype(np.float32).view(np.uint32)
    sign = (bits >> 16) & 0x8000
    e = ((bits >> 23) & 0xFF).astype(np.int64) - 127 + 15
    mant = (bits >> 13) & 0x3FF
    normal = (sign | (np.clip(e, 0, 31).astype(np.uint32) << 10) | mant)
    out = np.where(e >= 31, sign | 0x7C00, np.where(e <= 0, sign, normal))
    return out.astype(np.uint16)


def attn(kc: np.ndarray, q: np.ndarray, scale: float, round16: bool) -> np.ndarray:
    K = kc.astype(np.float64)
    Q = q.astype(np.float16).astype(np.float64) if round16 else q.astype(np.float64)
    s = np.einsum("thd,kd->thk", Q, K) * scale
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    if round16:
        p = p.astype(np.float32).astype(np.float16).astype(np.float64)
    return np.einsum("thk,kc->htc", p, K[:, :D_V])


def main() -> None:
    i = np.arange(N_KV * D_K, dtype=np.int64)
    k = ((i * 7919) % 1000).astype(np.float32) / np.float32(1000.0) - np.float32(0.5)
    kbits = bench_f16_bits(k).reshape(N_KV, D_K)
    j = np.arange(N_HEAD * D_K, dtype=np.int64)
    q = (((j * 3571) % 1000).astype(np.float32) / np.float32(1000.0) - np.float32(0.5)).reshape(1, N_HEAD, D_K)
    kc = kbits.view(np.float16)
    scale = np.float32(1.0 / np.sqrt(320.0))
    out = Path(__file__).resolve().parent / "kqkv_bench_pattern.npz"
    np.savez_compressed(out, n_kv=np.int64(N_KV), n_head=np.int64(N_HEAD), kq_scale=scale,
                        kcache_bits=kbits, q=q,
                        out_f64=attn(kc, q, float(scale), False),
                        out_f64_rounded=attn(kc, q, float(scale), True))
    print(f"wrote {out}")


if __name__ == "__main__":
    main()

"""CPU tests that pin the oracle (oracle/, the C restatement of the reference's unfused ggml graph)
before it is trusted as the checker of the GPU kernels.

Nothing here retypes the oracle's formulas: each function is checked against an independent
computation (numpy float64 routines, numpy's own f16 conversion), a closed form the mathematics
fixes (identity W_kb, one dominant key, uniform scores, a one-key window), an invariant (key
permutation, the masked-tail sentinel, split/merge for any partition), or the reference's own
known-answer input pattern (engine/m1_kqkv_bench.hip:148-165) with the committed fixture of
tests/golden/.  Planted mistakes (the oracle's test-only `mutant` switch) must fail those checks.
"""
from pathlib import Path

import numpy as np
import pytest

from aubier_amd import inputs as I
from oracle import oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------------------------ helpers
def rnd(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def attn64(kc, q, mask, scale, d_v, q_round16=False, p_round16=False):
    """numpy float64 softmax attention; optional f16 rounding of q and of the normalised P (the
    rounding points of ggml-cpu's mul_mat for an F16 src0).  kc [n_kv, D_k], q [nt, H, D_k],
    mask [nt, n_kv] or None -> [H, nt, d_v]."""
    K = kc.astype(np.float64)
    Q = q.astype(np.float16).astype(np.float64) if q_round16 else q.astype(np.float64)
    s = np.einsum("thd,kd->thk", Q, K) * scale
    if mask is not None:
        s = s + mask.astype(np.float64)[:, None, :]
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    P = e / e.sum(axis=-1, keepdims=True)
    if p_round16:
        P = P.astype(np.float32).astype(np.float16).astype(np.float64)
    out = np.einsum("thk,kc->htc", P, K[:, :d_v])
    return out


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max() / np.abs(b).max())


def small_case(seed=1, n_kv=200, H=4, nt=2, d_k=96, d_v=64, f16=False, mask=True, scale=None):
    kc = rnd(seed, (n_kv, d_k), 0.5)
    q = rnd(seed + 1, (nt, H, d_k), 0.5)
    m = None
    if mask:
        g = np.random.default_rng(seed + 2)
        m = np.where(g.random((nt, n_kv)) < 0.3, -np.inf, 0.0).astype(np.float32)
        m[:, 0] = 0.0                      # at least one live key per row
    if f16:
        kc = kc.astype(np.float16)
    sc = float(np.float32(1.0 / np.sqrt(d_k) if scale is None else scale))   # kq_scale is an f32 op param
    return kc, q, m, sc, d_v


# ------------------------------------------------------------------------------ conversions
def test_f16_to_f32_exhaustive():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    g = np.random.default_rng(7)
    x = np.concatenate([
        (g.standard_normal(200000) * np.exp2(g.integers(-30, 20, 200000))).astype(np.float32),
        # exact ties between two f16 values (normal and subnormal), the overflow boundary, specials
        (np.arange(1, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        np.array([65504, 65519.99, 65520, 65536, 1e30, -1e30, 0.0, -0.0, 2.0 ** -25, 2.0 ** -26,
                  np.inf, -np.inf], dtype=np.float32),
    ])
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.isnan(orc.f16_bits_to_f32(orc.f32_to_f16_bits(np.array([np.nan], np.float32))))[0]


# ------------------------------------------------------------------------------ generator
@pytest.mark.parametrize("seed", [0, 1, I.SEED_BASE + 49])
def test_randn_matches_numpy_generator(seed):
    a = orc.randn(seed, 100001)
    b = I.randn(seed, 100001)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # value i depends only on (seed, i)
    assert np.array_equal(orc.randn(seed, 1001), a[:1001])
    # N(0, 1) * 0.05
    assert abs(float(a.mean())) < 0.05 * 0.02 and abs(float(a.std()) / 0.05 - 1.0) < 0.01


def test_kqkv_bench_pattern_known_inputs():
    kc, q = orc.kqkv_bench_pattern(64, d_k=320, n_head=2)
    i = np.arange(64 * 320)
    v = ((i * 7919) % 1000).astype(np.float32) / np.float32(1000.0) - np.float32(0.5)
    # the bench's conversion truncates the mantissa (round toward zero) and flushes f16 subnormals
    bits = v.view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int64) - 127 + 15
    trunc = (((bits >> 16) & 0x8000) | np.where(e > 0, (e.clip(0, 31) << 10) | ((bits >> 13) & 0x3FF), 0)).astype(np.uint16)
    assert np.array_equal(kc.reshape(-1).view(np.uint16), trunc)
    j = np.arange(2 * 320)
    assert np.array_equal(q.reshape(-1), ((j * 3571) % 1000).astype(np.float32) / np.float32(1000.0) - np.float32(0.5))


# ------------------------------------------------------------------------------ KQKV
def test_attn_f64_matches_numpy():
    kc, q, m, sc, dv = small_case(f16=True)
    assert rel(orc.attn_f64(kc, q, m, sc, d_v=dv), attn64(kc, q, m, sc, dv)) < 1e-12


def test_kqkv_f32_cache_matches_float64():
    kc, q, m, sc, dv = small_case()
    assert rel(orc.kqkv(kc, q, m, sc, d_v=dv), attn64(kc, q, m, sc, dv)) < 3e-6


def test_kqkv_f16_cache_follows_ggml_rounding_points():
    kc, q, m, sc, dv = small_case(f16=True, n_kv=300)
    got = orc.kqkv(kc, q, m, sc, d_v=dv)
    emul = attn64(kc, q, m, sc, dv, q_round16=True, p_round16=True)
    plain = attn64(kc, q, m, sc, dv)
    # f32 vs f64 exp/dot can move a P value across an f16 rounding boundary: a few f16 ulps
    assert rel(got, emul) < 2e-4
    # ... while the rounding points themselves are a larger, visible effect
    assert rel(got, plain) > 3 * rel(got, emul)


def test_kqkv_dominant_key_returns_its_value_row():
    kc, q, _, _, dv = small_case(n_kv=120, H=3, nt=1, mask=False)
    j = 77
    kc[j] = q[0, 0] * 40.0                 # head 0: key j's score dwarfs every other
    out = orc.kqkv(kc, q, None, 1.0, d_v=dv)
    assert np.allclose(out[0, 0], kc[j, :dv], rtol=0, atol=1e-6 * np.abs(kc[j, :dv]).max())


def test_kqkv_zero_scale_is_mean_of_live_rows():
    kc, q, m, _, dv = small_case(n_kv=150, H=2, nt=2)
    out = orc.kqkv(kc, q, m, 0.0, d_v=dv)
    for t in range(2):
        live = m[t] == 0
        assert np.allclose(out[:, t], kc[live, :dv].astype(np.float64).mean(0)[None], atol=2e-6)


def test_kqkv_single_key_window():
    kc, q, _, sc, dv = small_case(n_kv=1, H=5, nt=3, mask=False)
    out = orc.kqkv(kc, q, None, sc, d_v=dv)
    assert np.array_equal(out, np.broadcast_to(kc[0, :dv], out.shape))


def test_kqkv_key_permutation_invariance():
    kc, q, m, sc, dv = small_case(n_kv=257, f16=True)
    perm = np.random.default_rng(3).permutation(kc.shape[0])
    a = orc.kqkv(kc, q, m, sc, d_v=dv)
    b = orc.kqkv(kc[perm], q, m[:, perm], sc, d_v=dv)
    assert rel(b, a) < 1e-5


def test_kqkv_masked_tail_sentinel_invariance():
    kc, q, _, sc, dv = small_case(n_kv=300, nt=1, mask=False)
    live = 241
    m = np.zeros((1, 300), np.float32)
    m[:, live:] = -np.inf
    filled = kc.copy()
    filled[live:] = I.SENTINEL
    a = orc.kqkv(filled, q, m, sc, d_v=dv)
    b = orc.kqkv(kc[:live], q, None, sc, d_v=dv)
    assert np.array_equal(a, b)


def test_known_answer_pattern_fixture():
    """The reference bench's deterministic inputs; the expected output was computed once in float64
    by tests/golden/make_golden.py (numpy only) and committed."""
    fx = np.load(GOLDEN / "kqkv_bench_pattern.npz", allow_pickle=False)
    kc, q = orc.kqkv_bench_pattern(int(fx["n_kv"]), d_k=320, n_head=int(fx["n_head"]))
    assert np.array_equal(kc.view(np.uint16), fx["kcache_bits"])
    assert np.array_equal(q, fx["q"])
    sc = float(fx["kq_scale"])
    assert rel(orc.attn_f64(kc, q, None, sc, d_v=256), fx["out_f64"]) < 1e-12
    got = orc.kqkv(kc, q, None, sc, d_v=256)
    assert rel(got, fx["out_f64_rounded"]) < 2e-4            # f16 q/P rounding points
    assert rel(got, fx["out_f64"]) < 2e-2


# ------------------------------------------------------------------------------ split-K
@pytest.mark.parametrize("S", [1, 2, 5, 13])
def test_partials_merge_equals_full_softmax(S):
    kc, q, m, sc, dv = small_case(n_kv=64 * 13 + 7)
    ref = attn64(kc, q, m, sc, dv)
    part = orc.partials(kc, q, m, sc, orc.split_bounds(kc.shape[0], S), d_v=dv)
    assert rel(orc.merge(part), ref) < 2e-6


def test_merge_of_one_split_is_normalised_output():
    kc, q, m, sc, dv = small_case(n_kv=100)
    part = orc.partials(kc, q, m, sc, [0, 100], d_v=dv)
    assert np.allclose(orc.merge(part)[..., :], part[..., 0, 4:] / part[..., 0, 1:2], rtol=1e-6, atol=0)


def test_merge_skips_empty_splits_and_all_empty_gives_zero():
    kc, q, _, sc, dv = small_case(n_kv=128, nt=1, mask=False)
    m = np.zeros((1, 128), np.float32)
    m[:, 64:] = -np.inf                      # the second split is fully masked
    part = orc.partials(kc, q, m, sc, [0, 64, 128], d_v=dv)
    assert np.all(part[..., 1, 0] == -np.inf)
    assert rel(orc.merge(part), attn64(kc[:64], q, None, sc, dv)) < 2e-6
    part[..., 0, 0] = -np.inf
    assert np.array_equal(orc.merge(part), np.zeros_like(orc.merge(part)))


def test_split_bounds_balanced_whole_tiles():
    b = orc.split_bounds(64 * 10 + 5, 4)
    assert list(b) == [0, 192, 384, 576, 645]


# ------------------------------------------------------------------------------ WKB
def test_wkb_matches_float64():
    w = rnd(11, (4, 96, 64), 0.1)
    qn = rnd(12, (3, 4, 64))
    got = orc.wkb(w, qn)
    ref = np.einsum("hcd,thd->thc", w.astype(np.float64), qn.astype(np.float64))
    assert rel(got, ref) < 1e-6


def test_wkb_identity_blocks_and_zero_query():
    H, dv, dn = 3, 96, 64
    w = np.zeros((H, dv, dn), np.float32)
    w[:, :dn, :] = np.eye(dn, dtype=np.float32)
    qn = rnd(13, (2, H, dn))
    out = orc.wkb(w, qn)
    assert np.array_equal(out[..., :dn], qn) and not out[..., dn:].any()
    assert not orc.wkb(rnd(14, (H, dv, dn)), np.zeros((2, H, dn), np.float32)).any()


def test_mla_step_is_wkb_then_concat_then_kqkv():
    inp = I.make_config(2, n_kv=256)
    qcur, out = orc.mla_step(inp)
    assert np.array_equal(qcur[..., :I.D_V], orc.wkb(inp.w_kb, inp.q_nope))
    assert np.array_equal(qcur[..., I.D_V:], inp.q_pe)
    assert np.array_equal(out, orc.kqkv(inp.kcache, qcur, inp.mask, inp.kq_scale))


# ------------------------------------------------------------------------------ negative controls
def test_mutants_fail_the_checks():
    """Each planted mistake must be caught by the check above that targets it."""
    kc, q, m, sc, dv = small_case()
    ref = attn64(kc, q, m, sc, dv)
    assert rel(orc.kqkv(kc, q, m, sc, d_v=dv, mutant=1), ref) > 1e-2        # kq_scale dropped
    assert rel(orc.kqkv(kc, q, m, sc, d_v=dv, mutant=3), ref) > 1e-2        # V read from the rope end
    assert rel(orc.kqkv(kc, q, m, sc, d_v=dv, mutant=4), ref) > 1e-2        # mask row of token 0 reused
    k16, q16, m16, sc16, dv16 = small_case(f16=True, n_kv=300)
    emul = attn64(k16, q16, m16, sc16, dv16, q_round16=True, p_round16=True)
    assert rel(orc.kqkv(k16, q16, m16, sc16, d_v=dv16, mutant=2), emul) > 2e-4   # no f16 rounding
    w = rnd(15, (2, 64, 64), 0.1)
    qn = rnd(16, (1, 2, 64))
    ref_w = np.einsum("hcd,thd->thc", w.astype(np.float64), qn.astype(np.float64))
    assert rel(orc.wkb(w, qn, mutant=5), ref_w) > 1e-2                        # W block transposed
    part = orc.partials(kc, q, m, sc, orc.split_bounds(kc.shape[0], 3), d_v=dv)
    assert rel(orc.merge(part, mutant=6), ref) > 1e-3                         # l not rescaled

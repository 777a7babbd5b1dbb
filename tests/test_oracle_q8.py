"""CPU checks that pin the oracle's Q8_0 x Q8_1 restatements (oracle/mla_oracle.c: orc_wkb_q8,
orc_wvb_q8, orc_kvwrite, orc_rope_yarn_corr_dims) -- the reference geometry's quantised ops
(patches/ggml-m4/m4-wkb.cu:21-69, m4-phase.cu:52-200).  The reference holds no vectors for them, so
they are pinned by:
  * exact closed forms: inputs whose activation quantisation is exact (block maxima 127 * 2^-7,
    entries integer multiples of 2^-7) and power-of-two weight scales, where every product and
    sum is exact in f32, so the result must equal the integer arithmetic bit for bit;
  * the bound of the quantisation error against a float64 dot of the dequantised weights;
  * RMS-norm and rope closed forms (pos = 0; the textbook rotation with YaRN off) and the YaRN
    correction dims worked out by hand;
  * planted mutants (block mix-up, the other quantisation form, a serial sum for the butterfly, a
    sign slip in the rotation, the wrong cache row) that must fail.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def exact_q8(rng, rows, ne0, qmax=7, d_exp=-6):
    """Q8_0 bytes with qs in [-qmax, qmax] and every scale 2^d_exp."""
    nb = ne0 // 32
    qs = rng.integers(-qmax, qmax + 1, size=(rows, nb, 32)).astype(np.int8)
    d = np.full((rows, nb), 2.0 ** d_exp, dtype=np.float16)
    out = np.empty((rows, nb, 34), dtype=np.uint8)
    out[:, :, :2] = d.view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.view(np.uint8)
    return out.reshape(rows, nb * 34), qs.astype(np.int64)


def exact_act(rng, shape, n):
    """f32 activations [..., n]: per 32-block one entry +-127 * 2^-7 (so d = 2^-7 exactly), the rest
    integers in [-7, 7] times 2^-7; returns (x, integer quants)."""
    qi = rng.integers(-7, 8, size=shape + (n,)).astype(np.int64)
    blocks = qi.reshape(shape + (n // 32, 32))
    pos = rng.integers(0, 32, size=shape + (n // 32,))
    sign = rng.choice([-1, 1], size=shape + (n // 32,))
    np.put_along_axis(blocks, pos[..., None], (127 * sign)[..., None], axis=-1)
    qi = blocks.reshape(shape + (n,))
    return (qi.astype(np.float64) * 2.0 ** -7).astype(np.float32), qi


@pytest.mark.parametrize("d_n,d_v", [(64, 256), (128, 512)])
def test_wkb_q8_exact_closed_form(d_n, d_v):
    rng = np.random.default_rng(11)
    H, nt = 4, 3
    w, qs = exact_q8(rng, H * d_v, d_n)
    x, qx = exact_act(rng, (nt, H), d_n)
    got = orc.wkb_q8(w, d_n, d_v, H, x)
    # sum_b 2^-6 * 2^-7 * sum_k qw qx -- exact in f32 at these magnitudes
    ref = np.einsum("hcd,thd->thc", qs.reshape(H, d_v, d_n), qx) * 2.0 ** -13
    assert np.array_equal(got, ref.astype(np.float32))
    assert not np.array_equal(orc.wkb_q8(w, d_n, d_v, H, x, mutant=2), got)


def test_wkb_q8_quantisation_error_bound():
    rng = np.random.default_rng(12)
    H, d_n, d_v, nt = 32, 64, 256, 2
    w = orc.q8_0_random(13, H * d_v, d_n)
    x = (rng.standard_normal((nt, H, d_n)) * 0.05).astype(np.float32)
    got = orc.wkb_q8(w, d_n, d_v, H, x).astype(np.float64)
    wf = orc.q8_0_dequant(w, d_n).reshape(H, d_v, d_n).astype(np.float64)
    ref = np.einsum("hcd,thd->thc", wf, x.astype(np.float64))
    # per element |x - q d16| <= d / 2 + |q| |d - d16| (d16 = f16(d): relative 2^-11) <= d (1/2 + 127 * 2^-11)
    amax = np.abs(x.reshape(nt, H, d_n // 32, 32)).max(-1) / 127.0                       # d per block
    dq = np.repeat(amax * (0.5 + 127 * 2.0 ** -11), 32, axis=-1)                          # [nt, H, d_n]
    bound = np.einsum("hcd,thd->thc", np.abs(wf), dq) * 1.001 + 1e-6
    assert np.all(np.abs(got - ref) <= bound)
    assert np.abs(got - ref).max() > 0                      # the quantisation is really there


def test_wkb_q8_uses_the_division_form():
    """m4-wkb.cu:47 quantises with roundf(x / d); the PHASE kernels with roundf(x * (1/d)).  Find
    an activation where the two round differently and check the oracle follows the division."""
    rng = np.random.default_rng(14)
    H, d_n, d_v = 1, 32, 32
    w, qs = exact_q8(rng, d_v, d_n, qmax=1, d_exp=0)

    def roundf(v):                               # C roundf: half away from zero (v is f32, exact in f64)
        v = np.float64(v)
        return np.sign(v) * np.floor(np.abs(v) + 0.5)

    found = None
    for amax in rng.uniform(0.5, 2.0, 64).astype(np.float32):     # walk f32 neighbours of (k + 1/2) d
        d = np.float32(amax / np.float32(127.0))
        idv = np.float32(np.float32(1.0) / d)
        for k in range(126):
            x0 = np.float32((k + 0.5) * np.float64(d))
            for step in range(-3, 4):
                x1 = np.nextafter(x0, np.float32(np.inf) if step > 0 else np.float32(-np.inf), dtype=np.float32) \
                    if step else x0
                for _ in range(abs(step) - 1):
                    x1 = np.nextafter(x1, np.float32(np.inf) if step > 0 else np.float32(-np.inf), dtype=np.float32)
                if roundf(np.float32(x1 / d)) != roundf(np.float32(x1 * idv)):
                    found = (amax, x1, d)
                    break
            if found:
                break
        if found:
            break
    assert found, "no activation separates roundf(x / d) from roundf(x * (1 / d))"
    amax, x1, d = found
    x = np.zeros(32, dtype=np.float32)
    x[0], x[5] = amax, x1
    q_div = np.array([roundf(np.float32(v / d)) for v in x])
    xs = x.reshape(1, 1, 32)
    a = orc.wkb_q8(w, d_n, d_v, H, xs)
    b = orc.wkb_q8(w, d_n, d_v, H, xs, mutant=1)
    d16 = np.float32(np.float16(d))
    expect = (qs.reshape(d_v, 32) @ q_div.astype(np.int64)).astype(np.float64) * float(d16)
    assert np.array_equal(a[0, 0], expect.astype(np.float32))
    assert not np.array_equal(a, b)


@pytest.mark.parametrize("d_in,d_out", [(256, 128), (512, 128)])
def test_wvb_q8_exact_closed_form(d_in, d_out):
    rng = np.random.default_rng(21)
    H, nt = 4, 2
    w, qs = exact_q8(rng, H * d_out, d_in)
    x, qx = exact_act(rng, (nt, H), d_in)
    got = orc.wvb_q8(w, d_in, d_out, H, x)
    ref = np.einsum("hod,thd->tho", qs.reshape(H, d_out, d_in), qx) * 2.0 ** -13
    assert np.array_equal(got, ref.astype(np.float32))


def test_wvb_q8_butterfly_and_bound():
    rng = np.random.default_rng(22)
    H, d_in, d_out, nt = 32, 256, 128, 1
    w = orc.q8_0_random(23, H * d_out, d_in)
    x = (rng.standard_normal((nt, H, d_in)) * 0.05).astype(np.float32)
    got = orc.wvb_q8(w, d_in, d_out, H, x)
    serial = orc.wvb_q8(w, d_in, d_out, H, x, mutant=2)
    assert not np.array_equal(got, serial)                 # the association is observable ...
    assert np.allclose(got, serial, rtol=1e-5, atol=1e-7)   # ... at the f32 rounding level
    wf = orc.q8_0_dequant(w, d_in).reshape(H, d_out, d_in).astype(np.float64)
    ref = np.einsum("hod,thd->tho", wf, x.astype(np.float64))
    amax = np.abs(x.reshape(nt, H, d_in // 32, 32)).max(-1) / 127.0
    dq = np.repeat(amax * (0.5 + 127 * 2.0 ** -11), 32, axis=-1)
    bound = np.einsum("hod,thd->tho", np.abs(wf), dq) * 1.001 + 1e-6
    assert np.all(np.abs(got - ref) <= bound)


def test_rope_yarn_corr_dims_known_values():
    # n_dims ln(n_ctx / (beta 2 pi)) / (2 ln base): 64 ln(4096 / 64 pi) / (2 ln 1e4) = 10.47 -> floor 10,
    # 64 ln(4096 / 2 pi) / (2 ln 1e4) = 22.50 -> ceil 23; clamped into [0, n_dims - 1]
    assert orc.rope_yarn_corr_dims(64, 4096, 10000.0, 32.0, 1.0) == (10.0, 23.0)
    assert orc.rope_yarn_corr_dims(64, 4096, 10000.0, 1e6, 1e-6) == (0.0, 63.0)


RP_PLAIN = dict(freq_base=10000.0, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
                eps=1e-6, n_ctx_orig=4096)
RP_YARN = dict(freq_base=1e6, freq_scale=0.25, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
               eps=1e-5, n_ctx_orig=8192)


def kv_inputs(rng, n_embd, d_lat, n_rope, n_kv):
    w, qs = exact_q8(rng, d_lat + n_rope, n_embd)
    cur, qx = exact_act(rng, (), n_embd)
    nw = (1.0 + 0.25 * rng.standard_normal(d_lat)).astype(np.float32)
    kc = rng.integers(0, 0x7bff, size=(n_kv, d_lat + n_rope)).astype(np.uint16)
    gemv = (qs.reshape(d_lat + n_rope, n_embd) @ qx) * 2.0 ** -13          # exact
    return w, cur, nw, kc, gemv


@pytest.mark.parametrize("n_embd,d_lat", [(4096, 256), (7168, 512)])
def test_kvwrite_pos0_closed_form(n_embd, d_lat):
    """pos = 0: the rope is a pure scaling by mscale; the latent rows are the RMS norm."""
    rng = np.random.default_rng(31)
    n_rope, n_kv, row = 64, 40, 17
    w, cur, nw, kc, gemv = kv_inputs(rng, n_embd, d_lat, n_rope, n_kv)
    kc0 = kc.copy()
    for rp in (RP_PLAIN, RP_YARN):
        kc = kc0.copy()
        dst = orc.kvwrite(cur, w, d_lat, n_rope, nw, kc, row, 0, rp)
        v = gemv[:d_lat]
        norm = v / np.sqrt((v ** 2).mean() + rp["eps"]) * nw
        assert np.allclose(dst[:d_lat], norm, rtol=2e-6, atol=1e-7)
        ms = rp["attn_factor"] * ((1.0 + 0.1 * np.log(1.0 / rp["freq_scale"])) if rp["ext_factor"] else 1.0)
        assert np.allclose(dst[d_lat:], gemv[d_lat:] * ms, rtol=2e-6, atol=1e-7)
        # the cache received exactly this row as f16 (round to nearest even), nothing else changed
        assert np.array_equal(kc[row], dst.astype(np.float16).view(np.uint16))
        others = np.ones(n_kv, bool)
        others[row] = False
        assert np.array_equal(kc[others], kc0[others])
    kc = kc0.copy()
    orc.kvwrite(cur, w, d_lat, n_rope, nw, kc, row, 0, RP_PLAIN, mutant=2)
    assert np.array_equal(kc[row], kc0[row])                # the wrong-row mutant is caught


@pytest.mark.parametrize("pos", [1, 37, 1000])
def test_kvwrite_rope_textbook(pos):
    """YaRN off (ext_factor 0, freq_scale 1, attn_factor 1): pair p rotated by pos base^(-2p/n)."""
    rng = np.random.default_rng(32)
    n_embd, d_lat, n_rope = 4096, 256, 64
    w, cur, nw, kc, gemv = kv_inputs(rng, n_embd, d_lat, n_rope, 4)
    dst = orc.kvwrite(cur, w, d_lat, n_rope, nw, kc, 1, pos, RP_PLAIN)
    x0, x1 = gemv[d_lat::2], gemv[d_lat + 1::2]
    th = pos * 10000.0 ** (-2.0 * np.arange(n_rope // 2) / n_rope)
    r0 = x0 * np.cos(th) - x1 * np.sin(th)
    r1 = x0 * np.sin(th) + x1 * np.cos(th)
    tol = 1e-6 + 4e-7 * pos * np.abs(gemv[d_lat:]).max()    # f32 theta: ~pos ulp of the angle
    assert np.abs(dst[d_lat::2] - r0).max() <= tol
    assert np.abs(dst[d_lat + 1::2] - r1).max() <= tol
    bad = orc.kvwrite(cur, w, d_lat, n_rope, nw, kc, 1, pos, RP_PLAIN, mutant=1)
    assert np.abs(bad[d_lat + 1::2] - r1).max() > 10 * tol


def yarn_corr_dims_f64(n_dims, n_ctx_orig, base, beta_fast, beta_slow):
    """The YaRN correction range (Peng et al., 2023, reference implementation
    `_yarn_find_correction_range`): the pair index at which a frequency completes `beta` rotations
    over the original context, floor / ceil, clamped to [0, n_dims - 1]; computed in float64."""
    def dim(rot):
        return n_dims * math.log(n_ctx_orig / (rot * 2.0 * math.pi)) / (2.0 * math.log(base))
    return max(0.0, math.floor(dim(beta_fast))), min(n_dims - 1.0, math.ceil(dim(beta_slow)))


def yarn_theta_f64(pos, p, n_dims, rp):
    """theta of pair p under YaRN, written from the paper's reference implementation: a linear
    ramp mask over the pair index between the correction dims, mask = (1 - clamp((p - low) /
    max(high - low, 0.001), 0, 1)) * ext_factor, and the frequency mixed as
    interp * (1 - mask) + extrap * mask with interp = freq_scale * extrap."""
    low, high = yarn_corr_dims_f64(n_dims, rp["n_ctx_orig"], rp["freq_base"], rp["beta_fast"], rp["beta_slow"])
    extrap = pos * rp["freq_base"] ** (-2.0 * p / n_dims)
    ramp = min(1.0, max(0.0, (p - low) / max(high - low, 0.001)))
    mask = (1.0 - ramp) * rp["ext_factor"]
    return rp["freq_scale"] * extrap * (1.0 - mask) + extrap * mask


def yarn_rows(gemv, d_lat, n_rope, pos, rp, pairs):
    """Expected roped rows (x0, x1) of the given pairs: rotated by the YaRN theta and scaled by the
    YaRN magnitude attn_factor * (1 + 0.1 ln(1 / freq_scale))."""
    ms = rp["attn_factor"] * (1.0 + 0.1 * math.log(1.0 / rp["freq_scale"]))
    x0 = gemv[d_lat + 2 * np.asarray(pairs)].astype(np.float64)
    x1 = gemv[d_lat + 2 * np.asarray(pairs) + 1].astype(np.float64)
    th = np.array([yarn_theta_f64(pos, p, n_rope, rp) for p in pairs])
    return (x0 * np.cos(th) - x1 * np.sin(th)) * ms, (x0 * np.sin(th) + x1 * np.cos(th)) * ms


def yarn_max_err(dst, gemv, d_lat, n_rope, pos, rp, pairs):
    r0, r1 = yarn_rows(gemv, d_lat, n_rope, pos, rp, pairs)
    idx = d_lat + 2 * np.asarray(pairs)
    return max(np.abs(dst[idx] - r0).max(), np.abs(dst[idx + 1] - r1).max())


@pytest.mark.parametrize("pos", [77, 5000])
def test_kvwrite_yarn_ramp(pos):
    """YaRN on (ext_factor 1, freq_scale 1/4) at pos > 0, where theta is not zero.  Closed forms at
    both ends of the ramp -- pairs p <= low keep the extrapolated theta pos * base^(-2p/n), pairs
    p >= high take freq_scale times it -- and every interior pair against the ramp of the YaRN
    reference implementation computed here in float64.  Planted mutants (correction dims swapped;
    the ramp's 1 - clamp(y) written as clamp(y)) must fail the same checks."""
    rng = np.random.default_rng(33)
    n_embd, d_lat, n_rope = 4096, 256, 64
    rp = RP_YARN
    w, cur, nw, kc, gemv = kv_inputs(rng, n_embd, d_lat, n_rope, 4)
    low, high = yarn_corr_dims_f64(n_rope, rp["n_ctx_orig"], rp["freq_base"], rp["beta_fast"], rp["beta_slow"])
    assert orc.rope_yarn_corr_dims(n_rope, rp["n_ctx_orig"], rp["freq_base"], rp["beta_fast"], rp["beta_slow"]) == (low, high)
    assert 0 < low < high < n_rope // 2 - 1          # both ramp ends and an interior fall inside the pairs
    lo_pairs = [p for p in range(n_rope // 2) if p <= low]
    hi_pairs = [p for p in range(n_rope // 2) if p >= high]
    mid_pairs = [p for p in range(n_rope // 2) if low < p < high]
    tol = 1e-6 + 4e-7 * pos * np.abs(gemv[d_lat:]).max()
    dst = orc.kvwrite(cur, w, d_lat, n_rope, nw, kc, 1, pos, rp)
    # the closed forms at the ends: theta_extrap / freq_scale * theta_extrap, no ramp involved
    ms = rp["attn_factor"] * (1.0 + 0.1 * math.log(1.0 / rp["freq_scale"]))
    for pairs, f in ((lo_pairs, 1.0), (hi_pairs, rp["freq_scale"])):
        p = np.asarray(pairs)
        th = f * pos * rp["freq_base"] ** (-2.0 * p / n_rope)
        x0, x1 = gemv[d_lat + 2 * p], gemv[d_lat + 2 * p + 1]
        assert np.abs(dst[d_lat + 2 * p] - (x0 * np.cos(th) - x1 * np.sin(th)) * ms).max() <= tol
        assert np.abs(dst[d_lat + 2 * p + 1] - (x0 * np.sin(th) + x1 * np.cos(th)) * ms).max() <= tol
    # the interior against the reference implementation's ramp
    assert yarn_max_err(dst, gemv, d_lat, n_rope, pos, rp, mid_pairs) <= tol
    # the mutants are caught
    for mutant in (3, 4):
        bad = orc.kvwrite(cur, w, d_lat, n_rope, nw, kc.copy(), 1, pos, rp, mutant=mutant)
        assert yarn_max_err(bad, gemv, d_lat, n_rope, pos, rp, list(range(n_rope // 2))) > 10 * tol, mutant


# ---------------------------------------------------------------- the 8-bit (Q8_0) latent cache
def q8_fields(wq, ne0):
    b = np.ascontiguousarray(wq).reshape(wq.shape[0], ne0 // 32, 34)
    d16 = b[:, :, :2].copy().view(np.float16).reshape(wq.shape[0], ne0 // 32)
    qs = b[:, :, 2:].copy().view(np.int8).astype(np.int64)
    return d16, qs


def q8_checks(x, wq):
    """Independent float64 checks of a Q8_0 quantisation of x: (stored scale is the f16 nearest to
    amax / 127, every q is the integer nearest to x / d away from the ties, the max element maps to
    +-127, zero blocks stay zero); returns a list of the failed checks."""
    ne0 = x.shape[1]
    d16, qs = q8_fields(wq, ne0)
    b = x.astype(np.float64).reshape(x.shape[0], ne0 // 32, 32)
    amax = np.abs(b).max(axis=2)
    d = amax / 127.0
    bad = []
    # the f16 nearest to d: within half an f16 ulp (ulp from the f16 exponent of d)
    ulp = np.where(d > 0, 2.0 ** (np.floor(np.log2(np.maximum(d, 2.0 ** -24))) - 10), 2.0 ** -24)
    if not (np.abs(d16.astype(np.float64) - d) <= 0.5 * ulp * (1 + 1e-9)).all():
        bad.append("scale")
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d[:, :, None] > 0, b / d[:, :, None], 0.0)
    away = np.sign(r) * np.floor(np.abs(r) + 0.5)
    clear = np.abs(np.abs(r - np.trunc(r)) - 0.5) > 1e-4          # not near a tie
    if not (qs[clear] == away[clear]).all():
        bad.append("nearest")
    if not (np.abs(qs).max(axis=2)[amax > 0] == 127).all() or (qs[amax == 0] != 0).any():
        bad.append("ends")
    return bad


def test_q8_0_quantiser_known_answers_and_mutants():
    """ggml's quantize_row_q8_0_ref (ggml-quants.c:276-299): d = amax / 127 stored as the nearest
    f16, q = roundf(x * (1 / d)), half away from zero.  A block with amax = 127 has d = 1, so its q
    are roundf(x) exactly: 62.5 -> 63, -62.5 -> -63, 0.5 -> 1, 2.5 -> 3."""
    x = np.zeros((2, 32), np.float32)
    x[0, :8] = [127, -127, 62.5, -62.5, 0.5, -0.5, 2.5, 1.4999999]
    wq = orc.q8_0_quantize(x)
    d16, qs = q8_fields(wq, 32)
    assert d16[0, 0] == 1.0 and d16[1, 0] == 0.0
    assert qs[0, 0, :8].tolist() == [127, -127, 63, -63, 1, -1, 3, 1]
    assert (qs[1] == 0).all()
    assert orc.q8_0_quantize(x, mutant=1).reshape(2, 34)[0, 2:10].view(np.int8).tolist() != qs[0, 0, :8].tolist()
    # random rows of both cache widths: every independent check holds, and each mutant fails one
    rng = np.random.default_rng(77)
    for ne0 in (576, 320):
        xr = (rng.standard_normal((64, ne0)) * rng.uniform(0.01, 3.0, (64, 1))).astype(np.float32)
        xr[3, 32:64] = 0.0                                          # a zero block
        assert q8_checks(xr, orc.q8_0_quantize(xr)) == []
        assert "nearest" in q8_checks(xr, orc.q8_0_quantize(xr, mutant=2))    # id from the f16 scale
        assert "scale" in q8_checks(xr, orc.q8_0_quantize(xr, mutant=3))      # scale off its nearest f16


def test_q8_0_round_trip_and_f16_dequantisation():
    """|x - q d16| <= d16 / 2 + 127 |d16 - d| per element; the f16 cache values of the Q8_0 kernel
    are f16(q * d16) with the product exact (computed here in float64)."""
    rng = np.random.default_rng(78)
    x = (rng.standard_normal((100, 576)) * 0.7).astype(np.float32)
    wq = orc.q8_0_quantize(x)
    d16, qs = q8_fields(wq, 576)
    d = np.abs(x.astype(np.float64)).reshape(100, 18, 32).max(axis=2) / 127.0
    deq = orc.q8_0_dequant(wq, 576).astype(np.float64).reshape(100, 18, 32)
    bound = d16.astype(np.float64) / 2 + 127 * np.abs(d16.astype(np.float64) - d) + 1e-12
    assert (np.abs(x.astype(np.float64).reshape(100, 18, 32) - deq) <= bound[:, :, None]).all()
    exact = (qs.astype(np.float64) * d16.astype(np.float64)[:, :, None]).reshape(100, 576)
    assert np.array_equal(orc.q8_0_dequant_f16(wq, 576), exact.astype(np.float16))
    assert np.array_equal(orc.q8_0_dequant(wq, 576).astype(np.float64), exact)


def test_synthetic_q8_cache_matches_the_oracle_quantiser():
    """aubier_amd.inputs builds the benchmark's Q8_0 caches with its own copy of the quantiser: it
    must produce the oracle's bytes, and with_q8_cache's f16 values must be the oracle's f16(q d)."""
    from aubier_amd import inputs as I
    rng = np.random.default_rng(79)
    x = (rng.standard_normal((300, 576)) * rng.uniform(0.001, 2.0, (300, 1))).astype(np.float32)
    x[7, :64] = 0.0
    x[8, 5] = 62.5 * (np.abs(x[8, :32]).max() / 127.0)       # a value near a rounding tie
    assert np.array_equal(I.q8_0_rows(x), orc.q8_0_quantize(x))
    inp = I.with_q8_cache(I.make_config(2, n_kv=300))
    assert np.array_equal(inp.kcache_q8, orc.q8_0_quantize(I.make_config(2, n_kv=300).kcache.astype(np.float32)))
    assert np.array_equal(inp.kcache, orc.q8_0_dequant_f16(inp.kcache_q8, 576))

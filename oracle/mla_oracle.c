/*
 * mla_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of the reference's *unfused* ggml CPU graph for the MLA attention path, used
 * as the numerics oracle for the HIP kernels in aubier_amd/.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the checker or as the timed
 * CPU baseline -- never as the product path.
 *
 * What it restates (reference = /root/reference, vendored ggml under vendor/llama.cpp/ggml/src):
 *   - the op sequence of engine/m1_layer.cpp:444-446 (WKB: mul_mat(W_kb, permute(q_nope))) and
 *     engine/m1_layer.cpp:477-495 (kq = mul_mat(K_view, permute(Qcur)); soft_max_ext(kq, mask,
 *     kq_scale, 0); kqv = mul_mat(cont(transpose(V_view)), kq));
 *   - ggml-cpu mul_mat (ggml-cpu/ggml-cpu.c:1259-1420): src1 is converted to the vec_dot_type of
 *     src0 (ggml-cpu.c:216-227, 1328-1378).  For an F16 src0 that is F16, so q and the softmax
 *     probabilities P are rounded to f16 (round-to-nearest-even) before the dot; for F32 src0
 *     nothing is converted.  Dots are accumulated in f32 over 16 interleaved lanes, the shape of
 *     ggml's SIMD/tinyBLAS f32 accumulation (llamafile/sgemm.cpp, vec.cpp:264-313).
 *   - ggml soft_max_f32 (ggml-cpu/ops.cpp:5813-5923, vec.cpp:531-600): wp = kq*scale (f32), then
 *     wp += mask (f32); max; y = expf(wp - max) in f32 with the sum in double (ggml_float);
 *     then y *= (float)(1.0/sum).
 *   - the split-K combine of patches/ggml-m4/m4-kqkv.cu:314-338 (LSE merge; splits with m = -inf
 *     are skipped; an all-masked row gives 0).
 * Plus a double-precision brute force of softmax attention (no f16 rounding of q or P) and the
 * seeded input generator (splitmix64 + Box-Muller).
 *
 * Every function is checked by tests/test_oracle.py against: numpy/torch float64 library routines,
 * closed forms (identity W_kb, one dominant key, uniform scores, W = 1), invariants (key
 * permutation, masked-tail sentinel, split/merge), and planted mutants that must fail.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

/* ------------------------------------------------------------------ generator */

static inline uint64_t splitmix64_next(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0, 1]: 53 random bits, never 0 (log(0) would be -inf in Box-Muller) */
static inline double u01_open0(uint64_t *s) {
    return ((double)(splitmix64_next(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

/* N(0,1)*scale, n values, Box-Muller in double, rounded once to f32.  Value i depends only on
 * (seed, i): pair p = i/2 draws two uniforms from the stream started at seed + p*2*golden, so any
 * slice can be regenerated independently (and in parallel). */
void orc_randn(uint64_t seed, int64_t n, float scale, float *out) {
    const double two_pi = 6.283185307179586476925286766559;
    const int64_t npairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < npairs; ++p) {
        uint64_t s = seed ^ (0xD1B54A32D192ED03ull * (uint64_t)(p + 1));
        const double u1 = u01_open0(&s);
        const double u2 = u01_open0(&s);
        const double r = sqrt(-2.0 * log(u1));
        const double z0 = r * cos(two_pi * u2);
        const double z1 = r * sin(two_pi * u2);
        out[2 * p] = (float)(z0 * (double)scale);
        if (2 * p + 1 < n) out[2 * p + 1] = (float)(z1 * (double)scale);
    }
}

/* ------------------------------------------------------------------ f16 */

/* f32 -> IEEE binary16, round to nearest even, with subnormals, overflow to inf, NaN kept.
 * This is what ggml's from_float for F16 does on x86 (F16C _mm_cvtps_ph, rounding mode 0). */
static inline uint16_t f32_to_f16_rne(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) {                       /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u | ((absx >> 13) & 0x3ffu) : 0u));
    }
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 rounds to inf */
    if (absx < 0x38800000u) {                        /* result is subnormal or zero (< 2^-14) */
        /* value = absx as float; f16 subnormal unit = 2^-24.  q = round_even(value / 2^-24) */
        if (absx < 0x33000000u) return (uint16_t)sign;            /* < 2^-25: rounds to 0 (2^-25 ties to even 0) */
        const uint32_t e = absx >> 23;               /* biased exponent, 102..112 */
        const uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;             /* value/2^-24 = m * 2^(e-127-23+24) = m >> (126-e) */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    /* normal range */
    uint32_t e16 = ((absx >> 23) - 127u + 15u);
    uint32_t m = absx & 0x7fffffu;
    uint32_t q = (e16 << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;   /* carry may bump the exponent: correct */
    return (uint16_t)(sign | q);
}

static inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) { x = sign; }
        else {                                        /* subnormal: m * 2^-24 exactly */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float r; memcpy(&r, &x, 4);
    return r;
}

void orc_f32_to_f16(const float *in, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16_rne(in[i]);
}

void orc_f16_to_f32(const uint16_t *in, float *out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------ tensor views
 * A minimal view with ggml's conventions: ne[] elements per axis (fastest first), nb[] byte
 * strides, type 0 = F32, 1 = F16 (ggml_type numbering). */

typedef struct {
    void   *data;
    int32_t type;
    int64_t ne[4];
    int64_t nb[4];
} orc_tensor;

enum { ORC_F32 = 0, ORC_F16 = 1 };

static inline float tget(const orc_tensor *t, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    const char *p = (const char *)t->data + i0 * t->nb[0] + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
    return t->type == ORC_F16 ? f16_to_f32(*(const uint16_t *)p) : *(const float *)p;
}

/* f32 dot with 16 interleaved accumulators, folded pairwise (the SIMD accumulation shape) */
static inline float dot_f32_lanes(const float *a, const float *b, int64_t n) {
    float acc[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; ++j) acc[j] += a[i + j] * b[i + j];
    for (int j = 0; i < n; ++i, ++j) acc[j] += a[i] * b[i];
    for (int w = 8; w > 0; w >>= 1)
        for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
    return acc[0];
}

/*
 * ggml mul_mat: dst[i0, i1, i2, i3] = sum_k src0[k, i0, i2/r2, i3/r3] * conv(src1[k, i1, i2, i3]),
 * dst ne = [ne01, ne11, ne12, ne13] contiguous f32.  conv() rounds src1 to f16 when src0 is F16
 * (vec_dot_type), identity for F32.  src0 rows are read through nb (any strides); the caller's
 * "mutant" hook is a test-only switch that plants a mistake (0 = none).
 */
static void orc_mul_mat(const orc_tensor *src0, const orc_tensor *src1, float *dst, int nthreads, int mutant) {
    const int64_t K = src0->ne[0];
    const int64_t ne01 = src0->ne[1], ne02 = src0->ne[2], ne03 = src0->ne[3];
    const int64_t ne11 = src1->ne[1], ne12 = src1->ne[2], ne13 = src1->ne[3];
    const int64_t r2 = ne12 / ne02, r3 = ne13 / ne03;
    const int round16 = (src0->type == ORC_F16) && mutant != 2;

    /* widen src0 to f32 once (exact), per (i2, i3) plane */
    const int64_t planes0 = ne02 * ne03;
    float *a = (float *)malloc(sizeof(float) * (size_t)(K * ne01 * planes0));
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t r = 0; r < ne01 * planes0; ++r) {
        const int64_t i1 = r % ne01, p = r / ne01;
        const int64_t i2 = p % ne02, i3 = p / ne02;
        for (int64_t k = 0; k < K; ++k) a[r * K + k] = tget(src0, k, i1, i2, i3);
    }
    /* convert src1 rows (vec_dot_type) */
    const int64_t rows1 = ne11 * ne12 * ne13;
    float *b = (float *)malloc(sizeof(float) * (size_t)(K * rows1));
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t r = 0; r < rows1; ++r) {
        const int64_t i1 = r % ne11, p = r / ne11;
        const int64_t i2 = p % ne12, i3 = p / ne12;
        for (int64_t k = 0; k < K; ++k) {
            float v = tget(src1, k, i1, i2, i3);
            if (round16) v = f16_to_f32(f32_to_f16_rne(v));
            b[r * K + k] = v;
        }
    }
    /* dst rows: (i1, i2, i3) -> ne01 outputs; blocked over src0 rows for cache reuse */
    const int64_t BLK = 64;
    const int64_t nblk = (ne01 + BLK - 1) / BLK;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1) collapse(2)
    for (int64_t r = 0; r < rows1; ++r) {
        for (int64_t bi = 0; bi < nblk; ++bi) {
            const int64_t p = r / ne11;
            const int64_t i2 = p % ne12, i3 = p / ne12;
            const int64_t plane0 = (i2 / r2) + (i3 / r3) * ne02;
            const float *brow = b + r * K;
            float *drow = dst + r * ne01;
            const int64_t i0e = (bi + 1) * BLK < ne01 ? (bi + 1) * BLK : ne01;
            for (int64_t i0 = bi * BLK; i0 < i0e; ++i0)
                drow[i0] = dot_f32_lanes(a + (plane0 * ne01 + i0) * K, brow, K);
        }
    }
    free(a);
    free(b);
}

/*
 * ggml soft_max_ext(kq, mask, scale, max_bias = 0), in place on a contiguous f32
 * [ne0 = n_kv, ne1 = rows, ne2 = heads] tensor; mask is f32 [n_kv, >= rows] with row stride
 * mask_nb1 bytes, broadcast across heads (mask row = i1).  mask may be NULL.
 */
static void orc_soft_max_ext(float *kq, int64_t n_kv, int64_t rows, int64_t heads,
                             const float *mask, int64_t mask_nb1, float scale, int nthreads, int mutant) {
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
    for (int64_t h = 0; h < heads; ++h) {
        for (int64_t r = 0; r < rows; ++r) {
            float *wp = kq + (h * rows + r) * n_kv;
            const float *mp = mask ? (const float *)((const char *)mask + r * mask_nb1) : NULL;
            for (int64_t i = 0; i < n_kv; ++i) {
                float v = wp[i];
                if (mutant != 1) v *= scale;          /* ggml_vec_scale_f32 */
                if (mp) v += mp[i];                   /* slope = 1 (max_bias = 0) */
                wp[i] = v;
            }
            float mx = -INFINITY;
            for (int64_t i = 0; i < n_kv; ++i) mx = wp[i] > mx ? wp[i] : mx;
            double sum = 0.0;                          /* ggml_float */
            for (int64_t i = 0; i < n_kv; ++i) {
                const float e = expf(wp[i] - mx);
                sum += (double)e;
                wp[i] = e;
            }
            const float inv = (float)(1.0 / sum);
            for (int64_t i = 0; i < n_kv; ++i) wp[i] *= inv;
        }
    }
}

/*
 * The unfused KQKV graph (engine/m1_layer.cpp:477-495) on CPU.
 *   kcache: type F32/F16, ne [D_k, n_kv], row stride kc_nb1 bytes (K = all D_k cols, V = first D_v)
 *   q:      f32 ne [D_k, H, nt], byte strides q_nb1 (head), q_nb2 (token)
 *   mask:   f32 ne [n_kv, >= nt], row stride mask_nb1 bytes (0 / -inf), or NULL
 *   out:    f32 ne [D_v, nt, H] contiguous
 * mutant: 0 none, 1 drop kq_scale, 2 skip the f16 rounding of q and P, 3 read V from the rope end
 * of the row (columns [D_k-D_v, D_k)), 4 broadcast the mask of token 0 to every token.
 */
int orc_kqkv(const void *kcache, int32_t kc_type, int64_t d_k, int64_t n_kv, int64_t kc_nb1,
             const float *q, int64_t n_head, int64_t nt, int64_t q_nb1, int64_t q_nb2,
             const float *mask, int64_t mask_nb1, float kq_scale, int64_t d_v,
             float *out, int nthreads, int mutant) {
    if (d_v > d_k || n_kv < 1 || nt < 1 || n_head < 1) return -1;
    const int64_t esz = kc_type == ORC_F16 ? 2 : 4;
    /* kp = permute(view(kcache)) : ne [D_k, n_kv, 1, 1] */
    orc_tensor kp = { (void *)kcache, kc_type, { d_k, n_kv, 1, 1 }, { esz, kc_nb1, kc_nb1 * n_kv, kc_nb1 * n_kv } };
    /* qp = permute(q4, 0, 2, 1, 3) : ne [D_k, nt, H, 1] */
    orc_tensor qp = { (void *)q, ORC_F32, { d_k, nt, n_head, 1 }, { 4, q_nb2, q_nb1, q_nb2 * nt } };
    float *kq = (float *)malloc(sizeof(float) * (size_t)(n_kv * nt * n_head));
    orc_mul_mat(&kp, &qp, kq, nthreads, mutant);                 /* [n_kv, nt, H] */
    const float *mk = mask;
    int64_t mnb1 = mask_nb1;
    if (mutant == 4) mnb1 = 0;
    orc_soft_max_ext(kq, n_kv, nt, n_head, mk, mnb1, kq_scale, nthreads, mutant);

    /* vT = cont(transpose(permute(V view))) : ne [n_kv, D_v], same type as the cache */
    const int64_t voff = (mutant == 3) ? (d_k - d_v) : 0;
    void *vt = malloc((size_t)(esz * n_kv * d_v));
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t c = 0; c < d_v; ++c) {
        for (int64_t j = 0; j < n_kv; ++j) {
            const char *src = (const char *)kcache + j * kc_nb1 + (c + voff) * esz;
            if (esz == 2) ((uint16_t *)vt)[c * n_kv + j] = *(const uint16_t *)src;
            else ((float *)vt)[c * n_kv + j] = *(const float *)src;
        }
    }
    orc_tensor vtt = { vt, kc_type, { n_kv, d_v, 1, 1 }, { esz, esz * n_kv, esz * n_kv * d_v, esz * n_kv * d_v } };
    /* kqv = mul_mat(vT, kq) : src1 = kq ne [n_kv, nt, H] */
    orc_tensor kqt = { kq, ORC_F32, { n_kv, nt, n_head, 1 }, { 4, 4 * n_kv, 4 * n_kv * nt, 4 * n_kv * nt * n_head } };
    orc_mul_mat(&vtt, &kqt, out, nthreads, mutant);              /* [D_v, nt, H] */
    free(vt);
    free(kq);
    return 0;
}

/*
 * The unfused WKB (engine/m1_layer.cpp:444-446): q_nope_abs = permute(mul_mat(W_kb, permute(q_nope))).
 *   w:      f32 ne [d_n, D_v, H] contiguous (W[h][c][d])
 *   q_nope: f32 ne [d_n, H, nt] with byte strides q_nb1 (head), q_nb2 (token)
 *   out:    f32 ne [D_v, H, nt] with byte strides o_nb1 (head), o_nb2 (token)
 * F32 src0 -> vec_dot_type F32: no rounding.  mutant 5 transposes the W block (reads W[h][d][c]).
 */
int orc_wkb(const float *w, int64_t d_n, int64_t d_v, int64_t n_head,
            const float *q_nope, int64_t nt, int64_t q_nb1, int64_t q_nb2,
            float *out, int64_t o_nb1, int64_t o_nb2, int nthreads, int mutant) {
    if (mutant == 5 && d_n != d_v) return -1;
    orc_tensor wt = { (void *)w, ORC_F32, { d_n, d_v, n_head, 1 }, { 4, 4 * d_n, 4 * d_n * d_v, 4 * d_n * d_v * n_head } };
    if (mutant == 5) { wt.nb[0] = 4 * d_n; wt.nb[1] = 4; }
    /* permute(q_nope, 0, 2, 1, 3): ne [d_n, nt, H] */
    orc_tensor qp = { (void *)q_nope, ORC_F32, { d_n, nt, n_head, 1 }, { 4, q_nb2, q_nb1, q_nb2 * nt } };
    float *tmp = (float *)malloc(sizeof(float) * (size_t)(d_v * nt * n_head));
    orc_mul_mat(&wt, &qp, tmp, nthreads, 0);                      /* [D_v, nt, H] */
    for (int64_t h = 0; h < n_head; ++h)
        for (int64_t t = 0; t < nt; ++t)
            memcpy((char *)out + h * o_nb1 + t * o_nb2, tmp + (h * nt + t) * d_v, sizeof(float) * (size_t)d_v);
    free(tmp);
    return 0;
}

/*
 * Double-precision brute force of masked softmax attention (no f16 rounding anywhere; the cache
 * values are read exactly).  Same tensor conventions as orc_kqkv.  A row whose keys are all
 * masked gives 0 (the convention of the split-K combine).
 */
int orc_attn_f64(const void *kcache, int32_t kc_type, int64_t d_k, int64_t n_kv, int64_t kc_nb1,
                 const float *q, int64_t n_head, int64_t nt, int64_t q_nb1, int64_t q_nb2,
                 const float *mask, int64_t mask_nb1, float kq_scale, int64_t d_v,
                 double *out, int nthreads) {
    const int64_t esz = kc_type == ORC_F16 ? 2 : 4;
#pragma omp parallel num_threads(nthreads)
    {
        double *s = (double *)malloc(sizeof(double) * (size_t)n_kv);
        double *kr = (double *)malloc(sizeof(double) * (size_t)d_k);
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int64_t h = 0; h < n_head; ++h) {
            for (int64_t t = 0; t < nt; ++t) {
                const float *qh = (const float *)((const char *)q + h * q_nb1 + t * q_nb2);
                const float *mp = mask ? (const float *)((const char *)mask + t * mask_nb1) : NULL;
                double mx = -INFINITY;
                for (int64_t j = 0; j < n_kv; ++j) {
                    const char *row = (const char *)kcache + j * kc_nb1;
                    double acc = 0.0;
                    for (int64_t k = 0; k < d_k; ++k) {
                        const double kv = esz == 2 ? (double)f16_to_f32(((const uint16_t *)row)[k]) : (double)((const float *)row)[k];
                        acc += kv * (double)qh[k];
                    }
                    double v = acc * (double)kq_scale + (mp ? (double)mp[j] : 0.0);
                    s[j] = v;
                    if (v > mx) mx = v;
                }
                double *o = out + (h * nt + t) * d_v;
                for (int64_t c = 0; c < d_v; ++c) o[c] = 0.0;
                if (mx == -INFINITY) continue;
                double sum = 0.0;
                for (int64_t j = 0; j < n_kv; ++j) {
                    const double e = s[j] == -INFINITY ? 0.0 : exp(s[j] - mx);
                    s[j] = e;
                    sum += e;
                }
                for (int64_t j = 0; j < n_kv; ++j) {
                    if (s[j] == 0.0) continue;
                    const char *row = (const char *)kcache + j * kc_nb1;
                    const double p = s[j] / sum;
                    for (int64_t c = 0; c < d_v; ++c) {
                        const double vv = esz == 2 ? (double)f16_to_f32(((const uint16_t *)row)[c]) : (double)((const float *)row)[c];
                        o[c] += p * vv;
                    }
                }
            }
        }
        free(s);
        free(kr);
    }
    return 0;
}

/*
 * Split-K partials in double, the pass-1 contract of patches/ggml-m4/m4-kqkv.cu:201-312 with an
 * explicit key range per split: split s covers keys [bounds[s], bounds[s+1]).  Record layout
 * (our partial format): rec[0] = m (natural-log units), rec[1] = l, rec[2..3] = 0, rec[4..4+D_v)
 * = o (unnormalised: sum_j exp(s_j - m) * V_j).  part is f32 [(4 + D_v), n_split, nt, H].
 */
int orc_partials(const void *kcache, int32_t kc_type, int64_t d_k, int64_t n_kv, int64_t kc_nb1,
                 const float *q, int64_t n_head, int64_t nt, int64_t q_nb1, int64_t q_nb2,
                 const float *mask, int64_t mask_nb1, float kq_scale, int64_t d_v,
                 const int64_t *bounds, int64_t n_split, float *part) {
    const int64_t esz = kc_type == ORC_F16 ? 2 : 4;
    const int64_t rs = 4 + d_v;
    (void)n_kv;
#pragma omp parallel for schedule(dynamic, 1) collapse(3)
    for (int64_t h = 0; h < n_head; ++h) {
        for (int64_t t = 0; t < nt; ++t) {
            for (int64_t sp = 0; sp < n_split; ++sp) {
                const float *qh = (const float *)((const char *)q + h * q_nb1 + t * q_nb2);
                const float *mp = mask ? (const float *)((const char *)mask + t * mask_nb1) : NULL;
                float *rec = part + ((h * nt + t) * n_split + sp) * rs;
                double mx = -INFINITY;
                const int64_t j0 = bounds[sp], j1 = bounds[sp + 1];
                double *s = (double *)malloc(sizeof(double) * (size_t)(j1 > j0 ? j1 - j0 : 1));
                for (int64_t j = j0; j < j1; ++j) {
                    const char *row = (const char *)kcache + j * kc_nb1;
                    double acc = 0.0;
                    for (int64_t k = 0; k < d_k; ++k) {
                        const double kv = esz == 2 ? (double)f16_to_f32(((const uint16_t *)row)[k]) : (double)((const float *)row)[k];
                        acc += kv * (double)qh[k];
                    }
                    s[j - j0] = acc * (double)kq_scale + (mp ? (double)mp[j] : 0.0);
                    if (s[j - j0] > mx) mx = s[j - j0];
                }
                double l = 0.0;
                double *o = (double *)calloc((size_t)d_v, sizeof(double));
                if (mx > -INFINITY) {
                    for (int64_t j = j0; j < j1; ++j) {
                        if (s[j - j0] == -INFINITY) continue;
                        const double e = exp(s[j - j0] - mx);
                        l += e;
                        const char *row = (const char *)kcache + j * kc_nb1;
                        for (int64_t c = 0; c < d_v; ++c) {
                            const double vv = esz == 2 ? (double)f16_to_f32(((const uint16_t *)row)[c]) : (double)((const float *)row)[c];
                            o[c] += e * vv;
                        }
                    }
                }
                rec[0] = (float)mx;
                rec[1] = (float)l;
                rec[2] = 0.0f;
                rec[3] = 0.0f;
                for (int64_t c = 0; c < d_v; ++c) rec[4 + c] = (float)o[c];
                free(o);
                free(s);
            }
        }
    }
    return 0;
}

/*
 * The split-K merge (patches/ggml-m4/m4-kqkv.cu:314-338): m* = max m_s; l* = sum l_s e^(m_s-m*);
 * o* = sum o_s e^(m_s-m*) over splits with m_s > -inf; out = o* / l*, or 0 when every split is
 * empty.  part f32 [(4 + D_v), n_split, nt, H] (records as in orc_partials); out f32 [D_v, nt, H].
 * Done in double.  mutant 6 forgets to rescale l (uses sum l_s).
 */
int orc_merge(const float *part, int64_t d_v, int64_t n_split, int64_t nt, int64_t n_head,
              float *out, int mutant) {
    const int64_t rs = 4 + d_v;
    for (int64_t h = 0; h < n_head; ++h) {
        for (int64_t t = 0; t < nt; ++t) {
            const float *p = part + (h * nt + t) * n_split * rs;
            float *o = out + (h * nt + t) * d_v;
            double ms = -INFINITY;
            for (int64_t s = 0; s < n_split; ++s) if ((double)p[s * rs] > ms) ms = (double)p[s * rs];
            if (ms == -INFINITY) { for (int64_t c = 0; c < d_v; ++c) o[c] = 0.0f; continue; }
            double l = 0.0;
            for (int64_t s = 0; s < n_split; ++s) {
                const double m = (double)p[s * rs];
                if (m == -INFINITY) continue;
                l += (double)p[s * rs + 1] * (mutant == 6 ? 1.0 : exp(m - ms));
            }
            for (int64_t c = 0; c < d_v; ++c) {
                double acc = 0.0;
                for (int64_t s = 0; s < n_split; ++s) {
                    const double m = (double)p[s * rs];
                    if (m == -INFINITY) continue;
                    acc += (double)p[s * rs + 4 + c] * exp(m - ms);
                }
                o[c] = (float)(acc / l);
            }
        }
    }
    return 0;
}

/* The known-answer input pattern of the reference's standalone KQKV bench
 * (engine/m1_kqkv_bench.hip:148-165): K[i] = ((i*7919) % 1000)/1000 - 0.5 stored with a
 * round-toward-zero f16 conversion that flushes |v| < 2^-14 to signed zero; q[i] =
 * ((i*3571) % 1000)/1000 - 0.5 in f32. */
void orc_kqkv_bench_pattern(int64_t n_k, uint16_t *kc, int64_t n_q, float *q) {
    for (int64_t i = 0; i < n_k; ++i) {
        const float v = (float)((i * 7919) % 1000) / 1000.0f - 0.5f;
        uint32_t f; memcpy(&f, &v, 4);
        const uint32_t sign = (f >> 16) & 0x8000u;
        const int32_t e = (int32_t)((f >> 23) & 0xffu) - 127 + 15;
        uint16_t h;
        if (e >= 31) h = (uint16_t)(sign | 0x7c00u);
        else if (e <= 0) h = (uint16_t)sign;
        else h = (uint16_t)(sign | ((uint32_t)e << 10) | ((f >> 13) & 0x3ffu));
        kc[i] = h;
    }
    for (int64_t i = 0; i < n_q; ++i) q[i] = (float)((i * 3571) % 1000) / 1000.0f - 0.5f;
}

int orc_max_threads(void) { return omp_get_max_threads(); }

/* ------------------------------------------------------------------ Q8_0 x Q8_1 paths
 * The reference geometry's quantised ops follow the GPU MMVQ numerics (not ggml-cpu's Q8_0.Q8_0
 * mul_mat): the f32 activation is quantised per 32-value block to int8 with an f16 scale, the
 * block dot is an exact int32 sum, and the f32 result accumulates wd * d16 * sum.  The
 * restatements below keep the reference kernels' operation order: the floating steps are written
 * with explicit fmaf/fmaxf so the C compiler cannot contract or reassociate them (nvcc contracts
 * `acc += wd * d16 * (float)sum` into fma(wd * d16, sum, acc); wd * d16 is exact in f32, both
 * being f16 values).
 *
 * Q8_0 block (ggml block_q8_0): f16 d, then 32 int8 qs -- 34 bytes, rows of ne0 / 32 blocks. */

static inline float q8_scale(const uint8_t *blk) { uint16_t h; memcpy(&h, blk, 2); return f16_to_f32(h); }

/* Activation block quantisation, the WKB form (patches/ggml-m4/m4-wkb.cu:36-47):
 * d = amax / 127, d16 = f16(d), q = roundf(x / d) (0 when amax == 0). */
static void quant_block_div(const float *x, int8_t *q, float *d16) {
    float amax = 0.0f;
    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(x[k]));
    const float d = amax / 127.0f;
    *d16 = f16_to_f32(f32_to_f16_rne(d));
    for (int k = 0; k < 32; ++k) q[k] = (int8_t)(amax == 0.0f ? 0 : (int)roundf(x[k] / d));
}

/* The PHASE form (patches/ggml-m4/m4-phase.cu:58-66, 106-111, quantize_q8_1's): id = d ? 1/d : 0,
 * q = roundf(x * id). */
static void quant_block_mul(const float *x, int8_t *q, float *d16) {
    float amax = 0.0f;
    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(x[k]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    *d16 = f16_to_f32(f32_to_f16_rne(d));
    for (int k = 0; k < 32; ++k) q[k] = (int8_t)(int)roundf(x[k] * id);
}

static inline int32_t dot_q8(const int8_t *a, const int8_t *b) {
    int32_t s = 0;
    for (int k = 0; k < 32; ++k) s += (int32_t)a[k] * (int32_t)b[k];
    return s;
}

/* The 32-lane butterfly of ggml-cuda's warp_reduce_sum (xor 16, 8, 4, 2, 1), value of lane 0. */
static float warp32_sum(const float *v_in) {
    float v[32], t[32];
    memcpy(v, v_in, sizeof v);
    for (int off = 16; off > 0; off >>= 1) {
        for (int k = 0; k < 32; ++k) t[k] = v[k] + v[k ^ off];
        memcpy(v, t, sizeof v);
    }
    return v[0];
}

/* GGML_OP_M4_WKB with a Q8_0 W_kb (patches/ggml-m4/m4-wkb.cu:21-69), generalised to d_n = 32 nb
 * and nt tokens: out[t][h][c] = sum_b fma(wd_b * xd_b, sum_b, .) over the row's blocks in order.
 * w: [n_head][d_v] rows of d_n / 32 blocks; q: f32, element (t, h, d) at q + t q_nb2 + h q_nb1
 * (bytes) + 4 d; out: element (t, h, c) at out + t d_nb2 + h d_nb1 + 4 c. */
int orc_wkb_q8(const uint8_t *w, int64_t d_n, int64_t d_v, int64_t n_head, const float *q, int64_t nt,
               int64_t q_nb1, int64_t q_nb2, float *out, int64_t d_nb1, int64_t d_nb2, int mutant) {
    if (d_n % 32 != 0 || d_n > 1024) return -1;
    const int64_t nb = d_n / 32;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < nt; ++t)
        for (int64_t h = 0; h < n_head; ++h) {
            int8_t xq[1024];
            float xd[32];
            const float *x = (const float *)((const char *)q + t * q_nb2 + h * q_nb1);
            for (int64_t b = 0; b < nb; ++b) {
                if (mutant == 1) quant_block_mul(x + 32 * b, xq + 32 * b, &xd[b]);   /* wrong form */
                else quant_block_div(x + 32 * b, xq + 32 * b, &xd[b]);
            }
            float *o = (float *)((char *)out + t * d_nb2 + h * d_nb1);
            for (int64_t c = 0; c < d_v; ++c) {
                const uint8_t *row = w + (h * d_v + c) * nb * 34;
                float acc = 0.0f;
                for (int64_t b = 0; b < nb; ++b) {
                    const uint8_t *blk = row + (mutant == 2 ? 34 * ((b + 1) % nb) : 34 * b);   /* block mix-up */
                    const int32_t s = dot_q8((const int8_t *)(blk + 2), xq + 32 * b);
                    acc = fmaf(q8_scale(blk) * xd[b], (float)s, acc);
                }
                o[c] = acc;
            }
        }
    return 0;
}

/* GGML_OP_M4_PHASE phase 1, wv_b (patches/ggml-m4/m4-phase.cu:52-88), generalised to d_in = 32 nb
 * inputs per head and nt tokens: per (token, head, output) the 32 lanes' partials
 * p_k = sum_b fma(wd_b * xd_b, q_w[b][k] * q_x[b][k], .) (blocks in order), then the butterfly.
 * w: [n_head][d_out] rows of d_in / 32 blocks; x: (t, h, i) at x + t x_nb2 + h x_nb1 + 4 i;
 * out: (t, h, o) at out + t o_nb2 + h o_nb1 + 4 o. */
int orc_wvb_q8(const uint8_t *w, int64_t d_in, int64_t d_out, int64_t n_head, const float *x, int64_t nt,
               int64_t x_nb1, int64_t x_nb2, float *out, int64_t o_nb1, int64_t o_nb2, int mutant) {
    if (d_in % 32 != 0 || d_in > 1024) return -1;
    const int64_t nb = d_in / 32;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < nt; ++t)
        for (int64_t h = 0; h < n_head; ++h) {
            int8_t xq[1024];
            float xd[32];
            const float *xh = (const float *)((const char *)x + t * x_nb2 + h * x_nb1);
            for (int64_t b = 0; b < nb; ++b) {
                if (mutant == 1) quant_block_div(xh + 32 * b, xq + 32 * b, &xd[b]);   /* wrong form */
                else quant_block_mul(xh + 32 * b, xq + 32 * b, &xd[b]);
            }
            float *o = (float *)((char *)out + t * o_nb2 + h * o_nb1);
            for (int64_t r = 0; r < d_out; ++r) {
                const uint8_t *row = w + (h * d_out + r) * nb * 34;
                float p[32];
                for (int k = 0; k < 32; ++k) {
                    float acc = 0.0f;
                    for (int64_t b = 0; b < nb; ++b) {
                        const uint8_t *blk = row + 34 * b;
                        const int32_t qq = (int32_t)((const int8_t *)(blk + 2))[k] * (int32_t)xq[32 * b + k];
                        acc = fmaf(q8_scale(blk) * xd[b], (float)qq, acc);
                    }
                    p[k] = acc;
                }
                float s = 0.0f;
                if (mutant == 2) { for (int k = 0; k < 32; ++k) s += p[k]; }   /* serial, not the butterfly */
                else s = warp32_sum(p);
                o[r] = s;
            }
        }
    return 0;
}

/* YaRN correction dims (vendor/llama.cpp/ggml/src/ggml.c:4632-4643). */
void orc_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow, float dims[2]) {
    const float pi = 3.14159265358979323846f;
    const float cf = (float)n_dims * logf((float)n_ctx_orig / (beta_fast * 2.0f * pi)) / (2.0f * logf(freq_base));
    const float cs = (float)n_dims * logf((float)n_ctx_orig / (beta_slow * 2.0f * pi)) / (2.0f * logf(freq_base));
    const float start = floorf(cf), end = ceilf(cs);
    dims[0] = start > 0.0f ? start : 0.0f;
    dims[1] = end < (float)(n_dims - 1) ? end : (float)(n_dims - 1);
}

/* GGML_OP_M4_PHASE phase 0, KV-write (patches/ggml-m4/m4-phase.cu:95-200), generalised to
 * n_embd = 1024 nw inputs and d_lat + n_rope outputs (reference: 4096 -> 256 + 64):
 *  1. gemv: out[o] = per 32-block b: wd d16 sum (plain products, d16 and q from the PHASE form of
 *     the block quantisation); the blocks of a warp (32 consecutive) reduced by the butterfly,
 *     then the warp partials summed in order;
 *  2. rms norm of rows [0, d_lat): squares reduced per 32 rows by the butterfly, the partials of
 *     all (d_lat + n_rope) / 32 warps summed in order, scale = 1 / sqrt(s / d_lat + eps),
 *     kcur = scale * v * nw;
 *  3. rope of rows [d_lat, d_lat + n_rope), pairs p: theta_e = pos * theta_scale^p, theta =
 *     freq_scale theta_e mixed with theta_e by the YaRN ramp when ext_factor != 0, mscale =
 *     attn_factor (1 + 0.1 ln(1 / freq_scale)) then, (x0, x1) rotated by theta and scaled;
 *  4. the row as f16 into kcache row kidx (round to nearest even); dst = kcur (f32).
 * The CUDA math of steps 2-3 (rsqrtf, powf, cosf, sinf, logf) is restated with the C library's
 * f32 functions: the GPU result differs by its own math library's ulps, which grow with pos
 * for the rope (documented in the test tolerances).
 * mutant (tests only): 1 sign slip in the rotation, 2 the wrong cache row, 3 the YaRN correction
 * dims swapped, 4 the YaRN ramp written as clamp(y) instead of 1 - clamp(y). */
int orc_kvwrite(const float *cur, int64_t n_embd, const uint8_t *w, int64_t d_lat, int64_t n_rope, const float *nw,
                uint16_t *kcache, int64_t kc_nb1, int64_t kidx, int32_t pos,
                float freq_base, float freq_scale, float ext_factor, float attn_factor, float beta_fast,
                float beta_slow, float eps, int32_t n_ctx_orig, float *dst, int mutant) {
    const int64_t n_out = d_lat + n_rope;
    const int64_t nb = n_embd / 32;
    if (n_embd % 1024 != 0 || n_out % 32 != 0 || d_lat % 32 != 0 || n_rope % 2 != 0 || n_rope > 2 * n_out) return -1;
    const int n_warps = (int)(nb / 32);
    float *kcur = (float *)malloc((size_t)n_out * sizeof(float));
    int8_t *xq = (int8_t *)malloc((size_t)n_embd);
    float *xd = (float *)malloc((size_t)nb * sizeof(float));
    if (!kcur || !xq || !xd) { free(kcur); free(xq); free(xd); return -2; }
    for (int64_t b = 0; b < nb; ++b) quant_block_mul(cur + 32 * b, xq + 32 * b, &xd[b]);
    /* 1. gemv */
    for (int64_t o = 0; o < n_out; ++o) {
        const uint8_t *row = w + o * nb * 34;
        float total = 0.0f;
        for (int wv = 0; wv < n_warps; ++wv) {
            float p[32];
            for (int k = 0; k < 32; ++k) {
                const int64_t b = 32 * wv + k;
                const uint8_t *blk = row + 34 * b;
                const int32_t s = dot_q8((const int8_t *)(blk + 2), xq + 32 * b);
                p[k] = (q8_scale(blk) * xd[b]) * (float)s;
            }
            const float ws = warp32_sum(p);
            total = (wv == 0) ? ws : total + ws;
        }
        kcur[o] = total;
    }
    /* 2. rms norm over [0, d_lat) */
    float s = 0.0f;
    for (int64_t wv = 0; wv < n_out / 32; ++wv) {
        float p[32];
        for (int k = 0; k < 32; ++k) {
            const int64_t r = 32 * wv + k;
            const float v = r < d_lat ? kcur[r] : 0.0f;
            p[k] = v * v;
        }
        s += warp32_sum(p);
    }
    const float scale = 1.0f / sqrtf(s / (float)d_lat + eps);
    /* 3. rope over [d_lat, d_lat + n_rope) */
    float corr[2];
    orc_rope_yarn_corr_dims((int)n_rope, n_ctx_orig, freq_base, beta_fast, beta_slow, corr);
    const float theta_scale = powf(freq_base, -2.0f / (float)n_rope);
    for (int64_t p = 0; p < n_rope / 2; ++p) {
        const float x0 = kcur[d_lat + 2 * p], x1 = kcur[d_lat + 2 * p + 1];
        const float theta_extrap = (float)pos * powf(theta_scale, (float)p);
        float mscale = attn_factor;
        float theta = freq_scale * theta_extrap;
        if (ext_factor != 0.0f) {
            const float c0 = mutant == 3 ? corr[1] : corr[0], c1 = mutant == 3 ? corr[0] : corr[1];   /* swapped dims */
            const float y = ((float)p - c0) / fmaxf(0.001f, c1 - c0);
            const float cl = fminf(1.0f, fmaxf(0.0f, y));
            const float ramp_mix = (mutant == 4 ? cl : 1.0f - cl) * ext_factor;                   /* ramp sign slip */
            theta = theta * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
        }
        const float co = cosf(theta) * mscale, si = sinf(theta) * mscale;
        kcur[d_lat + 2 * p] = x0 * co - x1 * si;
        kcur[d_lat + 2 * p + 1] = (mutant == 1 ? -x0 : x0) * si + x1 * co;    /* sign slip */
    }
    for (int64_t r = 0; r < d_lat; ++r) kcur[r] = scale * kcur[r] * nw[r];
    /* 4. the cache row and dst */
    uint16_t *crow = (uint16_t *)((char *)kcache + (mutant == 2 ? kidx + 1 : kidx) * kc_nb1);   /* wrong row */
    for (int64_t r = 0; r < n_out; ++r) {
        crow[r] = f32_to_f16_rne(kcur[r]);
        dst[r] = kcur[r];
    }
    free(kcur); free(xq); free(xd);
    return 0;
}

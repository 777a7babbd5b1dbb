// mla_merge.h -- the split-K merge of one unit (64 output columns of one head of one token), the
// body of the PHASE merge kernel (mla_kernels.h describes the partial records).  The combine of patches/ggml-m4/m4-kqkv.cu:314-338: m* = max m_s,
// l* = sum l_s e^(m_s - m*), o* = sum l_s e^(m_s - m*) (o_s / l_s), out = o* / l* (0 if every split
// is empty).
#pragma once

#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

// Scratch for one unit's cross-wavefront fold (LDS, 16-byte aligned).
struct MergeScratch {
    float sm[4][8];
    float sL[4][8];
    f32x4 sO[4][8][2];
};

// One workgroup (256 threads) per unit: 8 column-lanes (8 f16 columns = 16 bytes
// each) x 32 split-lanes (the record layout of mla_kernels.h).  Split-lane sl takes splits sl, sl + 32, ...: the loads of a 256-split
// chunk (16 bytes of o/l plus m, l) all issue before the first use, then the chunk is folded with
// the max taken first.  Split-lanes are combined with wavefront shuffles, then across the four
// wavefronts through LDS.  Accumulators: (m, L = sum l_s e^(m_s - m), O = sum l_s e^(m_s - m) o_s).
template <typename OT>
__device__ __forceinline__ void merge_unit(const char * __restrict__ part, int dv, int n_split, int nt, int cblk, int h,
                                           int t, float * __restrict__ dst, MergeScratch & sc) {
    float (&sm)[4][8] = sc.sm;
    float (&sL)[4][8] = sc.sL;
    f32x4 (&sO)[4][8][2] = sc.sO;

    constexpr int J = 8;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c8 = tid & 7, sl_i = tid >> 3;               // column lane, split lane (0..31)
    const int c = cblk * 64 + 8 * c8;
    const int hh = h % PART_HEADS;
    const char * rec = part_record(part, h / PART_HEADS, nt, t, n_split, dv, (int)sizeof(OT));
    const int cc = min(c, dv - 8);
    // the record's o blocks, read through a buffer resource: an empty split's block (never
    // written) is skipped by an out-of-range offset, which reads zeros without a memory access.
    // Each o line has one reader, so it is loaded non-temporal: records read with the default
    // policy stay in the readers' L2s, and the next step's partial kernel, rewriting the same
    // workspace, then ran ~0.65 us longer from its last workgroup to the merge's first loads
    // (config 3, 192 splits: step 20.0 -> 19.35 us; the (m, l) pairs, read by every column block
    // of a head, keep the default policy).
    const char * obase = rec + part_o_off(n_split, 0, dv, (int)sizeof(OT));
    const uint32_t oblk = (uint32_t)(PART_HEADS * dv * (int)sizeof(OT));
    const uint32_t orecs = (uint32_t)n_split * oblk;
    const uint32_t ocol = (uint32_t)((hh * dv + cc) * (int)sizeof(OT));

    float m = -INFINITY, L = 0.0f;
    float O[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_split; s0 += 32 * J) {
        float ms[J], ls[J];
        float os[J][8];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int s = s0 + 32 * j + sl_i;
            const int sc_ = min(s, n_split - 1);
            // (m, l): consecutive split-lanes read consecutive pairs of this head's row
            const f32x2 ml = *reinterpret_cast<const f32x2 *>(rec + part_ml_off(n_split, hh, sc_));
            ms[j] = (s < n_split) ? ml[0] : -INFINITY;
            ls[j] = ml[1];
            // o only where the split has a live key
            const uint32_t off = (ms[j] != -INFINITY) ? (uint32_t)sc_ * oblk + ocol : 0xFFFFFFE0u;   // (+16 stays out of range)
            if constexpr (sizeof(OT) == 2) {
                const half8 v = __builtin_bit_cast(half8, buf_ld16<true>(obase, orecs, off));
#pragma unroll
                for (int k = 0; k < 8; ++k) os[j][k] = (float)v[k];
            } else {
                const f32x4 v0 = __builtin_bit_cast(f32x4, buf_ld16<true>(obase, orecs, off));
                const f32x4 v1 = __builtin_bit_cast(f32x4, buf_ld16<true>(obase, orecs, off + 16u));
#pragma unroll
                for (int k = 0; k < 4; ++k) { os[j][k] = v0[k]; os[j][4 + k] = v1[k]; }
            }
        }
        float mx = m;
#pragma unroll
        for (int j = 0; j < J; ++j) mx = fmaxf(mx, ms[j]);
        const float f0 = exp2_unless(m == -INFINITY, (m - mx) * LOG2E);
        L *= f0;
#pragma unroll
        for (int k = 0; k < 8; ++k) O[k] *= f0;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float f = ls[j] * exp2_unless(ms[j] == -INFINITY, (ms[j] - mx) * LOG2E);
            L += f;
#pragma unroll
            for (int k = 0; k < 8; ++k) O[k] += f * os[j][k];
        }
        m = mx;
    }
    // fold the 8 split-lanes of this wavefront (lane bits 3..5) without LDS round trips: the
    // partner l ^ 8 by DPP, then the symmetric combine of the two 16-lane rows of each pair and of
    // the two halves (v_permlane16_swap / v_permlane32_swap give both operands at every lane)
    auto combine = [](float m1, float L1, const float (&O1)[8], float m2, float L2, const float (&O2)[8], float & mo,
                      float & Lo, float (&Oo)[8]) {
        const float M = fmaxf(m1, m2);
        const float f1 = exp2_unless(m1 == -INFINITY, (m1 - M) * LOG2E);
        const float f2 = exp2_unless(m2 == -INFINITY, (m2 - M) * LOG2E);
        Lo = L1 * f1 + L2 * f2;
#pragma unroll
        for (int k = 0; k < 8; ++k) Oo[k] = O1[k] * f1 + O2[k] * f2;
        mo = M;
    };
    {
        float O2[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) O2[k] = dpp_xor<8>(O[k]);
        combine(m, L, O, dpp_xor<8>(m), dpp_xor<8>(L), O2, m, L, O);
    }
    {
        float ma, mb, La, Lb, Oa[8], Ob[8];
        rows_pair16(m, ma, mb);
        rows_pair16(L, La, Lb);
#pragma unroll
        for (int k = 0; k < 8; ++k) rows_pair16(O[k], Oa[k], Ob[k]);
        combine(ma, La, Oa, mb, Lb, Ob, m, L, O);
    }
    {
        float ma, mb, La, Lb, Oa[8], Ob[8];
        halves_pair(m, ma, mb);
        halves_pair(L, La, Lb);
#pragma unroll
        for (int k = 0; k < 8; ++k) halves_pair(O[k], Oa[k], Ob[k]);
        combine(ma, La, Oa, mb, Lb, Ob, m, L, O);
    }
    if (lane < 8) {
        sm[w][c8] = m;
        sL[w][c8] = L;
        sO[w][c8][0] = f32x4{O[0], O[1], O[2], O[3]};
        sO[w][c8][1] = f32x4{O[4], O[5], O[6], O[7]};
    }
    __syncthreads();
    if (tid < 8 && c < dv) {
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) M = fmaxf(M, sm[i][c8]);
        f32x4 r0 = {0.f, 0.f, 0.f, 0.f}, r1 = {0.f, 0.f, 0.f, 0.f};
        if (M > -INFINITY) {
            float LL = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float f = exp2_unless(sm[i][c8] == -INFINITY, (sm[i][c8] - M) * LOG2E);
                LL += sL[i][c8] * f;
                r0 += sO[i][c8][0] * f;
                r1 += sO[i][c8][1] * f;
            }
            const float inv = 1.0f / LL;
            r0 *= inv;
            r1 *= inv;
        }
        float * d = dst + ((size_t)h * nt + t) * dv + c;
        *reinterpret_cast<f32x4 *>(d) = r0;
        *reinterpret_cast<f32x4 *>(d + 4) = r1;
    }
}

}  // namespace mla

// kqkv_prefill.hip -- GGML_OP_M4_KQKV for several query tokens (chunked prefill), on MFMA.
//
// The op of patches/ggml-m4/m4-kqkv.cu:340-378 (which the reference only runs for one token) for
// nt >= 16 tokens: out[h, t] = softmax_j(kq_scale q[t, h] . K[j] + mask[t, j]) . V[j] over the
// cache.  With many tokens the work is a dense contraction (config 5: 285 GFLOP over a 9.4 MB
// cache), so the design is MFMA-bound rather than HBM-bound:
//   * One workgroup per (split, 32-head group, 4 tokens); wave w owns token 4 z + w with all 32
//     heads: its q fragments (144 VGPRs, loaded once), its online softmax and its o^T for all D_v
//     columns (16 accumulator tiles in AGPRs).  No state crosses waves, so each finishes its token
//     on its own.
//   * The four waves share every 64-key tile: each streams one 16-key slice of it into a two-stage
//     LDS ring (decode_common.h layout, cached DMA: the cache is re-read by every token group and
//     stays in L2 / MALL) plus its own token's 64 mask values, and then every wave runs all four
//     slices -- 4 tokens x 32 heads share each K / V byte read from LDS.  One workgroup barrier
//     per tile; the next tile's DMA goes out one instruction per even Q.K^T step of the first two
//     slices.
//   * Per slice: S^T = K . Q^T (16 keys x 32 heads, v_mfma_f32_16x16x32_f16, accumulators in
//     VGPRs: the output tiles fill the AGPRs), scores with the token's mask, a lazily moved
//     reference max (P = exp2(s - m) <= 2^15; the move test on each lane's own maxima), P^T for P.V
//     by two v_permlane16_swap, o^T += V^T . P^T (v_mfma_f32_32x32x16_f16, V^T by
//     ds_read_b64_tr_b16).  l is summed from the same f16 P values.  q enters as f16, where
//     ggml-cpu's mul_mat rounds it; P enters as f16 too, but UNNORMALISED (exp2 of the score minus
//     the lazy reference max, <= 2^15), where ggml-cpu rounds the normalised softmax output -- at
//     long context the latter is subnormal in f16, so the two differ by more than one rounding
//     (this kernel is the closer of the two to exact arithmetic).  The next slice's first Q.K^T
//     operands and mask values are read
//     during P.V, the first V^T operands during the softmax.
//
// Grid = (n_split, ceil(H/32), ceil(nt/4)), 256 threads.  Output as the decode kernels: partial
// blocks [group][token][split] (mla_kernels.h) for the merge, or o/l in f32 to dst with one split.
#include "decode_common.h"

namespace mla {

namespace {

using namespace decode;

template <int DK, int DV>
struct PrefillCfg {
    using G = SliceGeom<DK>;
    static_assert(DV % 128 == 0 && DV <= DK, "geometry");
    static constexpr int NB = DV / 32;                  // 32-column o^T tiles per wave
    static constexpr int OPITCH = DV * 2 + 16;          // f16 output staging row pitch (bytes)
    static constexpr int CPR = DV / 8;                  // 16-byte output chunks per head row
    static_assert(NWAVE * HG * OPITCH <= G::RING, "the output staging fits the ring");
    static_assert(CPR % 2 == 0 && NB - 1 < 64, "layout");
};

template <int DK, int DV>
__global__ __launch_bounds__(NTHR, 1) void kqkv_prefill_f16_kernel(DecodeArgs a) {
    using G = SliceGeom<DK>;
    using C = PrefillCfg<DK, DV>;
    __shared__ __attribute__((aligned(16))) char ring[G::RING];          // [stage][wave] K rows + mask

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int g = lane >> 4;
    const int j16 = lane & 15;
    const int t_w = blockIdx.z * NWAVE + w;          // this wave's token
    const bool token_live = t_w < a.nt;
    const int t = min(t_w, a.nt - 1);                // (a wave past the last token mirrors it, unused)

    SliceStream<DK> ss(a, sp, t, w, lds_addr(ring), lane);
    ss.mvoff = 4u * (uint32_t)lane;                  // the mask slot holds this token's 64 keys of the tile
    const int n_my = ss.n_my;
    // DMA of tile k into stage s: this wave's 16-key slice of K rows (cached policy: every token
    // group re-reads the cache) and this wave's token's mask over the tile's 64 keys (zeros past
    // n_kv or without a mask)
    auto plan = [&](int s, int k) {
        SliceDma d = ss.plan(s, k);
        const int tile = min(ss.t0 + min(k, n_my - 1), ss.n_tiles - 1);
        const int mleft = a.n_kv - tile * TK;
        d.mrs = make_rsrc(ss.mrow + tile * TK, (ss.has_mask && mleft > 0) ? (uint32_t)mleft * 4u : 0u);
        return d;
    };
    // Rows over per-sequence regions (batch-of-N decode): a wave whose token has no live key in this
    // split still streams its slices for the others but computes nothing; a workgroup with no live
    // token records empty splits and leaves before any DMA.  (One split writes dst directly: every
    // row is computed.)
    const bool live_w = token_live && (a.dst != nullptr || split_live<DK>(a, ss, t, lane));
    if (!__syncthreads_or(live_w)) {
        if (token_live && a.dst == nullptr) write_empty_pairs(a, blockIdx.y, t, sp, DV, lane);
        return;
    }
    {
        const SliceDma d0 = plan(0, 0);
#pragma unroll
        for (int i = 0; i <= G::DMA_N; ++i) ss.template put<false>(d0, i);
    }

    // ---- q fragments of this wave's token: qreg[n][s] = head 16 n + j16, d = 32 s + 8 g .. +7 ----
    half8 qreg[2][G::QSTEPS];
    {
        constexpr int QB = G::QSTEPS % 6 == 0 ? 6 : (G::QSTEPS % 5 == 0 ? 5 : 2);
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const int h = hg0 + 16 * n + j16;
            const bool hv = h < a.n_head;
            const char * row = reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 + (size_t)min(h, a.n_head - 1) * a.q_nb1;
#pragma unroll
            for (int s0 = 0; s0 < G::QSTEPS; s0 += QB) {
                f32x4 x[QB][2];
#pragma unroll
                for (int b = 0; b < QB; ++b) {
                    x[b][0] = *reinterpret_cast<const f32x4 *>(row + 4 * (32 * (s0 + b) + 8 * g));
                    x[b][1] = *reinterpret_cast<const f32x4 *>(row + 4 * (32 * (s0 + b) + 8 * g + 4));
                }
#pragma unroll
                for (int b = 0; b < QB; ++b) {
                    half8 hq = {to_half(x[b][0][0]), to_half(x[b][0][1]), to_half(x[b][0][2]), to_half(x[b][0][3]),
                                to_half(x[b][1][0]), to_half(x[b][1][1]), to_half(x[b][1][2]), to_half(x[b][1][3])};
                    if (!hv) hq = half8{0, 0, 0, 0, 0, 0, 0, 0};
                    asm volatile("" : "+v"(hq));     // keep the f16 fragment (not the f32 values) live
                    qreg[n][s0 + b] = hq;
                }
            }
        }
    }

    // ---- per-wave state ----
    float m_run[2] = {M_NONE, M_NONE};       // heads 16 n + j16, log2 units
    float l_acc = 0.0f;                      // head lane & 31, keys 8 (lane >> 5) .. +7 of each slice
    f32x16 o[C::NB];                         // o^T tile i: C row = column 32 i + 8 (r / 4) + 4 (lane >> 5) + (r & 3), C col = head lane & 31
#pragma unroll
    for (int i = 0; i < C::NB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
    const PvAddr pv(lane);
    const int own_h = (lane >> 4) & 1;

    for (int k = 0; k < n_my; ++k) {
        wait_vm<0>();                        // this wave's slot of tile k (and its mask row) has landed
        __syncthreads();                     // all four have; every wave is done with tile k - 1
        const bool pf = k + 1 < n_my;
        const SliceDma dn = plan((k + 1) & 1, k + 1);
        const int par = k & 1;
        const int key_t = (ss.t0 + k) * TK;
        const char * mkb = ring + ss.stage_off(par, w) + G::ROWS_BYTES;    // this token's mask, 64 keys
        if (!live_w) {                       // only this wave's slice of the next tile
            if (pf) {
#pragma unroll
                for (int i = 0; i <= G::DMA_N; ++i) ss.template put<false>(dn, i);
            }
            continue;
        }
        // slice 0's first Q.K^T operands and mask values (later slices': during the P.V before)
        half8 abuf[QPF_LANDED];
        qk_operands<DK>(ring + ss.stage_off(par, 0), lane, abuf);
        f32x4 mk_next = *reinterpret_cast<const f32x4 *>(mkb + 16 * g);
#pragma unroll 1
        for (int ks = 0; ks < NWAVE; ++ks) {
            const char * sb = ring + ss.stage_off(par, ks);
            const f32x4 mk = mk_next;
            f32x4 s0, s1;
            // tile k + 1's DMA, one instruction per even Q.K^T step of slices 0 and 1 (row blocks
            // DMA_N / 2 * ks + s / 2) and the mask slot after slice 1's last step: the CU's 76 KB of
            // DMA per tile, issued within one slice, held the issuing waves ~450 cycles
            if (pf && ks < 2) {
                qk_slice_landed<DK>(sb, lane, qreg, abuf, s0, s1, [&](int st) {
                    constexpr int HALF = G::DMA_N / 2;
                    static_assert(G::DMA_N % 2 == 0 && G::QSTEPS == G::DMA_N, "two slices of row blocks");
                    if ((st & 1) == 0) ss.template put<false>(dn, HALF * ks + st / 2);
                    else if (st == G::QSTEPS - 1 && ks == 1) ss.template put<false>(dn, G::DMA_N);
                });
            } else {
                qk_slice_landed<DK>(sb, lane, qreg, abuf, s0, s1, [](int) {});
            }
            // the first V^T operands of P.V, read ahead so that their latency passes under the softmax
            constexpr int VPF = 3;
            half8 vb[VPF];
#pragma unroll
            for (int i = 0; i < VPF; ++i) vb[i] = pv.load(sb, i);
            __builtin_amdgcn_sched_barrier(0);
            float sc[2][4], mx[2];
            slice_scores<false>(a, mk, key_t + WK * ks, lane, s0, s1, sc, mx);     // this lane's maxima
            if (__builtin_amdgcn_ballot_w64(ref_moves(m_run[0], mx[0]) || ref_moves(m_run[1], mx[1])) != 0) {
                // rare: move the reference to the head's slice max, rescale
                float al[2];
                bool mv[2];
#pragma unroll
                for (int n = 0; n < 2; ++n) {
                    mx[n] = rows4_max(mx[n]);
                    mv[n] = ref_moves(m_run[n], mx[n]);
                    al[n] = !mv[n] ? 1.0f : exp2_fast(m_run[n] - mx[n]);     // 0 from M_NONE
                    m_run[n] = mv[n] ? mx[n] : m_run[n];
                }
                const float a_own = al[own_h];
                l_acc *= a_own;
                // in place on the accumulator registers (kept in AGPRs); the s_nops cover the
                // MFMA -> VALU read distance
                asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
                for (int i = 0; i < C::NB; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float tmp;
                        asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                                     : "+a"(o[i][r]), "=&v"(tmp) : "v"(a_own));
                    }
                asm volatile("s_nop 7" ::: "memory");
            }
            // P^T operand: Q.K^T's C layout (lane: keys 4 g .. +3 of heads j16 and 16 + j16) into
            // P.V's B layout (lane: keys 8 (lane >> 5) .. +7 of head lane & 31), one
            // v_permlane16_swap per pair of f16 values
            uint32_t px[2], py[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float x0 = exp2_fast(sc[0][2 * e] - m_run[0]);
                const float x1 = exp2_fast(sc[0][2 * e + 1] - m_run[0]);
                const float y0 = exp2_fast(sc[1][2 * e] - m_run[1]);
                const float y1 = exp2_fast(sc[1][2 * e + 1] - m_run[1]);
                px[e] = __builtin_bit_cast(uint32_t, half2{to_half(x0), to_half(x1)});
                py[e] = __builtin_bit_cast(uint32_t, half2{to_half(y0), to_half(y1)});
                const auto sw = __builtin_amdgcn_permlane16_swap(px[e], py[e], false, false);
                px[e] = sw[0];
                py[e] = sw[1];
            }
            const half8 pt = __builtin_bit_cast(half8, u32x4{px[0], px[1], py[0], py[1]});
#pragma unroll
            for (int e = 0; e < 8; e += 2) l_acc = __builtin_amdgcn_fdot2(half2{pt[e], pt[e + 1]}, ONE2, l_acc, false);
            {
#pragma unroll
                for (int i = 0; i < C::NB; ++i) {
                    const half8 va = vb[i % VPF];
                    if (i + VPF < C::NB) vb[i % VPF] = pv.load(sb, i + VPF);
                    o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pt, o[i], 0, 0, 0);
                    if (i == C::NB / 2 && ks + 1 < NWAVE) {     // the next slice's operands and mask
                        qk_operands<DK>(ring + ss.stage_off(par, ks + 1), lane, abuf);
                        mk_next = *reinterpret_cast<const f32x4 *>(mkb + 64 * (ks + 1) + 16 * g);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
    wait_vm<0>();
    __syncthreads();                         // the ring becomes the output staging
#pragma unroll
    for (int n = 0; n < 2; ++n) m_run[n] = (m_run[n] == M_NONE) ? -INFINITY : m_run[n];     // no live key: -inf

    int tid_e;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid_e) : "v"(tid));
    const int lane_e = tid_e & 63;
    const int hl = lane_e & 31;
    const float L = halves_sum(l_acc);         // head hl, all keys of the split
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (!token_live) return;
    if (!live_w) {                           // (a.dst == nullptr here)
        write_empty_pairs(a, blockIdx.y, t, sp, DV, lane_e);
        return;
    }
    const int hi4 = 4 * (lane_e >> 5);
    if (a.dst != nullptr) {                  // single split: o / l in f32 straight to dst
        const int h = hg0 + hl;
        if (h < a.n_head) {
            float * d = a.dst + ((size_t)h * a.nt + t) * DV + hi4;
#pragma unroll
            for (int i = 0; i < C::NB; ++i)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                    *reinterpret_cast<f32x4 *>(d + 32 * i + 8 * q4) =
                        f32x4{o[i][4 * q4] * inv, o[i][4 * q4 + 1] * inv, o[i][4 * q4 + 2] * inv, o[i][4 * q4 + 3] * inv};
        }
        return;
    }
    char * rec = part_record(a.part, blockIdx.y, a.nt, t, a.n_split, DV, 2);
    char * blk = rec + part_o_off(a.n_split, sp, DV, 2);
    if (lane_e < HG) {
        const float mr = m_run[(lane_e >> 4) & 1];        // lane_e's head 16 ((lane_e >> 4) & 1) + j16
        *reinterpret_cast<f32x2 *>(rec + part_ml_off(a.n_split, lane_e, sp)) =
            f32x2{(mr == -INFINITY) ? -INFINITY : mr * LN2, L};                   // m in natural-log units
    }
    // o / l in f16 through this wave's staging rows [32 heads][D_v], then 16-byte row chunks out
    char * stg = ring + w * HG * C::OPITCH;
#pragma unroll
    for (int i = 0; i < C::NB; ++i)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const half4 hv = {to_half(o[i][4 * q4] * inv), to_half(o[i][4 * q4 + 1] * inv), to_half(o[i][4 * q4 + 2] * inv),
                              to_half(o[i][4 * q4 + 3] * inv)};
            *reinterpret_cast<half4 *>(stg + hl * C::OPITCH + (32 * i + 8 * q4 + hi4) * 2) = hv;
        }
#pragma unroll
    for (int it = 0; it < C::CPR / 2; ++it) {
        const int q = 64 * it + lane_e;
        const int row = q / C::CPR, ch = q % C::CPR;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + row * C::OPITCH + 16 * ch);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(blk + ((size_t)row * DV + 8 * ch) * 2));
    }
}

}  // namespace

template <int DK, int DV>
static hipError_t launch_prefill(const DecodeArgs & a, int n_hgroups, hipStream_t stream) {
    dim3 grid(a.n_split, n_hgroups, (a.nt + NWAVE - 1) / NWAVE);
    hipLaunchKernelGGL((kqkv_prefill_f16_kernel<DK, DV>), grid, dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kqkv_prefill_f16(int dk, int dv, const DecodeArgs & a, hipStream_t stream) {
    const int n_hgroups = (a.n_head + HG - 1) / HG;
    if (dk == 576 && dv == 512) return launch_prefill<576, 512>(a, n_hgroups, stream);
    if (dk == 320 && dv == 256) return launch_prefill<320, 256>(a, n_hgroups, stream);
    return hipErrorInvalidValue;
}

}  // namespace mla

// kqkv_decode_long.hip -- split-K MLA decode attention over an f16 latent+rope KV cache, for long
// splits (many 64-key tiles per workgroup): the same work as kqkv_decode.hip (reference:
// patches/ggml-m4/m4-kqkv.cu:201-312), organised for throughput rather than for the tail.
//   * The four waves (one per SIMD) run independent pipelines over their 16-key slices of the
//     split's tiles (decode_common.h): each streams its own slots, keeps its own online softmax
//     state and its own o^T for all D_v columns (16 accumulator tiles in AGPRs).  No workgroup
//     barrier runs in the main loop, so a wave whose slice lands early never waits for the others;
//     the four states are merged once, at the end (which costs more than kqkv_decode.hip's
//     epilogue: the library picks this kernel when a split has many tiles).
//   * Q.K^T: S^T[16 keys x 32 heads] = K . Q^T.  Its C layout becomes the B operand of P.V
//     (P^T[16 keys x 32 heads]) with two v_permlane16_swap, and P.V runs as o^T = V^T . P^T, so
//     every accumulator column is one head and the softmax rescale is a per-lane scalar.
//   * Online softmax in log2 units against a per-wave reference max moved lazily (only when a
//     slice raises a head's max by more than 2^15: P = exp2(s - m) <= 32768, exact range in f16, and
//     the accumulator rescale is rare).  l is summed from the same f16 P values the MFMAs consume.
//
// Grid = (n_split, ceil(H/32), nt), 256 threads; output as kqkv_decode.hip.
#include "decode_common.h"

namespace mla {

namespace {

using namespace decode;

template <int DK, int DV>
struct LongCfg {
    using G = SliceGeom<DK>;
    static_assert(DV % 128 == 0 && DV <= DK, "geometry");
    static constexpr int NB = DV / 32;                  // 32-column o^T tiles (all of D_v, per wave)
    static constexpr int NBQ = NB / NWAVE;              // tiles of the quarter a wave finishes
    static constexpr int DVQ = DV / NWAVE;              // columns of that quarter
    static constexpr int XCH = NBQ * 2 * 64 * 16;       // one wave's f16 share of one quarter
    static constexpr int OPITCH = DVQ * 2 + 16;         // output staging row pitch (bytes)
    static constexpr int CPR = DVQ / 8;                 // 16-byte output chunks per head row
    static_assert(NB % NWAVE == 0 && CPR % 2 == 0, "whole quarters");
    static_assert(NWAVE * (NWAVE - 1) * XCH <= G::RING, "the end-of-split exchange fits the ring");
    static_assert(HG * OPITCH <= (NWAVE - 1) * XCH, "the output staging fits a quarter's exchange area");
    static_assert(NB - 1 < 64, "V^T operand offsets fit the DS immediate");
};

template <int DK, int DV>
__global__ __launch_bounds__(NTHR, 1) void kqkv_decode_f16_long_kernel(DecodeArgs a) {
    using G = SliceGeom<DK>;
    using C = LongCfg<DK, DV>;
    __shared__ __attribute__((aligned(16))) char ring[G::RING];          // [stage][wave] K rows + mask
    __shared__ __attribute__((aligned(16))) float fin_m[HG][NWAVE];      // per head: each wave's max (log2)
    __shared__ __attribute__((aligned(16))) float fin_l[HG][NWAVE];      // and sum relative to it

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int t = blockIdx.z;
    const int j16 = lane & 15;

    const SliceStream<DK> ss(a, sp, t, w, lds_addr(ring), lane);
    const int n_my = ss.n_my;
    // several rows (batch-of-N decode over per-sequence regions): a split that holds no live key
    // of this row only records that, before any DMA
    if (a.nt > 1 && a.dst == nullptr && !split_live<DK>(a, ss, t, lane)) {
        if (w == 0) write_empty_pairs(a, blockIdx.y, t, sp, DV, lane);
        return;
    }
    half8 qreg[2][G::QSTEPS];
    stage_q<DK>(a, ss, ring, hg0, t, lane, qreg);

    // ---- per-wave state: reference max, l from the f16 P operands, o^T over all columns ----
    float m_run[2] = {M_NONE, M_NONE};       // heads 16 n + j16, log2 units
    // sum of the P values this lane feeds to the P.V MFMAs: head lane & 31, keys 8 (lane >> 5) .. +7
    // of each of the wave's slices (lane ^ 32 holds the other half)
    float l_acc = 0.0f;
    // o^T tile i: C row = column 32 i + 8 (r / 4) + 4 (lane >> 5) + (r & 3), C col = head lane & 31
    f32x16 o[C::NB];
#pragma unroll
    for (int i = 0; i < C::NB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
    const PvAddr pv(lane);
    const int own_h = (lane >> 4) & 1;       // this lane's o^T head lane & 31 = 16 own_h + j16

    for (int k = 0; k < n_my; ++k) {
        // the wave's other slot held slice k - 1, whose last reader was this wave's P.V of k - 1:
        // it takes slice k + 1, DMA spread over this slice's Q.K^T steps
        const SliceDma dn = ss.plan((k + 1) & 1, k + 1);
        const char * sb = ring + ss.stage_off(k & 1, w);
        const int kbase = (ss.t0 + k) * TK + WK * w;
        f32x4 s0, s1;
        if (k + 1 < n_my) qk_slice<DK, true, true, true, true>(ss, dn, sb, lane, qreg, s0, s1);
        else qk_slice<DK, false, true, true, true>(ss, dn, sb, lane, qreg, s0, s1);
        float sc[2][4], mx[2];
        slice_scores<false>(a, slice_mask<DK>(sb, lane), kbase, lane, s0, s1, sc, mx);     // this lane's maxima
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
            if (k > 0) {                          // (before the first slice the accumulators are 0)
                // in place on the accumulator registers, one asm block per element, so that they
                // stay in AGPRs across this branch; the s_nops cover the MFMA -> VALU read distance
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
        }
        // P = 2^(s - m) <= 2^15 in f16; lane (j16, g) holds keys 4 g .. 4 g + 3 of heads j16 (x) and
        // 16 + j16 (y).  Swapping the odd 16-lane rows of x with the even rows of y leaves lane l
        // with head l & 31, keys 8 (l >> 5) .. +7 in (x, y): the P^T operand of P.V.
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

        // o^T[:, heads] += V^T . P^T over the slice's 16 keys, all D_v columns; the V^T operands
        // run VPF tiles ahead of their MFMAs
        {
            constexpr int VPF = 3;
            half8 vb[VPF];
#pragma unroll
            for (int i = 0; i < VPF; ++i) vb[i] = pv.load(sb, i);
#pragma unroll
            for (int i = 0; i < C::NB; ++i) {
                const half8 va = vb[i % VPF];
                if (i + VPF < C::NB) vb[i % VPF] = pv.load(sb, i + VPF);
                o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pt, o[i], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    wait_vm<0>();                            // nothing of this wave may still target the ring
#pragma unroll
    for (int n = 0; n < 2; ++n) m_run[n] = (m_run[n] == M_NONE) ? -INFINITY : m_run[n];     // no live key: -inf

    // thread indices re-derived through an opaque move, so that the epilogue's address arithmetic
    // is computed here rather than before the loop and kept alive (or spilled) across it
    int tid_e;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid_e) : "v"(tid));
    const int lane_e = tid_e & 63;
    const int hl = lane_e & 31;

    // ---- merge of the four waves' states, per head ----
    const float lw = halves_sum(l_acc);         // head hl, all of this wave's keys
    if (lane_e < HG) {
        fin_m[lane_e][w] = m_run[(lane_e >> 4) & 1];      // lane_e's head is 16 ((lane_e >> 4) & 1) + j16
        fin_l[lane_e][w] = lw;
    }
    __syncthreads();                         // every wave is out of its loop: the ring is idle
    const f32x4 mm = *reinterpret_cast<const f32x4 *>(&fin_m[hl][0]);
    const f32x4 ll = *reinterpret_cast<const f32x4 *>(&fin_l[hl][0]);
    const float M = fmaxf(fmaxf(mm[0], mm[1]), fmaxf(mm[2], mm[3]));
    float L = 0.0f;
#pragma unroll
    for (int v = 0; v < NWAVE; ++v) L += ll[v] * exp2_unless(mm[v] == -INFINITY, mm[v] - M);
    const float m_w = (w == 0) ? mm[0] : (w == 1) ? mm[1] : (w == 2) ? mm[2] : mm[3];
    const float cw = (m_w == -INFINITY || !(L > 0.0f)) ? 0.0f : exp2_fast(m_w - M) / L;   // this wave's weight

    // Exchange: wave w hands its weighted o^T tiles of every other wave's quarter to that wave, as
    // f16 in the same lane order ([quarter][contributor][tile][half][lane] 16-byte chunks).
    auto xch = [&](int u, int c) { return ring + (u * (NWAVE - 1) + c) * C::XCH; };
#pragma unroll
    for (int u = 0; u < NWAVE; ++u) {
        if (u == w) continue;
        char * dstx = xch(u, w < u ? w : w - 1);
#pragma unroll
        for (int jb = 0; jb < C::NBQ; ++jb) {
            const f32x16 v = o[C::NBQ * u + jb];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                half8 hv;
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = to_half(v[8 * hf + e] * cw);
                *reinterpret_cast<half8 *>(dstx + ((jb * 2 + hf) * 64 + lane_e) * 16) = hv;
            }
        }
    }
    __syncthreads();
    // own quarter: weighted own tiles plus the three contributions
    f32x16 fo[C::NBQ];
#pragma unroll
    for (int u = 0; u < NWAVE; ++u) {
        if (u != w) continue;
#pragma unroll
        for (int jb = 0; jb < C::NBQ; ++jb) fo[jb] = o[C::NBQ * u + jb] * cw;
    }
#pragma unroll
    for (int c = 0; c < NWAVE - 1; ++c) {
        const char * srcx = xch(w, c);
#pragma unroll
        for (int jb = 0; jb < C::NBQ; ++jb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const half8 hv = *reinterpret_cast<const half8 *>(srcx + ((jb * 2 + hf) * 64 + lane_e) * 16);
#pragma unroll
                for (int e = 0; e < 8; ++e) fo[jb][8 * hf + e] += (float)hv[e];
            }
    }
    // fo[jb][r]: head hl, quarter column 32 jb + 8 (r / 4) + 4 (lane_e >> 5) + (r & 3)
    const int h_out = hg0 + hl;
    const bool direct = a.dst != nullptr;                 // single split: final f32 output to dst
    if (direct) {
        if (h_out < a.n_head) {
            float * d = a.dst + ((size_t)h_out * a.nt + t) * DV + C::DVQ * w + 4 * (lane_e >> 5);
#pragma unroll
            for (int jb = 0; jb < C::NBQ; ++jb)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                    *reinterpret_cast<f32x4 *>(d + 32 * jb + 8 * q4) =
                        f32x4{fo[jb][4 * q4], fo[jb][4 * q4 + 1], fo[jb][4 * q4 + 2], fo[jb][4 * q4 + 3]};
        }
        return;
    }
    char * rec = part_record(a.part, blockIdx.y, a.nt, t, a.n_split, DV, 2);
    char * blk = rec + part_o_off(a.n_split, sp, DV, 2);
    if (w == 0 && lane_e < HG)
        *reinterpret_cast<f32x2 *>(rec + part_ml_off(a.n_split, lane_e, sp)) =
            f32x2{(M == -INFINITY) ? -INFINITY : M * LN2, L};                     // m in natural-log units
    // f16 [32 heads][DVQ] staging in this wave's own (consumed) exchange area, then 16-byte rows
    // out: the same wave writes and reads it, in LDS order
    char * stg = xch(w, 0);
#pragma unroll
    for (int jb = 0; jb < C::NBQ; ++jb)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const half4 hv = {to_half(fo[jb][4 * q4]), to_half(fo[jb][4 * q4 + 1]), to_half(fo[jb][4 * q4 + 2]),
                              to_half(fo[jb][4 * q4 + 3])};
            *reinterpret_cast<half4 *>(stg + hl * C::OPITCH + (32 * jb + 8 * q4 + 4 * (lane_e >> 5)) * 2) = hv;
        }
#pragma unroll
    for (int it = 0; it < C::CPR / 2; ++it) {
        const int q = 64 * it + lane_e;
        const int row = q / C::CPR, ch = q % C::CPR;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + row * C::OPITCH + 16 * ch);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(blk + ((size_t)row * DV + C::DVQ * w + 8 * ch) * 2));
    }
}

}  // namespace

template <int DK, int DV>
static hipError_t launch_long(const DecodeArgs & a, int n_hgroups, hipStream_t stream) {
    dim3 grid(a.n_split, n_hgroups, a.nt);
    hipLaunchKernelGGL((kqkv_decode_f16_long_kernel<DK, DV>), grid, dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kqkv_decode_f16_long(int dk, int dv, const DecodeArgs & a, hipStream_t stream) {
    const int n_hgroups = (a.n_head + HG - 1) / HG;
    if (dk == 576 && dv == 512) return launch_long<576, 512>(a, n_hgroups, stream);
    if (dk == 320 && dv == 256) return launch_long<320, 256>(a, n_hgroups, stream);
    return hipErrorInvalidValue;
}

}  // namespace mla

// kqkv_decode.hip -- split-K MLA decode attention over an f16 latent+rope KV cache, on MFMA, for
// splits of any number of 64-key tiles (the 32K-key decode step: two or three tiles per workgroup;
// 262,144 keys: sixteen).
//
// The pass-1 kernel of GGML_OP_M4_KQKV (reference: patches/ggml-m4/m4-kqkv.cu:201-312), designed
// for gfx950 rather than translated:
//   * ALL heads of a 32-head group live in one workgroup, so every KV byte is fetched from HBM
//     exactly once per token (MLA's single latent row serves every head).
//   * Q.K^T and P.V are dense contractions ([32 x D_k].[D_k x keys] and [32 x keys].[keys x D_v],
//     60 FLOP per cache byte): they run on v_mfma_f32_16x16x32_f16 / v_mfma_f32_32x32x16_f16 with
//     f32 accumulation.  q enters the MFMA as f16, where the unfused ggml-cpu graph rounds it (its
//     mul_mat converts src1 to F16 for an F16 src0).  P enters as f16 as well, but UNNORMALISED
//     (exp2 of the score minus the lazy reference max below, at most 2^15), whereas ggml-cpu rounds
//     the normalised softmax output to f16; at long context that is subnormal in f16, so the two
//     rounding points differ (this kernel is the closer of the two to exact arithmetic).
//   * Work split of a 64-key tile over the 4 waves (one per SIMD): for Q.K^T wave w owns its slice,
//     keys 16 w .. 16 w + 15, against all 32 heads (decode_common.h: slice DMA into a two-stage
//     LDS ring, per-block DMA waits, q fragments in VGPRs); for P.V wave w owns the output columns
//     D_v/4 * w .. + D_v/4 against all 64 keys (accumulators in AGPRs).  P moves between the two
//     through a 4.5 KB LDS exchange; that and the slice maxima need one workgroup barrier per tile,
//     and the end of the split needs none, which keeps the tail after the last tile short.
//   * Online softmax in log2 units (v_exp_f32) against a reference max shared by the waves and
//     moved lazily: only when a tile raises a head's max by more than 2^15, so P = exp2(s - m_ref)
//     <= 32768 (exact range in f16) and the accumulator rescale is rare.  P is computed against the
//     current reference before the barrier and recomputed after it only when the reference moves.
//   * l is summed from the same f16 P values the P.V MFMAs consume (every wave reads the whole P
//     exchange for its heads), so o / l is an exact convex combination of V rows and each wave
//     finishes on its own; the header's m is the shared reference maximum (l relative to it),
//     which is all the log-sum-exp merge needs.
//
// Grid = (n_split, ceil(H/32), nt), 256 threads.  Output: one partial block per (32-head group,
// token, split) -- m and l per head in f32 and the split's normalised output o/l in f16,
// [32 heads][D_v] (mla_kernels.h) -- or, with a single split, o/l in f32 to dst.
#include "decode_common.h"

namespace mla {

namespace {

using namespace decode;

// One row (token) t of the split: the whole pass, from the q staging to the partial record.
template <int DK, int DV>
__device__ __forceinline__ void decode_row(const DecodeArgs & a, int t, DecodeLds<DK, DV> & sh) {
    using G = SliceGeom<DK>;
    using C = DecodeCfg<DK, DV>;
    char (&ring)[G::RING] = sh.ring;
    half_t (&px)[2][HG * C::PROW] = sh.px;
    float (&red)[2][HG][NWAVE] = sh.red;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int g = lane >> 4;                 // 16-lane group
    const int j16 = lane & 15;

    const SliceStream<DK> ss(a, sp, t, w, lds_addr(ring), lane);
    const int n_my = ss.n_my;
    half8 qreg[2][G::QSTEPS];
    stage_q<DK>(a, ss, ring, hg0, t, lane, qreg);

    // ---- running state: reference max identical in every wave; l from the f16 P operands ----
    float m_ref[2] = {M_NONE, M_NONE};       // heads 16 n + j16, log2 units
    // sum of the P values this lane feeds to the P.V MFMAs: head lane & 31, keys 8 (lane >> 5) .. +7
    // of each 16-key slice (the lane ^ 32 holds the other half)
    float l_acc = 0.0f;
    // o^T tile i: C row = column DVQ w + 32 i + 8 (r / 4) + 4 (lane >> 5) + (r & 3), C col = head lane & 31
    f32x16 o[C::NTQ];
#pragma unroll
    for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
    // P.V operands: A = P rows (lane & 31), keys 16 ks + 8 (lane >> 5); B = V of slice ks, this
    // wave's column tiles NTQ w + i
    const PvAddr pv(lane);

    for (int k = 0; k < n_my; ++k) {
        // every wave is past P.V of tile k - 1, so stage (k + 1) & 1 can take tile k + 1: its DMA
        // is spread over this tile's Q.K^T steps, which the memory stream then paces (measured
        // slightly faster than issuing tile 1 whole right after the q staging)
        if (k >= 1) __syncthreads();
        const SliceDma dn = ss.plan((k + 1) & 1, k + 1);
        const int par = k & 1;
        const char * sb = ring + ss.stage_off(par, w);
        const int kbase = (ss.t0 + k) * TK + WK * w;
        f32x4 s0, s1;
        if (k + 1 < n_my) qk_slice<DK, true>(ss, dn, sb, lane, qreg, s0, s1);
        else qk_slice<DK, false>(ss, dn, sb, lane, qreg, s0, s1);
        float sc[2][4], mx[2];
        slice_scores(a, slice_mask<DK>(sb, lane), kbase, lane, s0, s1, sc, mx);
        // P against the current reference (exact unless the reference moves below; the clamp only
        // keeps a provisional value finite), into the exchange as [32 heads][64 keys]
        half_t * pxv = px[par];
        auto put_p = [&]() {
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                half4 ph;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ph[r] = to_half(exp2_fast(fminf(sc[n][r] - m_ref[n], 15.0f)));     // masked: 2^-inf = 0
                *reinterpret_cast<half4 *>(&pxv[(16 * n + j16) * C::PROW + WK * w + 4 * g]) = ph;
            }
        };
        put_p();
        if (lane < 16) {
            red[par][lane][w] = mx[0];
            red[par][16 + lane][w] = mx[1];
        }
        __syncthreads();
        // the tile's max per head; every wave reads the same values and holds the same reference,
        // so the decision below is uniform over the workgroup
        bool move = false;
        float tm[2];
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const f32x4 r4 = *reinterpret_cast<const f32x4 *>(&red[par][16 * n + j16][0]);
            tm[n] = fmaxf(fmaxf(r4[0], r4[1]), fmaxf(r4[2], r4[3]));
            move |= ref_moves(m_ref[n], tm[n]);
        }
        if (__builtin_amdgcn_ballot_w64(move) != 0) {     // rare: move the reference, rescale, redo P
            float al[2];
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const bool mv = ref_moves(m_ref[n], tm[n]);
                al[n] = !mv ? 1.0f : exp2_fast(m_ref[n] - tm[n]);      // 0 from M_NONE
                m_ref[n] = mv ? tm[n] : m_ref[n];
            }
            l_acc *= al[(lane >> 4) & 1];         // this lane's head is 16 ((lane >> 4) & 1) + j16
            if (k > 0) {                          // (on the first tile the accumulators are still 0)
                // every accumulator column is this lane's head: one factor per lane.  In place on
                // the accumulator registers, one asm block per element, so that they stay in AGPRs
                // across this branch; the s_nops cover the MFMA -> VALU read distance.
                const float a_own = al[(lane >> 4) & 1];
                asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
                for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float tmp;
                        asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                                     : "+a"(o[i][r]), "=&v"(tmp) : "v"(a_own));
                    }
                asm volatile("s_nop 7" ::: "memory");
            }
            put_p();
            __syncthreads();
        }

        pv_tile<DK, DV>(ring, pxv, par, w, lane, pv, o, l_acc);
    }
    wait_vm<0>();                            // nothing of this wave may still target the ring

    // staging: this wave's slot of the stage the last tile did not use (no wave reads it any more:
    // the last tile's loop-top barrier follows every P.V of the one before)
    decode_epilogue<DK, DV>(a, ring + stage_byte<DK>(n_my & 1, w), w, tid, t, hg0, sp, o, l_acc, m_ref);
}

// ROWS = false: row blockIdx.z (one token, the plain decode step).  ROWS = true: rows blockIdx.z,
// blockIdx.z + gridDim.z, ... of split blockIdx.x (batch-of-N decode puts every row of the split in
// one workgroup); with a mask, the rows that hold no live key of the split (per-sequence regions)
// are found first, in one round trip, and only record an empty split; the others run the whole
// pass in turn.
template <int DK, int DV, bool ROWS>
__global__ __launch_bounds__(NTHR, 1) void kqkv_decode_f16_kernel(DecodeArgs a) {
    __shared__ DecodeLds<DK, DV> sh;
    if constexpr (!ROWS) {
        decode_row<DK, DV>(a, blockIdx.z, sh);
        return;
    }
    __shared__ uint32_t live_w[NWAVE];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t live = ~0u;
    if (a.nt > 1 && a.dst == nullptr && a.mask != nullptr) {
        const uint32_t bits = live_rows_of_wave<LIVE_ROUND_TILES>(a, blockIdx.x, w, lane);
        if (lane == 0) live_w[w] = bits;
        __syncthreads();
        live = live_w[0] | live_w[1] | live_w[2] | live_w[3];
    }
    int i = 0;
    for (int t = blockIdx.z; t < a.nt; t += gridDim.z, ++i) {
        if (!((live >> i) & 1u)) {
            if (w == 0) write_empty_pairs(a, blockIdx.y, t, blockIdx.x, DV, lane);
            continue;
        }
        decode_row<DK, DV>(a, t, sh);
        __syncthreads();                     // the next row's q staging reuses the ring
    }
}

}  // namespace

template <int DK, int DV>
static hipError_t launch_decode(const DecodeArgs & a, int n_hgroups, hipStream_t stream) {
    if (a.nt == 1)
        hipLaunchKernelGGL((kqkv_decode_f16_kernel<DK, DV, false>), dim3(a.n_split, n_hgroups, 1), dim3(NTHR), 0, stream, a);
    else
        hipLaunchKernelGGL((kqkv_decode_f16_kernel<DK, DV, true>), dim3(a.n_split, n_hgroups, decode_row_groups(a, n_hgroups)),
                           dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kqkv_decode_f16(int dk, int dv, const DecodeArgs & a, hipStream_t stream) {
    const int n_hgroups = (a.n_head + decode::HG - 1) / decode::HG;
    if (dk == 576 && dv == 512) return launch_decode<576, 512>(a, n_hgroups, stream);
    if (dk == 320 && dv == 256) return launch_decode<320, 256>(a, n_hgroups, stream);
    return hipErrorInvalidValue;
}

bool decode_f16_supported(int dk, int dv) {
    return (dk == 576 && dv == 512) || (dk == 320 && dv == 256);
}

}  // namespace mla

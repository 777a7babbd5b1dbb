// kqkv_decode.hip -- split-K MLA decode attention over an f16 latent+rope KV cache, on MFMA.
//
// The pass-1 kernel of GGML_OP_M4_KQKV (reference: patches/ggml-m4/m4-kqkv.cu:201-312), designed
// for gfx950 rather than translated:
//   * ALL heads of a 32-head group live in one workgroup, so every KV byte is fetched from HBM
//     exactly once per token (MLA's single latent row serves every head).
//   * Q.K^T and P.V are dense contractions ([32 x D_k].[D_k x keys] and [32 x keys].[keys x D_v],
//     60 FLOP per cache byte): they run on v_mfma_f32_16x16x32_f16 / v_mfma_f32_32x32x16_f16 with
//     f32 accumulation.  q and P enter the MFMA as f16 -- the same rounding points as the unfused
//     ggml-cpu graph, whose mul_mat converts src1 to F16 for an F16 src0.
//   * Work split of a 64-key tile over the 4 waves (one per SIMD): for Q.K^T wave w owns keys
//     16 w .. 16 w + 15 against all 32 heads (q fragments held in VGPRs); for P.V wave w owns the
//     output columns D_v/4 * w .. + D_v/4 against all 64 keys (accumulators in AGPRs).  P moves
//     between the two through a 4.5 KB LDS exchange, the only workgroup barrier per tile.
//   * Each wave's key slices stream into a two-stage LDS ring by bounds-checked LDS DMA
//     (buffer_load_dwordx4 ... lds: no staging registers, keys past n_kv read as zeros).  The stage
//     layout (below) makes the Q.K^T operand reads and the transposed V reads (ds_read_b64_tr_b16)
//     bank-conflict free and each a lane-invariant base plus an immediate offset.
//   * Online softmax in log2 units (v_exp_f32) against a reference max shared by the waves and
//     moved lazily: only when a tile raises a head's max by more than 2^8, so P = exp2(s - m_ref)
//     <= 256 (exact range in f16) and the accumulator rescale is rare.  P is computed against the
//     current reference before the barrier and recomputed after it only when the reference moves.
//
// Grid = (n_split, ceil(H/32), nt), 256 threads.  Output: one partial block per (32-head group,
// token, split) -- m (the split's exact max) and l per head in f32 and the split's normalised
// output o/l in f16, [32 heads][D_v] (mla_kernels.h) -- or, with a single split, o/l in f32 to dst.
#include <type_traits>

#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

constexpr int TK = 64;          // keys per split tile (splits are whole tiles)
constexpr int NWAVE = 4;
constexpr int NTHR = 64 * NWAVE;
constexpr int WK = TK / NWAVE;  // keys per wave slice
constexpr int HG = 32;          // heads per workgroup
constexpr float LAZY = 8.0f;    // log2 slack before the reference max moves

template <int DK, int DV>
struct DecodeCfg {
    static_assert(DK % 64 == 0 && DV % 128 == 0 && DV <= DK, "geometry");
    static constexpr int CH = DK * 2 / 16;              // 16-byte chunks per cache row
    static_assert(CH % 4 == 0, "1 KB stage blocks of 4 chunks x 16 rows");
    static constexpr int DMA_N = WK * CH / 64;          // 16-byte DMA instructions per slice
    static constexpr int ROWS_BYTES = WK * DK * 2;
    static constexpr int STAGE = ROWS_BYTES + 256;      // 16 K rows + the mask slot
    static constexpr int RING = 2 * NWAVE * STAGE;
    static constexpr int QSTEPS = DK / 32;              // K-steps of the 16x16x32 MFMA
    static constexpr int DVQ = DV / NWAVE;              // output columns per wave
    static constexpr int NTQ = DVQ / 32;                // 32-column output tiles per wave
    static constexpr int QC = DK / 4;                   // 16-byte f32 chunks per q row
    static constexpr int QD = HG * QC / 64 / NWAVE;     // q DMA instructions per wave
    static constexpr int PROW = TK + 8;                 // P exchange row pitch (halves)
    static constexpr int OREG = DVQ * HG * 2;           // a wave's f16 [DVQ][32 heads] output region
    static constexpr int OPT = HG * DVQ / 8 / 64;       // 16-byte output chunks per lane
    static_assert(QC % 16 == 0 && (HG * QC) % (64 * NWAVE) == 0, "q staging swizzle, whole q DMA instructions");
    static_assert(HG * DK * 4 <= NWAVE * STAGE, "the f32 q staging fits stage 1 of the ring");
    static_assert(NWAVE * OREG <= RING, "the output regions fit the ring");
    static_assert((NWAVE - 1) * STAGE + 1024 * NTQ < 65536, "P.V operand offsets fit the DS immediate");
};

// Stage layout (one wave slice, 16 cache rows): 1 KB blocks i = 0 .. CH/4 - 1, block i holding chunks
// 4 i .. 4 i + 3 (16 bytes each) of the 16 rows, chunk 4 i + q of row r at slot 16 q + (r ^ 4 q).
// DMA instruction i fills block i, lane l fetching row (l & 15) ^ 4 (l >> 4), chunk 4 i + (l >> 4),
// so its global offset is lane-only plus 64 i.  The XOR keeps the Q.K^T reads (16 rows, one chunk)
// and the transpose reads (4 rows x 4 chunks per 32 lanes) on distinct banks, at 128 or 256 bytes
// per LDS clock alike.
__device__ __forceinline__ int slot_of(int r, int q) { return 16 * q + (r ^ (4 * q)); }

// Unit swizzle of the output regions ([DVQ rows][32 heads] f16, rows of 8 8-byte units): unit u of
// row dv sits at slot u ^ ounit(dv), ounit = 4 b1 ^ b2 ^ 6 b3 ^ 2 b4 (b_i = bit i of dv).  The
// stores (32 consecutive rows, one unit) and the transpose reads (4 rows x 4 units per 16 lanes,
// rows 8 apart across 16-lane pairs) then hit distinct banks at 128 or 256 bytes per LDS clock.
__device__ __forceinline__ int ounit(int dv) {
    return (((dv >> 1) & 1) << 2) ^ ((dv >> 2) & 1) ^ (((dv >> 3) & 1) * 6) ^ (((dv >> 4) & 1) << 1);
}

template <int DK, int DV>
__global__ __launch_bounds__(NTHR, 1) void kqkv_decode_f16_kernel(DecodeArgs a) {
    using C = DecodeCfg<DK, DV>;
    __shared__ __attribute__((aligned(16))) char ring[C::RING];          // [stage][wave] K rows + mask
    __shared__ __attribute__((aligned(16))) half_t px[2][HG * C::PROW];  // P exchange, by tile parity
    __shared__ __attribute__((aligned(16))) float red[2][HG][NWAVE];     // slice maxima [head][wave], by tile parity
    __shared__ float fin_t[NWAVE][HG];
    __shared__ float fin_l[NWAVE][HG];
    __shared__ float fin_r[HG];
    __shared__ __attribute__((aligned(16))) float inv_l[HG];
    __shared__ float hdr[2 * HG];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int t = blockIdx.z;
    const int g = lane >> 4;                 // 16-lane group
    const int j16 = lane & 15;

    // ---- split range (balanced partition of whole 64-key tiles) ----
    const int base_t = a.n_tiles / a.n_split;
    const int rem = a.n_tiles % a.n_split;
    const int t0 = sp * base_t + min(sp, rem);
    const int n_my = base_t + (sp < rem ? 1 : 0);

    const bool has_mask = a.mask != nullptr;
    const float * mrow = has_mask ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1) : a.q;

    // ---- DMA of this wave's 16-key slice of tile k into stage s: DMA_N + 1 loads ----
    // The resources are rebased on the slice, num_records = bytes up to the end of row n_kv - 1,
    // so rows (and mask entries) at or past n_kv are returned as zeros by the range check.
    const uint32_t ring_lds = lds_addr(ring);
    auto stage_off = [&](int s, int v) { return (s * NWAVE + v) * C::STAGE; };
    const uint32_t kvoff = (uint32_t)(((lane & 15) ^ (4 * (lane >> 4))) * a.kc_nb1) + 16u * (uint32_t)(lane >> 4);
    const uint32_t mvoff = 4u * (uint32_t)j16;
    struct SliceDma { i32x4 krs, mrs; uint32_t sb; };
    auto plan = [&](int s, int k) {
        const int tile = min(t0 + min(k, n_my - 1), a.n_tiles - 1);
        const int key0 = tile * TK + WK * w;
        const int left = a.n_kv - key0;                  // rows of this slice that exist (may be <= 0)
        SliceDma d;
        d.krs = make_rsrc(a.kc + (int64_t)key0 * a.kc_nb1, left > 0 ? (uint32_t)((int64_t)(left - 1) * a.kc_nb1 + DK * 2) : 0u);
        d.mrs = make_rsrc(mrow + key0, (has_mask && left > 0) ? (uint32_t)left * 4u : 0u);
        d.sb = ring_lds + (uint32_t)stage_off(s, w);
        return d;
    };
    // instruction i < DMA_N: block i of the rows; i == DMA_N: the mask slot (float l = key key0 + (l & 15))
    auto put = [&](const SliceDma & d, int i) {
        if (i < C::DMA_N) dma16_nt(d.krs, kvoff, (uint32_t)(64 * i), d.sb + (uint32_t)(1024 * i));
        else dma4(d.mrs, mvoff, 0u, d.sb + (uint32_t)C::ROWS_BYTES);
    };

    // ---- q block (32 heads x DK f32) -> stage 1 by DMA, then f16 B fragments in registers ----
    // Staging slot of f32 chunk c (4 floats) of head h: h * QC + (c ^ (h & 15)), so the fragment
    // reads below (16 heads, one chunk) hit distinct banks.  The q DMA goes first and tile 0
    // streams behind it; heads past n_head read as zeros.
    {
        const int nh = min(HG, a.n_head - hg0);
        const i32x4 qrs = make_rsrc(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 + (size_t)hg0 * a.q_nb1,
                                    (uint32_t)((int64_t)(nh - 1) * a.q_nb1 + DK * 4));
        const uint32_t qsb = ring_lds + (uint32_t)(NWAVE * C::STAGE);
#pragma unroll
        for (int i = 0; i < C::QD; ++i) {
            const int p = (w * C::QD + i) * 64 + lane;
            const int h = p / C::QC;
            const int c = (p - h * C::QC) ^ (h & 15);
            dma16(qrs, (uint32_t)(h * a.q_nb1) + 16u * (uint32_t)c, 0u, qsb + (uint32_t)((w * C::QD + i) * 1024));
        }
        const SliceDma d0 = plan(0, 0);
#pragma unroll
        for (int i = 0; i <= C::DMA_N; ++i) put(d0, i);
    }
    wait_vm<C::DMA_N + 1>();                 // this wave's part of q has landed
    __syncthreads();
    half8 qreg[2][C::QSTEPS];   // [head tile n][step s]: head 16 n + j16, d = 32 s + 8 g .. +7
    {
        // reads in batches of QB fragments ahead of their conversion (a read-convert chain per
        // fragment would serialise on the LDS latency)
        constexpr int QB = C::QSTEPS % 6 == 0 ? 6 : (C::QSTEPS % 5 == 0 ? 5 : 2);
        static_assert(C::QSTEPS % QB == 0, "whole batches");
        const float * qs = reinterpret_cast<const float *>(ring + NWAVE * C::STAGE);
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const float * row = qs + 4 * (16 * n + j16) * C::QC;
#pragma unroll
            for (int s0 = 0; s0 < C::QSTEPS; s0 += QB) {
                f32x4 x[QB][2];
#pragma unroll
                for (int b = 0; b < QB; ++b) {
                    x[b][0] = *reinterpret_cast<const f32x4 *>(row + 4 * ((8 * (s0 + b) + 2 * g) ^ j16));
                    x[b][1] = *reinterpret_cast<const f32x4 *>(row + 4 * ((8 * (s0 + b) + 2 * g + 1) ^ j16));
                }
#pragma unroll
                for (int b = 0; b < QB; ++b) {
                    half8 h = {to_half(x[b][0][0]), to_half(x[b][0][1]), to_half(x[b][0][2]), to_half(x[b][0][3]),
                               to_half(x[b][1][0]), to_half(x[b][1][1]), to_half(x[b][1][2]), to_half(x[b][1][3])};
                    // materialise the f16 fragment here: left alone, the compiler keeps the f32
                    // values (twice the registers) and re-converts them at every use in the loop
                    asm volatile("" : "+v"(h));
                    qreg[n][s0 + b] = h;
                }
            }
        }
    }
    __syncthreads();                         // the q staging in stage 1 is free again

    // ---- running state: reference max identical in every wave; l and exact max of own keys ----
    float m_ref[2] = {-INFINITY, -INFINITY}; // heads 16 n + j16, log2 units
    float m_top[2] = {-INFINITY, -INFINITY};
    float l_part[2] = {0.0f, 0.0f};
    f32x16 o[C::NTQ];                        // tile i: C row = head, C col = column DVQ w + 32 i + (lane & 31)
#pragma unroll
    for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;

    // P.V operand addresses: A = P rows (lane & 31), keys 16 ks + 8 (lane >> 5); B = two transpose
    // reads per tile, in 16-lane group g lane j supplying row 8 (g >> 1) + (j >> 2) (then + 4) of key
    // slice ks, 4 columns at DVQ w + 32 i + 16 (g & 1) + 4 (j & 3)
    const int pv_r0 = 8 * (g >> 1) + (j16 >> 2);
    const int pv_cq = 2 * (g & 1) + ((j16 & 3) >> 1);
    const int pv_lo = 16 * slot_of(pv_r0, pv_cq) + 8 * (j16 & 1) + 1024 * (C::NTQ * w);
    const int pv_hi = 16 * slot_of(pv_r0 + 4, pv_cq) + 8 * (j16 & 1) + 1024 * (C::NTQ * w);

    for (int k = 0; k < n_my; ++k) {
        wait_vm<0>();                        // this wave's slice of tile k has landed
        // every wave is past P.V of tile k - 1, so stage (k + 1) & 1 can take tile k + 1: its DMA
        // is spread over this tile's Q.K^T steps, which the memory stream then paces
        if (k >= 1) __syncthreads();
        const bool pf = k + 1 < n_my;
        const SliceDma dn = plan((k + 1) & 1, k + 1);
        const int par = k & 1;
        const char * sb = ring + stage_off(par, w);
        const int kbase = (t0 + k) * TK + WK * w;

        // S^T = K . Q^T : the wave's 16 keys (C rows) x 32 heads (C cols, two 16-wide tiles)
        // two accumulator chains per head tile (even / odd K-steps), so consecutive MFMAs never
        // wait on each other's result
        f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
        f32x4 acc2 = {0.f, 0.f, 0.f, 0.f}, acc3 = {0.f, 0.f, 0.f, 0.f};
        // operand reads run QPF steps ahead of the MFMAs that consume them; the scheduling
        // barriers keep the compiler from sinking them back next to their use.  Two copies of the
        // loop (with and without the next tile's DMA) keep branches out of the steps.
        auto qk = [&](auto with_dma) {
            constexpr int QPF = 4;
            const char * abase = sb + 16 * slot_of(j16, g);     // row j16, chunk 4 s + g of block s
            half8 abuf[QPF];
#pragma unroll
            for (int s = 0; s < QPF; ++s) abuf[s] = *reinterpret_cast<const half8 *>(abase + 1024 * s);
#pragma unroll
            for (int s = 0; s < C::QSTEPS; ++s) {
                const half8 av = abuf[s % QPF];
                if (s + QPF < C::QSTEPS) abuf[s % QPF] = *reinterpret_cast<const half8 *>(abase + 1024 * (s + QPF));
                if (s & 1) {
                    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[0][s], acc2, 0, 0, 0);
                    acc3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[1][s], acc3, 0, 0, 0);
                } else {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[0][s], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[1][s], acc1, 0, 0, 0);
                }
                if constexpr (decltype(with_dma)::value)
                    if (s <= C::DMA_N) put(dn, s);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (decltype(with_dma)::value) {
#pragma unroll
                for (int i = C::QSTEPS; i <= C::DMA_N; ++i) put(dn, i);
            }
        };
        if (pf) qk(std::true_type{}); else qk(std::false_type{});
        acc0 += acc2;
        acc1 += acc3;
        // scores (log2 units) of keys 4 g + r for heads j16 (n = 0) and 16 + j16 (n = 1)
        const f32x4 mk = *reinterpret_cast<const f32x4 *>(sb + C::ROWS_BYTES + 16 * g);
        float sc[2][4];
        float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool live = kbase + 4 * g + r < a.n_kv;
            const float mb = mk[r] * LOG2E;              // zeros when there is no mask
            sc[0][r] = live ? acc0[r] * a.scale_log2 + mb : -INFINITY;
            sc[1][r] = live ? acc1[r] * a.scale_log2 + mb : -INFINITY;
            mx[0] = fmaxf(mx[0], sc[0][r]);
            mx[1] = fmaxf(mx[1], sc[1][r]);
        }
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            mx[n] = fmaxf(mx[n], shfl_xor(mx[n], 16));
            mx[n] = fmaxf(mx[n], shfl_xor(mx[n], 32));
            m_top[n] = fmaxf(m_top[n], mx[n]);
        }
        // P against the current reference (exact unless the reference moves below; the clamp only
        // keeps a provisional value finite), into the exchange as [32 heads][64 keys]
        half_t * pxv = px[par];
        float p[2][4];
        auto put_p = [&]() {
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                half4 ph;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[n][r] = (sc[n][r] == -INFINITY) ? 0.0f : exp2_fast(fminf(sc[n][r] - m_ref[n], 15.0f));
                    ph[r] = to_half(p[n][r]);
                }
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
            move |= (m_ref[n] == -INFINITY) ? (tm[n] != -INFINITY) : (tm[n] > m_ref[n] + LAZY);
        }
        if (__builtin_amdgcn_ballot_w64(move) != 0) {     // rare: move the reference, rescale, redo P
            float al[2];
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const bool mv = (m_ref[n] == -INFINITY) ? (tm[n] != -INFINITY) : (tm[n] > m_ref[n] + LAZY);
                al[n] = !mv ? 1.0f : (m_ref[n] == -INFINITY ? 0.0f : exp2_fast(m_ref[n] - tm[n]));
                m_ref[n] = mv ? tm[n] : m_ref[n];
                l_part[n] *= al[n];
            }
            if (k > 0) {                          // (on the first tile the accumulators are still 0)
                // accumulator rows are heads 8 (r / 4) + 4 (lane >> 5) + (r & 3): fetch their
                // factors from the lanes holding them (head h's in lane h & 15 of set n = h >> 4)
                f32x16 al16;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int h = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const float a0 = __shfl(al[0], h & 15, 64), a1 = __shfl(al[1], h & 15, 64);
                    al16[r] = (h >> 4) ? a1 : a0;
                }
                // In place on the accumulator registers, one asm block per element, so that they
                // stay in AGPRs across this branch (a plain multiply makes the register allocator
                // move the tile set through VGPRs).  The s_nops cover the MFMA -> VALU read distance.
                asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
                for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float tmp;
                        asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                                     : "+a"(o[i][r]), "=&v"(tmp) : "v"(al16[r]));
                    }
                asm volatile("s_nop 7" ::: "memory");
            }
            put_p();
            __syncthreads();
        }
#pragma unroll
        for (int n = 0; n < 2; ++n) l_part[n] += (p[n][0] + p[n][1]) + (p[n][2] + p[n][3]);

        // O[:, own columns] += P . V over the tile's 64 keys (4 slices x 16); the operands of
        // slice ks + 1 are read while the MFMAs of slice ks run
        {
            half8 pa[2], vb[2][C::NTQ];
            auto load = [&](int ks, int b) {
                pa[b] = *reinterpret_cast<const half8 *>(&pxv[(lane & 31) * C::PROW + WK * ks + 8 * (lane >> 5)]);
                const char * vs = ring + stage_off(par, ks);
#pragma unroll
                for (int i = 0; i < C::NTQ; ++i) {
                    const half4 lo = lds_read_tr16(reinterpret_cast<const half_t *>(vs + pv_lo + 1024 * i));
                    const half4 hi = lds_read_tr16(reinterpret_cast<const half_t *>(vs + pv_hi + 1024 * i));
                    vb[b][i] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            };
            load(0, 0);
#pragma unroll
            for (int ks = 0; ks < NWAVE; ++ks) {
                if (ks + 1 < NWAVE) load(ks + 1, (ks + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < C::NTQ; ++i)
                    o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[ks & 1], vb[ks & 1][i], o[i], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    wait_vm<0>();                            // nothing of this wave may still target the ring

    // thread indices re-derived through an opaque move, so that the epilogue's address arithmetic
    // is computed here rather than before the loop and kept alive (or spilled) across it
    int tid_e;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid_e) : "v"(tid));
    const int lane_e = tid_e & 63;

    // ---- per head: M = exact max over the waves, L = sum of the waves' l (common reference) ----
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        l_part[n] += shfl_xor(l_part[n], 16);
        l_part[n] += shfl_xor(l_part[n], 32);
    }
    if (lane_e < 16) {
        fin_t[w][lane_e] = m_top[0];
        fin_t[w][16 + lane_e] = m_top[1];
        fin_l[w][lane_e] = l_part[0];
        fin_l[w][16 + lane_e] = l_part[1];
        if (w == 0) {
            fin_r[lane_e] = m_ref[0];
            fin_r[16 + lane_e] = m_ref[1];
        }
    }
    __syncthreads();
    if (tid_e < HG) {
        float M = -INFINITY, L = 0.0f;
#pragma unroll
        for (int v = 0; v < NWAVE; ++v) {
            M = fmaxf(M, fin_t[v][tid_e]);
            L += fin_l[v][tid_e];
        }
        inv_l[tid_e] = L > 0.0f ? 1.0f / L : 0.0f;
        hdr[tid_e] = (M == -INFINITY) ? -INFINITY : M * LN2;                        // natural-log units
        hdr[HG + tid_e] = L > 0.0f ? L * exp2_fast(fin_r[tid_e] - M) : 0.0f;       // relative to M
    }
    __syncthreads();

    const bool direct = a.dst != nullptr;                 // single split: final f32 output to dst
    if (direct) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4 s4 = *reinterpret_cast<const f32x4 *>(&inv_l[8 * q4 + 4 * (lane_e >> 5)]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int h = hg0 + 8 * q4 + 4 * (lane_e >> 5) + e;
                if (h < a.n_head) {
                    float * d = a.dst + ((size_t)h * a.nt + t) * DV + C::DVQ * w + (lane_e & 31);
#pragma unroll
                    for (int i = 0; i < C::NTQ; ++i) d[32 * i] = o[i][4 * q4 + e] * s4[e];
                }
            }
        }
        return;
    }
    // o / l in f16 into this wave's region of the (idle) ring, [DVQ rows][32 heads], then read back
    // transposed into [32 heads][D_v] chunks of 8 columns
    char * reg = ring + w * C::OREG;
    {
        const int dvl = lane_e & 31, hi32 = lane_e >> 5;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4 s4 = *reinterpret_cast<const f32x4 *>(&inv_l[8 * q4 + 4 * hi32]);
#pragma unroll
            for (int i = 0; i < C::NTQ; ++i) {
                const int dv = 32 * i + dvl;
                half4 hv;
                hv[0] = to_half(o[i][4 * q4 + 0] * s4[0]);
                hv[1] = to_half(o[i][4 * q4 + 1] * s4[1]);
                hv[2] = to_half(o[i][4 * q4 + 2] * s4[2]);
                hv[3] = to_half(o[i][4 * q4 + 3] * s4[3]);
                *reinterpret_cast<half4 *>(reg + dv * 64 + 8 * ((2 * q4 + hi32) ^ ounit(dv))) = hv;
            }
        }
    }
    __syncthreads();
    char * blk = a.part + (((size_t)blockIdx.y * a.nt + t) * a.n_split + sp) * part_block_bytes(DV, 2);
    if (tid_e < 2 * HG) reinterpret_cast<float *>(blk)[tid_e] = hdr[tid_e];
    // per 64-chunk group cg: heads 16 hb + (lane & 15), columns 8 (4 (cg >> 1) + (lane >> 4)) .. +7
    const int ge = lane_e >> 4, je = lane_e & 15;
#pragma unroll
    for (int cg = 0; cg < C::OPT; ++cg) {
        const int hb = cg & 1;
        const int dv8 = 4 * (cg >> 1) + ge;
        const int dv_lo = 8 * dv8 + (je >> 2), dv_hi = dv_lo + 4;
        const int u = 4 * hb + (je & 3);
        const half4 lo = lds_read_tr16(reinterpret_cast<const half_t *>(reg + dv_lo * 64 + 8 * (u ^ ounit(dv_lo))));
        const half4 hi = lds_read_tr16(reinterpret_cast<const half_t *>(reg + dv_hi * 64 + 8 * (u ^ ounit(dv_hi))));
        const half8 hv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, hv),
                                    reinterpret_cast<u32x4 *>(blk + 256 + ((size_t)(16 * hb + je) * DV + C::DVQ * w + 8 * dv8) * 2));
    }
}

}  // namespace

template <int DK, int DV>
static hipError_t launch_decode(const DecodeArgs & a, int n_hgroups, hipStream_t stream) {
    dim3 grid(a.n_split, n_hgroups, a.nt);
    hipLaunchKernelGGL((kqkv_decode_f16_kernel<DK, DV>), grid, dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kqkv_decode_f16(int dk, int dv, const DecodeArgs & a, hipStream_t stream) {
    const int n_hgroups = (a.n_head + HG - 1) / HG;
    if (dk == 576 && dv == 512) return launch_decode<576, 512>(a, n_hgroups, stream);
    if (dk == 320 && dv == 256) return launch_decode<320, 256>(a, n_hgroups, stream);
    return hipErrorInvalidValue;
}

bool decode_f16_supported(int dk, int dv) {
    return (dk == 576 && dv == 512) || (dk == 320 && dv == 256);
}

}  // namespace mla

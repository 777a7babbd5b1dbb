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
//   * The cache streams through 64-key tiles: coalesced 16-byte nontemporal loads into a register
//     double buffer keep tiles i+1 and i+2 in flight while tile i is computed out of LDS (rows
//     padded by 16 bytes so the MFMA operand reads are bank-conflict free).
//   * LDS traffic is the per-tile cost that matters, so every tile byte is read from LDS once by
//     Q.K^T: the contraction over D_k is split between two waves (each holds the f16 q fragments
//     of its D_k half for all 32 heads in registers), and the two half-scores are summed through a
//     1 KB-per-wave exchange.
//   * Online softmax in log2 units (v_exp_f32), rescaling the accumulators only by the per-tile
//     factor; all-masked prefixes are guarded (no exp(-inf - -inf)).
//
// Work split: grid = (n_split, ceil(H/32), nt), 256 threads = 4 waves, one per SIMD, so each wave
// has the whole 512-entry register file (q fragments, two in-flight tiles, output accumulators).
//   QK role:   wave w -> keys [32 kg, 32 kg + 32) (kg = w & 1) x all 32 heads over the D_k half
//              dh = w >> 1; afterwards the wave owns the scores of head tile dh for its 32 keys
//   PV role:   wave w -> output columns [w*D_v/4, (w+1)*D_v/4), all 32 heads
// Output: one partial block per (32-head group, token, split) -- m and l per head in f32 and the
// split's normalised output o/l in f16 (see mla_kernels.h) -- or, when the launch has a single
// split, the final o/l in f32 written to dst.
#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

constexpr int TK = 64;          // keys per tile
constexpr int NWAVE = 4;        // one wavefront per SIMD: the 512-entry register file per lane
constexpr int NTHR = 64 * NWAVE;
constexpr int HG = 32;          // heads per workgroup

template <int DK, int DV>
struct DecodeCfg {
    static_assert(DK % 64 == 0 && DV % 256 == 0 && DV <= DK, "geometry");
    static constexpr int KROW = DK + 8;                 // LDS row pitch in halves (+16 bytes)
    static constexpr int CH = DK * 2 / 16;              // 16-byte chunks per cache row
    static constexpr int NCHUNK = TK * CH;
    static constexpr int NPT = NCHUNK / NTHR;           // staged chunks per thread per tile
    static constexpr int QCH = HG * DK / 4;             // 16-byte f32 chunks of the WG's q block
    static constexpr int QPT = QCH / NTHR;              // q chunks per thread
    static constexpr int HSTEPS = DK / 64;              // 16x16x32 K-steps per D_k half
    static constexpr int DVW = DV / NWAVE;              // output columns per wave
    static constexpr int NT_DV = DVW / 32;              // 32-wide MFMA tiles per wave
    static constexpr int PROW = TK + 8;                 // P row pitch in halves
    static constexpr int OCH = HG * DV / 8;             // 16-byte f16 chunks of the WG's output block
    static constexpr int OPT = OCH / NTHR;
    static_assert(NCHUNK % NTHR == 0 && QCH % NTHR == 0 && OCH % NTHR == 0, "whole chunks per thread");
    static_assert(HG * DV * 2 <= TK * KROW * 2, "f16 output block fits the tile buffer");
};

template <int DK, int DV>
__global__ __launch_bounds__(NTHR, 1) void kqkv_decode_f16_kernel(DecodeArgs a) {
    using C = DecodeCfg<DK, DV>;
    __shared__ __attribute__((aligned(16))) half_t kt[TK * C::KROW];     // the current tile; the output block at the end
    __shared__ __attribute__((aligned(16))) half_t qs[HG * C::KROW];     // f16 q block [32 heads][DK] (prologue)
    __shared__ __attribute__((aligned(16))) half_t pl[HG * C::PROW];     // P [32 heads][64 keys]
    __shared__ __attribute__((aligned(16))) f32x4 sx[NWAVE][2][64];      // half-score exchange
    __shared__ __attribute__((aligned(16))) float mk[TK];              // the tile's mask values
    __shared__ float red_max[2][HG];
    __shared__ float red_sum[2][HG];
    __shared__ __attribute__((aligned(16))) float alpha_s[HG];
    __shared__ float l_fin[HG];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int t = blockIdx.z;

    // ---- split range (balanced partition of whole tiles) ----
    const int base_t = a.n_tiles / a.n_split;
    const int rem = a.n_tiles % a.n_split;
    const int t0 = sp * base_t + min(sp, rem);
    const int t1 = t0 + base_t + (sp < rem ? 1 : 0);

    const int kg = w & 1;                          // keys [32 kg, 32 kg + 32) of the tile
    const int dh = w >> 1;                         // QK: D_k half; softmax: head tile
    const int kl0 = 32 * kg + 4 * (lane >> 4);     // lane's score keys: kl0 + 16 m + r (m < 2, r < 4)
    const int hl = 16 * dh + (lane & 15);          // this lane's score head (workgroup-local)
    // no branch may guard a tile load: the compiler's wait counts are exact only when every path
    // issues the same loads, so a missing mask reads q's (valid) memory and is zeroed after the load
    const bool has_mask = a.mask != nullptr;
    const float * mrow = has_mask ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1) : a.q;
    const int n_my = t1 - t0;                                   // tiles of this split
    auto tile_of = [&](int j) { return min(t0 + min(j, n_my - 1), a.n_tiles - 1); };   // clamped, always valid

    // ---- 1. q block of this workgroup (32 heads x DK f32): one coalesced pass, issued first ----
    f32x4 qv[C::QPT];
#pragma unroll
    for (int i = 0; i < C::QPT; ++i) {
        const int c = i * NTHR + tid;
        const int hh = c / (DK / 4);
        const int d4 = c - hh * (DK / 4);
        const int h = min(hg0 + hh, a.n_head - 1);
        const f32x4 x = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 +
                                                       (size_t)h * a.q_nb1 + (size_t)d4 * 16);
        qv[i] = (hg0 + hh < a.n_head) ? x : f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // ---- 2. tile staging: a register double buffer A/B ----
    const uint32_t nb1 = (uint32_t)a.kc_nb1;
    // one mask value per key of the tile rides with the tile (thread t loads key t & 63; it is
    // staged through LDS at commit), so each tile is exactly NPT + 1 loads per thread
    u32x4 stgA[C::NPT], stgB[C::NPT];
    float mskA, mskB;
    auto issue = [&](u32x4 (&stg)[C::NPT], float & msk, int tile) {
        const char * tb = a.kc + (size_t)tile * TK * a.kc_nb1;     // wave-uniform tile base
        const int nk = min(TK, a.n_kv - tile * TK);
        const float mv = mrow[(size_t)(has_mask ? tile * TK : 0) + min(tid & (TK - 1), nk - 1)];
        msk = has_mask ? mv : 0.0f;
#pragma unroll
        for (int i = 0; i < C::NPT; ++i) {
            const int c = i * NTHR + tid;
            const int key = c / C::CH;
            const int cc = c - key * C::CH;
            stg[i] = ld16_stream(tb + (uint32_t)min(key, nk - 1) * nb1 + (uint32_t)cc * 16u);
        }
    };
    // Tile A goes in flight behind q; tile B only after q has been consumed, so that no wait below
    // ever needs more than the hardware's 63 outstanding vector-memory operations (beyond that the
    // compiler's conservative count makes the q conversion wait for both tiles).
    issue(stgA, mskA, tile_of(0));

    // ---- 3. q -> f16 via LDS -> this wave's B fragments: 32 heads x its D_k half ----
#pragma unroll
    for (int i = 0; i < C::QPT; ++i) {
        const int c = i * NTHR + tid;
        const int hh = c / (DK / 4);
        const int d4 = c - hh * (DK / 4);
        half4 h4;
        h4[0] = to_half(qv[i][0]); h4[1] = to_half(qv[i][1]); h4[2] = to_half(qv[i][2]); h4[3] = to_half(qv[i][3]);
        *reinterpret_cast<half4 *>(&qs[hh * C::KROW + 4 * d4]) = h4;
    }
    __syncthreads();
    half8 qreg[2][C::HSTEPS];  // [head tile][step]: head 16 n + (lane & 15), d = 32 (HSTEPS dh + s) + 8 (lane >> 4) .. +7
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        const half_t * qr = &qs[(16 * n + (lane & 15)) * C::KROW + 32 * C::HSTEPS * dh + 8 * (lane >> 4)];
#pragma unroll
        for (int s = 0; s < C::HSTEPS; ++s) qreg[n][s] = *reinterpret_cast<const half8 *>(qr + 32 * s);
    }
    issue(stgB, mskB, tile_of(1));

    // ---- running state: lane tracks head hl (replicated across the 2 key-group waves) ----
    float m_run = -INFINITY;   // log2 units
    float l_run = 0.0f;
    f32x16 o[C::NT_DV];
#pragma unroll
    for (int i = 0; i < C::NT_DV; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;

    auto compute = [&](u32x4 (&stg)[C::NPT], float & msk, int tile, bool refill) {
        __syncthreads();                                  // (A) previous tile's LDS reads done
#pragma unroll
        for (int i = 0; i < C::NPT; ++i) {
            const int c = i * NTHR + tid;
            const int key = c / C::CH;
            const int cc = c - key * C::CH;
            *reinterpret_cast<u32x4 *>(&kt[key * C::KROW + cc * 8]) = stg[i];
        }
        if (tid < TK) mk[tid] = msk;
        if (refill) issue(stg, msk, tile_of(tile - t0 + 2));   // refill this buffer two tiles ahead
        __syncthreads();                                  // (B) tile in LDS

        // half-scores: 32 keys (two 16-key M tiles) x 32 heads over this wave's D_k half; each
        // K chunk is read from LDS once and feeds both head tiles
        f32x4 acc[2][2];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int n = 0; n < 2; ++n) acc[m][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const half_t * arow = &kt[(32 * kg + 16 * m + (lane & 15)) * C::KROW + 32 * C::HSTEPS * dh + 8 * (lane >> 4)];
#pragma unroll
            for (int s = 0; s < C::HSTEPS; ++s) {
                const half8 av = *reinterpret_cast<const half8 *>(arow + 32 * s);
                acc[m][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[0][s], acc[m][0], 0, 0, 0);
                acc[m][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[1][s], acc[m][1], 0, 0, 0);
            }
        }
        // give the partner wave (same keys, other D_k half) the head tile it owns; keep ours
#pragma unroll
        for (int m = 0; m < 2; ++m) sx[w][m][lane] = dh ? acc[m][0] : acc[m][1];
        __syncthreads();                                  // (B2)

        const int kbase = tile * TK;
        float sc[8];
        float lmax = -INFINITY;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const f32x4 full = (dh ? acc[m][1] : acc[m][0]) + sx[w ^ 2][m][lane];
            const f32x4 mv = *reinterpret_cast<const f32x4 *>(&mk[kl0 + 16 * m]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = full[r] * a.scale_log2 + mv[r] * LOG2E;
                sc[4 * m + r] = (kbase + kl0 + 16 * m + r < a.n_kv) ? v : -INFINITY;
                lmax = fmaxf(lmax, sc[4 * m + r]);
            }
        }
        lmax = fmaxf(lmax, shfl_xor(lmax, 16));
        lmax = fmaxf(lmax, shfl_xor(lmax, 32));
        if (lane < 16) red_max[kg][hl] = lmax;
        __syncthreads();                                  // (C)

        const float tmax = fmaxf(red_max[0][hl], red_max[1][hl]);
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = (m_run == -INFINITY) ? 0.0f : exp2_fast(m_run - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            half4 ph;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = sc[4 * m + r];
                const float p = (x == -INFINITY) ? 0.0f : exp2_fast(x - m_new);
                psum += p;
                ph[r] = to_half(p);
            }
            *reinterpret_cast<half4 *>(&pl[hl * C::PROW + kl0 + 16 * m]) = ph;
        }
        psum += shfl_xor(psum, 16);
        psum += shfl_xor(psum, 32);
        if (lane < 16) {
            red_sum[kg][hl] = psum;
            if (kg == 0) alpha_s[hl] = alpha;
        }
        m_run = m_new;
        __syncthreads();                                  // (D)

        l_run = alpha * l_run + (red_sum[0][hl] + red_sum[1][hl]);

        // O[32 heads x DVW] = alpha * O + P . V ; lane's C rows: heads 8 (r/4) + 4 (lane>>5) + (r&3)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const float4 al = *reinterpret_cast<const float4 *>(&alpha_s[8 * q4 + 4 * (lane >> 5)]);
#pragma unroll
            for (int i = 0; i < C::NT_DV; ++i) {
                o[i][4 * q4 + 0] *= al.x;
                o[i][4 * q4 + 1] *= al.y;
                o[i][4 * q4 + 2] *= al.z;
                o[i][4 * q4 + 3] *= al.w;
            }
        }
        // B = V[keys][cols] straight from the row-major tile with the gfx950 transpose read: in each
        // 16-lane group, lane j supplies row (j >> 2), columns 4 (j & 3) .. +3 of a 4 x 16 block and
        // receives column j of it; two reads give the lane its 8 consecutive keys.
        const half_t * vbase = &kt[(8 * (lane >> 5) + ((lane & 15) >> 2)) * C::KROW + w * C::DVW +
                                   16 * ((lane >> 4) & 1) + 4 * (lane & 3)];
#pragma unroll 1
        for (int kk = 0; kk < TK / 16; ++kk) {           // not unrolled: bounds the live operand registers
            const half8 pa = *reinterpret_cast<const half8 *>(&pl[(lane & 31) * C::PROW + 16 * kk + 8 * (lane >> 5)]);
#pragma unroll
            for (int i = 0; i < C::NT_DV; ++i) {
                const half_t * vp = vbase + 16 * kk * C::KROW + 32 * i;
                const half4 lo = lds_read_tr16(vp);
                const half4 hi = lds_read_tr16(vp + 4 * C::KROW);
                const half8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, vb, o[i], 0, 0, 0);
            }
        }
    };

    // steady state: both refills are unconditional (an odd tile count loads one tile twice); the
    // last two tiles are peeled and issue nothing
    int j = 0;
    for (; j + 2 < n_my; j += 2) {
        compute(stgA, mskA, t0 + j, true);
        compute(stgB, mskB, t0 + j + 1, true);
    }
    if (j < n_my) compute(stgA, mskA, t0 + j, false);
    if (j + 1 < n_my) compute(stgB, mskB, t0 + j + 1, false);

    // ---- epilogue: o / l per head -> f16 block in LDS -> 16-byte stores ----
    if (kg == 0 && lane < 16) l_fin[hl] = l_run;
    __syncthreads();                                      // last tile's LDS reads done; l_fin visible
    const bool direct = a.dst != nullptr;                 // single split: final f32 output to dst
    char * blk = direct ? nullptr : a.part + (((size_t)blockIdx.y * a.nt + t) * a.n_split + sp) * part_block_bytes(DV, 2);
    if (!direct && kg == 0 && lane < 16) {
        float * hdr = reinterpret_cast<float *>(blk);
        hdr[hl] = (m_run == -INFINITY) ? -INFINITY : m_run * LN2;
        hdr[PART_HEADS + hl] = l_run;
    }
    half_t * ob = kt;                                     // [HG][DV] f16
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int hloc = 8 * q4 + 4 * (lane >> 5) + r4;
            const float l = l_fin[hloc];
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            const int dv = w * C::DVW + (lane & 31);
            if (direct) {
                if (hg0 + hloc < a.n_head) {
                    float * drow = a.dst + ((size_t)(hg0 + hloc) * a.nt + t) * DV + dv;
#pragma unroll
                    for (int i = 0; i < C::NT_DV; ++i) drow[32 * i] = o[i][4 * q4 + r4] * inv;
                }
            } else {
#pragma unroll
                for (int i = 0; i < C::NT_DV; ++i) ob[hloc * DV + dv + 32 * i] = to_half(o[i][4 * q4 + r4] * inv);
            }
        }
    if (direct) return;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < C::OPT; ++i) {
        const int c = i * NTHR + tid;                     // 16-byte chunk of the [HG][DV] f16 block
        if (hg0 + c / (DV / 8) < a.n_head)
            *reinterpret_cast<u32x4 *>(blk + 256 + (size_t)c * 16) = *reinterpret_cast<const u32x4 *>(&ob[c * 8]);
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

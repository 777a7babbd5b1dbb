// kqkv_decode_q8.hip -- split-K MLA decode attention over an 8-bit latent+rope KV cache (Q8_0).
//
// The cache is ggml's block_q8_0 rows: per 32 values an f16 scale d, then 32 int8 q (34 bytes), a
// row of D_k values D_k / 32 * 34 bytes, rows contiguous; value = q * d.  At D_k = 576 that is 612
// bytes per key (+ 4 of mask) against 1,152 for an f16 cache.  The reference has no cache type but
// F16 (its KQKV asserts it: patches/ggml-m4/m4-kqkv.cu:345); this is the same op over the smaller
// cache, with the partial records and the merge of the f16 path.
//
// Design: the f16 decode kernel's Q.K^T / softmax / P.V (decode_common.h, kqkv_decode.hip) on
// a single f16 tile that the four waves fill by dequantising their slices:
//   * wave w streams its 16-key slice of every tile (16 rows: one contiguous, 16-byte-aligned run)
//     with its 16 mask values into its own slot of a two-stage int8 ring by LDS DMA.  The first two
//     tiles go out right after the q block, so all of a 32K-key split is in flight from the start:
//     unlike the f16 kernel, the q staging does not share LDS with the stream;
//   * per tile: barrier (every wave is past the previous tile's P.V) -> each wave's Q.K^T of its
//     own slice straight from the int8 rows, each MFMA A fragment (8 values of one Q8_0 block)
//     dequantised in registers and also stored into the wave's slot of the f16 tile -> it issues
//     the DMA of tile k + 2 into the int8 slot it has just read -> scores, the maxima exchange (a
//     barrier, after which the whole f16 tile is in place), lazy reference max and P.V (the f16
//     kernel's, on the f16 tile).  The conversion's VALU work runs under the Q.K^T MFMAs of the
//     same wave rather than in a pass of its own;
//   * dequantisation: f16(q * d), the value a conversion of the dequantised f32 to f16 gives (the
//     product q * d is exact in f32, so both round once): each int8 enters f16 exactly as
//     (1024 + (q + 128)) - 1152 (the byte biased by 128 under the f16 bit pattern of 1024, then
//     v_pk_add_f16), times d by v_pk_mul_f16 (one rounding).
// LDS at D_k = 576: int8 ring 2 x 4 x (9,792 + 256) + f16 tile 4 x 18,688 + P exchange 4,608 +
// slice maxima 1,024 = 160,768 bytes.
//
// Grid = (n_split, ceil(H/32), row groups), 256 threads; the rows of a split share its workgroup as
// in kqkv_decode.hip (decode_row_groups), and a row with no live key in the split records an empty
// split.  The output is the f16 path's: partial blocks [group][token][split] with f16 o, or o/l in
// f32 to dst with one split.
#include "decode_common.h"

namespace mla {

namespace {

using namespace decode;

template <int DK>
struct Q8Geom {
    static constexpr int ROWB = DK / 32 * 34;                    // bytes per cache row
    static constexpr int ROWS_BYTES = WK * ROWB;                  // one slice: 16 rows
    static_assert(ROWS_BYTES % 16 == 0 && ROWB % 4 == 0, "16-byte DMA of whole slices");
    static constexpr int SLOT = ROWS_BYTES + 256;                 // rows, then the mask slot
    static constexpr int DMA_FULL = ROWS_BYTES / 1024;            // 64-lane 16-byte instructions
    static constexpr int DMA_TAIL = (ROWS_BYTES % 1024) / 16;     // lanes of the partial last one
    static constexpr int DMA_N = DMA_FULL + (DMA_TAIL ? 1 : 0) + 1;   // + the mask
    static constexpr int HB = DK / 16;                            // 16-value half-blocks per row
    static_assert((WK * HB) % 64 == 0, "whole half-blocks per lane");
    static constexpr int ITEMS = WK * HB / 64;                    // half-blocks per lane
};

template <int DK, int DV>
struct Q8Lds {
    __attribute__((aligned(16))) char ring8[2 * NWAVE * Q8Geom<DK>::SLOT];   // [stage][wave] int8 rows + mask
    __attribute__((aligned(16))) char tile[NWAVE * SliceGeom<DK>::STAGE];    // f16 slices; q staging first
    __attribute__((aligned(16))) half_t px[HG * DecodeCfg<DK, DV>::PROW];
    __attribute__((aligned(16))) float red[2][HG][NWAVE];
    static_assert(HG * DecodeCfg<DK, DV>::OPITCH <= Q8Geom<DK>::SLOT, "the output staging fits a wave's int8 slot");
};

// DMA of wave w's slice of tile k (clamped into the split) into its int8 slot of stage s: the rows as
// linear 16-byte chunks (rows at or past n_kv read as zeros: d = 0, q = 0), then this token's 16 mask
// values (lane l -> key key0 + (l & 15), as the f16 kernels' mask slot).  DMA_N instructions.
template <int DK>
__device__ __forceinline__ void q8_dma(const SliceStream<DK> & ss, uint32_t ring8, int s, int k, int lane) {
    using G8 = Q8Geom<DK>;
    const int tile = min(ss.t0 + min(k, ss.n_my - 1), ss.n_tiles - 1);
    const int key0 = tile * TK + WK * ss.w;
    const int left = ss.n_kv - key0;
    // the rows from key0 to the end of the cache: at most the whole cache, which the contract keeps
    // within 4 GiB (check_kqkv), so the byte count fits the 32-bit range once formed in 64 bits
    const i32x4 krs = make_rsrc(ss.kc + (int64_t)key0 * G8::ROWB, left > 0 ? (uint32_t)((int64_t)left * G8::ROWB) : 0u);
    const uint32_t sb = ring8 + (uint32_t)((s * NWAVE + ss.w) * G8::SLOT);
#pragma unroll
    for (int i = 0; i < G8::DMA_FULL; ++i) dma16_nt(krs, 1024u * (uint32_t)i + 16u * (uint32_t)lane, 0u, sb + 1024u * (uint32_t)i);
    if constexpr (G8::DMA_TAIL != 0) {
        // lanes past the slice stay off (lane 0 is always on, so the instruction is issued and counted)
        if (lane < G8::DMA_TAIL)
            dma16_nt(krs, 1024u * (uint32_t)G8::DMA_FULL + 16u * (uint32_t)lane, 0u, sb + 1024u * (uint32_t)G8::DMA_FULL);
    }
    const i32x4 mrs = make_rsrc(ss.mrow + key0, (ss.has_mask && left > 0) ? (uint32_t)left * 4u : 0u);
    dma4(mrs, 4u * (uint32_t)(lane & 15), 0u, sb + (uint32_t)G8::ROWS_BYTES);
}

// Eight int8 values and their block scale d -> f16(q * d).  w0..w2: the aligned dwords that hold
// the values from byte SH of w0 on (SH = 0: w0, w1 alone).  Each byte enters f16 exactly as
// (1024 + (q + 128)) - 1152 (the byte biased by 128 under the f16 bit pattern of 1024), then one
// multiplication by d rounds once: the value a conversion of the exact f32 product q * d gives.
template <int SH>
__device__ __forceinline__ half8 q8x8_to_f16(uint32_t w0, uint32_t w1, uint32_t w2, half_t d) {
    const half2 bias = {1152.0f16, 1152.0f16};
    const half2 dd = {d, d};
    uint32_t x[2];
    if constexpr (SH == 0) {
        x[0] = w0;
        x[1] = w1;
    } else {
        x[0] = __builtin_amdgcn_alignbyte(w1, w0, SH);
        x[1] = __builtin_amdgcn_alignbyte(w2, w1, SH);
    }
    half8 r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t y = x[k] ^ 0x80808080u;                                   // q + 128 per byte
        const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, y, 0x04010400u);  // bytes 0, 1 under 0x64
        const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, y, 0x04030402u);  // bytes 2, 3 under 0x64
        const half2 a = (__builtin_bit_cast(half2, lo) - bias) * dd;
        const half2 b = (__builtin_bit_cast(half2, hi) - bias) * dd;
        r[4 * k] = a[0];
        r[4 * k + 1] = a[1];
        r[4 * k + 2] = b[0];
        r[4 * k + 3] = b[1];
    }
    return r;
}

// S^T = K . Q^T for the wave's 16 keys, straight from its int8 slice at src (C rows = keys 4 g + r,
// C cols = heads j16 (s0) and 16 + j16 (s1)), dequantising each A fragment in registers: step s is
// Q8_0 block s of every row (D_k / 32 blocks = the K-steps of the 16x16x32 MFMA), lane (j16, g)
// taking values 8 g .. 8 g + 7 of block s of row j16 -- 8 bytes at 34 s + 2 + 8 g of the row, 4-byte
// aligned for odd s, 2 bytes past it for even s (rows are 612 bytes, a multiple of 4) -- and the
// block's scale.  Each converted fragment is also stored to its place in the f16 slot at dst (the
// layout of decode_common.h, slot_byte: chunk 4 s + g of row j16) when P.V reads it (the first D_v
// values of a row: steps s < D_v / 32), after the maxima barrier, so the dequantisation's VALU work
// runs under the Q.K^T MFMAs instead of in a pass of its own.  Operand reads run PF steps ahead of
// their conversion.  Every DMA of the slice has landed.
template <int DK, int DV>
__device__ __forceinline__ void qk_slice_q8(const char * src, char * dst, int lane,
                                            const half8 (&qreg)[2][SliceGeom<DK>::QSTEPS], f32x4 & s0, f32x4 & s1) {
    using G = SliceGeom<DK>;
    using G8 = Q8Geom<DK>;
    static_assert(G::QSTEPS == DK / 32 && G8::ROWB % 4 == 0, "one Q8_0 block per K-step, dword-aligned rows");
    constexpr int PF = 4;
    const int g = lane >> 4, j16 = lane & 15;
    const char * row = src + j16 * G8::ROWB;
    const int a0 = slot_byte(j16, g);
    uint32_t raw[PF][3];
    half_t dsc[PF];
    auto rd = [&](int s) {
        const int b = 34 * s + 2 + 8 * g;                  // = 2 (mod 4) for even s, 0 for odd s
        const uint32_t * p = reinterpret_cast<const uint32_t *>(row + (b & ~3));
        raw[s % PF][0] = p[0];
        raw[s % PF][1] = p[1];
        if ((s & 1) == 0) raw[s % PF][2] = p[2];
        dsc[s % PF] = *reinterpret_cast<const half_t *>(row + 34 * s);
    };
#pragma unroll
    for (int s = 0; s < PF; ++s) rd(s);
    f32x4 acc0, acc1, acc2, acc3;
#pragma unroll
    for (int s = 0; s < G::QSTEPS; ++s) {
        const uint32_t * r = raw[s % PF];
        const half8 av = (s & 1) ? q8x8_to_f16<0>(r[0], r[1], 0u, dsc[s % PF]) : q8x8_to_f16<2>(r[0], r[1], r[2], dsc[s % PF]);
        if (s + PF < G::QSTEPS) rd(s + PF);
        if (32 * s < DV) *reinterpret_cast<half8 *>(dst + (a0 ^ (64 * (s & 1))) + 2048 * (s >> 1)) = av;
        if (s & 1) {
            mfma16<false>(acc2, av, qreg[0][s], s == 1);
            mfma16<false>(acc3, av, qreg[1][s], s == 1);
        } else {
            mfma16<false>(acc0, av, qreg[0][s], s == 0);
            mfma16<false>(acc1, av, qreg[1][s], s == 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    s0 = acc0 + acc2;
    s1 = acc1 + acc3;
}

// One row (token) t of the split: the whole pass, from the q staging to the partial record.
template <int DK, int DV>
__device__ __forceinline__ void decode_row_q8(const DecodeArgs & a, int t, Q8Lds<DK, DV> & sh) {
    using G = SliceGeom<DK>;
    using G8 = Q8Geom<DK>;
    using C = DecodeCfg<DK, DV>;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int g = lane >> 4;
    const int j16 = lane & 15;

    // the split's tile range and this token's mask row (SliceStream's own DMA plan is not used)
    const SliceStream<DK> ss(a, sp, t, w, lds_addr(sh.tile), lane);
    const int n_my = ss.n_my;
    const uint32_t ring8 = lds_addr(sh.ring8);

    // ---- q block into the f16 tile area, the first two tiles' slices into the int8 ring ----
    half8 qreg[2][G::QSTEPS];
    q_dma<DK>(a, lds_addr(sh.tile), hg0, t, w, lane);
    q8_dma<DK>(ss, ring8, 0, 0, lane);
    if (n_my > 1) {
        q8_dma<DK>(ss, ring8, 1, 1, lane);
        wait_vm<2 * G8::DMA_N>();            // this wave's part of q has landed
    } else {
        wait_vm<G8::DMA_N>();
    }
    __syncthreads();
    q_convert<DK>(sh.tile, lane, qreg);
    __syncthreads();                         // the tile area is free

    float m_ref[2] = {M_NONE, M_NONE};       // heads 16 n + j16, log2 units
    float l_acc = 0.0f;                      // head lane & 31, keys 8 (lane >> 5) .. +7 of each slice
    f32x16 o[C::NTQ];                        // o^T tiles, as kqkv_decode.hip
#pragma unroll
    for (int i = 0; i < C::NTQ; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
    const PvAddr pv(lane);
    char * sb = sh.tile + stage_byte<DK>(0, w);

    for (int k = 0; k < n_my; ++k) {
        const int s = k & 1;
        // this wave's slice of tile k has landed (tile k + 1's may still be in flight)
        if (k + 1 < n_my) wait_vm<G8::DMA_N>();
        else wait_vm<0>();
        if (k > 0) __syncthreads();          // every wave is past the P.V of tile k - 1
        const char * src = sh.ring8 + (s * NWAVE + w) * G8::SLOT;
        // Q.K^T from the int8 slice, which also writes the slice's f16 values for P.V (which reads
        // every slice, after the maxima barrier below)
        f32x4 s0, s1;
        qk_slice_q8<DK, DV>(src, sb, lane, qreg, s0, s1);
        const f32x4 mk = *reinterpret_cast<const f32x4 *>(src + G8::ROWS_BYTES + 16 * g);
        // the slot has been read: tile k + 2 takes it.  One burst here measured faster than the same
        // instructions spread over the P.V MFMAs (2.60 against 2.85 us per tile at 16 tiles a split):
        // the address unit's time (16 B a lane) stalls the issuing wave either way, and between MFMAs
        // it holds them back as well
        if (k + 2 < n_my) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            q8_dma<DK>(ss, ring8, s, k + 2, lane);
        }
        const int par = k & 1;
        const int kbase = (ss.t0 + k) * TK + WK * w;
        float sc[2][4], mx[2];
        slice_scores(a, mk, kbase, lane, s0, s1, sc, mx);
        // P against the current reference (exact unless it moves below; the clamp only keeps a
        // provisional value finite), into the exchange as [32 heads][64 keys]
        auto put_p = [&]() {
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                half4 ph;
#pragma unroll
                for (int r = 0; r < 4; ++r) ph[r] = to_half(exp2_fast(fminf(sc[n][r] - m_ref[n], 15.0f)));
                *reinterpret_cast<half4 *>(&sh.px[(16 * n + j16) * C::PROW + WK * w + 4 * g]) = ph;
            }
        };
        put_p();
        if (lane < 16) {
            sh.red[par][lane][w] = mx[0];
            sh.red[par][16 + lane][w] = mx[1];
        }
        __syncthreads();
        bool move = false;
        float tm[2];
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const f32x4 r4 = *reinterpret_cast<const f32x4 *>(&sh.red[par][16 * n + j16][0]);
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
            l_acc *= al[(lane >> 4) & 1];
            if (k > 0) {
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
        pv_tile<DK, DV>(sh.tile, sh.px, 0, w, lane, pv, o, l_acc);
    }
    wait_vm<0>();                            // every DMA of this wave has landed

    // staging: this wave's int8 slot of stage 0 (only this wave ever read it)
    decode_epilogue<DK, DV>(a, sh.ring8 + w * G8::SLOT, w, tid, t, hg0, sp, o, l_acc, m_ref);
}

// ROWS = false: one row per workgroup (blockIdx.z).  ROWS = true: rows blockIdx.z, blockIdx.z +
// gridDim.z, ... of split blockIdx.x share the workgroup (batch-of-N decode puts every row of a
// split in one); with a mask, the rows that hold no live key of the split are found first, in
// rounds of a few tiles of mask reads, and only record an empty split, the others run the whole
// pass in turn.  As kqkv_decode_f16_kernel.
template <int DK, int DV, bool ROWS>
__global__ __launch_bounds__(NTHR, 1) void kqkv_decode_q8_kernel(DecodeArgs a) {
    __shared__ Q8Lds<DK, DV> sh;
    if constexpr (!ROWS) {
        decode_row_q8<DK, DV>(a, blockIdx.z, sh);
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
        decode_row_q8<DK, DV>(a, t, sh);
        __syncthreads();                     // the next row's staging reuses the LDS
    }
}

// Q8_0 rows -> f16 rows holding the values the kernel above computes with, f16(q * d) by the same
// instructions, for the chunked-prefill path (the f16 prefill kernel then runs on the copy).  One
// thread per 16-value half-block: its 2-byte-aligned run read as dwords and realigned (the fifth
// dword only when the run is misaligned, where it lies inside the row's next block), two 16-byte
// stores.
template <int DK>
__global__ __launch_bounds__(256) void q8_rows_to_f16_kernel(const char * __restrict__ src, half_t * __restrict__ dst, int n_kv) {
    using G8 = Q8Geom<DK>;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;      // half-block
    if (i >= (int64_t)n_kv * G8::HB) return;
    const int64_t row = i / G8::HB;
    const int hb = (int)(i - row * G8::HB);
    const char * r = src + row * G8::ROWB;
    const int o = 34 * (hb >> 1) + 2 + 16 * (hb & 1);
    const uint32_t sh = (hb & 2) ? 0u : 2u;                          // 34 b + 2 + 16 h = 2 (b + 1) mod 4
    const uint32_t * p = reinterpret_cast<const uint32_t *>(r + (o & ~3));
    const half_t d = *reinterpret_cast<const half_t *>(r + 34 * (hb >> 1));
    half8 v0, v1;
    if (sh) {
        const uint32_t wd[5] = {p[0], p[1], p[2], p[3], p[4]};
        v0 = q8x8_to_f16<2>(wd[0], wd[1], wd[2], d);
        v1 = q8x8_to_f16<2>(wd[2], wd[3], wd[4], d);
    } else {
        const uint32_t wd[4] = {p[0], p[1], p[2], p[3]};
        v0 = q8x8_to_f16<0>(wd[0], wd[1], 0u, d);
        v1 = q8x8_to_f16<0>(wd[2], wd[3], 0u, d);
    }
    half8 * out = reinterpret_cast<half8 *>(dst + row * DK + 16 * hb);
    out[0] = v0;
    out[1] = v1;
}

template <int DK, int DV>
hipError_t launch_q8(const DecodeArgs & a, int n_hgroups, hipStream_t stream) {
    if (a.nt == 1)
        hipLaunchKernelGGL((kqkv_decode_q8_kernel<DK, DV, false>), dim3(a.n_split, n_hgroups, 1), dim3(NTHR), 0, stream, a);
    else
        hipLaunchKernelGGL((kqkv_decode_q8_kernel<DK, DV, true>), dim3(a.n_split, n_hgroups, decode_row_groups(a, n_hgroups)),
                           dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_kqkv_decode_q8(int dk, int dv, const DecodeArgs & a, hipStream_t stream) {
    const int n_hgroups = (a.n_head + HG - 1) / HG;
    if (dk == 576 && dv == 512) return launch_q8<576, 512>(a, n_hgroups, stream);
    if (dk == 320 && dv == 256) return launch_q8<320, 256>(a, n_hgroups, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_q8_rows_to_f16(int dk, const char * src, int n_kv, void * dst, hipStream_t stream) {
    const int64_t n = (int64_t)n_kv * (dk / 16);
    const dim3 grid((unsigned)((n + 255) / 256));
    if (dk == 576) hipLaunchKernelGGL(q8_rows_to_f16_kernel<576>, grid, dim3(256), 0, stream, src, static_cast<half_t *>(dst), n_kv);
    else if (dk == 320) hipLaunchKernelGGL(q8_rows_to_f16_kernel<320>, grid, dim3(256), 0, stream, src, static_cast<half_t *>(dst), n_kv);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace mla

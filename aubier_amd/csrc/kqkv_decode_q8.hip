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
//   * per tile: barrier (every wave is past the previous tile's P.V) -> each wave dequantises its
//     slice into the f16 tile -> it issues the DMA of tile k + 2 into the slot it has just read ->
//     the f16 kernel's Q.K^T of its own slice, scores, the maxima exchange (a barrier, after which
//     the whole f16 tile is in place), lazy reference max and P.V;
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

// Wave w's int8 slice at src -> f16 values in its slot of the tile at dst (the slot layout of
// decode_common.h, slot_byte).  Lane item i: row r = lane & 15, half-block hb = (lane >> 4) + 4 i (16
// values of block b = hb / 2, at bytes 34 b + 2 + 16 (hb & 1) of the row: 2-byte aligned, read as
// five dwords and realigned).  The 16 lanes of a group read 16 rows, 612 bytes (153 dwords) apart:
// distinct LDS banks.  Items go in batches of IB whose reads all issue before the first convert.
template <int DK>
__device__ __forceinline__ void dequant_slice(const char * src, char * dst, int lane) {
    using G8 = Q8Geom<DK>;
    static_assert(G8::HB % 4 == 0 && G8::ITEMS * 4 == G8::HB, "four half-block groups per row");
    constexpr int IB = G8::ITEMS % 3 == 0 ? 3 : 1;
    const half2 bias = {1152.0f16, 1152.0f16};            // 1024 + 128
    const int r = lane & 15;
    const char * row = src + r * G8::ROWB;
#pragma unroll
    for (int i0 = 0; i0 < G8::ITEMS; i0 += IB) {
        uint32_t wd[IB][5];
        half_t d[IB];
        int hb[IB];
#pragma unroll
        for (int u = 0; u < IB; ++u) {
            hb[u] = (lane >> 4) + 4 * (i0 + u);
            const int o = 34 * (hb[u] >> 1) + 2 + 16 * (hb[u] & 1);
            const uint32_t * p = reinterpret_cast<const uint32_t *>(row + (o & ~3));
#pragma unroll
            for (int k = 0; k < 5; ++k) wd[u][k] = p[k];
            d[u] = *reinterpret_cast<const half_t *>(row + 34 * (hb[u] >> 1));
        }
#pragma unroll
        for (int u = 0; u < IB; ++u) {
            const uint32_t sh = (hb[u] & 2) ? 0u : 2u;       // 34 b + 2 + 16 h = 2 (b + 1) mod 4
            const half2 dd = {d[u], d[u]};
            uint32_t ow[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t x = __builtin_amdgcn_alignbyte(wd[u][k + 1], wd[u][k], sh) ^ 0x80808080u;   // q + 128 per byte
                const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);   // bytes 0, 1 under 0x64
                const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);   // bytes 2, 3 under 0x64
                ow[2 * k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2, lo) - bias) * dd);
                ow[2 * k + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2, hi) - bias) * dd);
            }
            const int c0 = 2 * hb[u];                         // 16-byte chunks c0, c0 + 1 of row r
            *reinterpret_cast<u32x4 *>(dst + slot_byte(r, c0)) = u32x4{ow[0], ow[1], ow[2], ow[3]};
            *reinterpret_cast<u32x4 *>(dst + slot_byte(r, c0 + 1)) = u32x4{ow[4], ow[5], ow[6], ow[7]};
        }
    }
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
        dequant_slice<DK>(src, sb, lane);
        const f32x4 mk = *reinterpret_cast<const f32x4 *>(src + G8::ROWS_BYTES + 16 * g);
        if (k + 2 < n_my) {                  // the slot has been read: tile k + 2 takes it
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            q8_dma<DK>(ss, ring8, s, k + 2, lane);
        }
        // no barrier here: Q.K^T reads only this wave's own slice (its LDS accesses are in order),
        // and P.V, which reads every slice, follows the maxima barrier below, which every wave
        // reaches after its dequantisation

        f32x4 s0, s1;
        qk_slice<DK, false, false>(ss, SliceDma{}, sb, lane, qreg, s0, s1);
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
    const uint32_t wd[5] = {p[0], p[1], p[2], p[3], sh ? p[4] : 0u};
    const half_t d = *reinterpret_cast<const half_t *>(r + 34 * (hb >> 1));
    const half2 bias = {1152.0f16, 1152.0f16};
    const half2 dd = {d, d};
    uint32_t ow[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t x = __builtin_amdgcn_alignbyte(wd[k + 1], wd[k], sh) ^ 0x80808080u;
        const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
        const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
        ow[2 * k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2, lo) - bias) * dd);
        ow[2 * k + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2, hi) - bias) * dd);
    }
    u32x4 * out = reinterpret_cast<u32x4 *>(dst + row * DK + 16 * hb);
    out[0] = u32x4{ow[0], ow[1], ow[2], ow[3]};
    out[1] = u32x4{ow[4], ow[5], ow[6], ow[7]};
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

// wkb.hip -- GGML_OP_M4_WKB on gfx950: the MLA absorption of q's nope half into the latent space,
// dst[t][h][c] = sum_d W_kb[h][c][d] * q_nope[t][h][d], f32 throughout (ggml-cpu's F32 mul_mat
// converts nothing).  Reference: patches/ggml-m4/m4-wkb.cu:55-86 (a fixed Q8_0 gemv); this kernel
// takes the geometry from the tensors and streams the f32 weight.
//
// Decode is a pure HBM stream of W_kb (8 MiB at d_n = 128, D_v = 512, H = 32): each wavefront
// owns 8 (d_n = 128) or 16 (d_n = 64) consecutive rows of one head, issues all its 16-byte row
// loads before the first use, and reduces each row over its d_n/4 lanes with xor shuffles.  For
// a few tokens the rows stay in registers while the tokens stream past; from 16 tokens on the op
// is a batched GEMM and runs on MFMA (wkb_gemm_kernel, f32 operands split into f16 pieces).
#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

constexpr int WKB_NI = 4;   // row loads in flight per wavefront

template <int DN>
__global__ __launch_bounds__(256) void wkb_f32_kernel(WkbArgs a) {
    constexpr int LPR = DN / 4;          // lanes per row
    static_assert(LPR == 16 || LPR == 32, "rows of one or two 16-lane DPP rows");
    constexpr int RPI = 64 / LPR;        // rows per load instruction
    constexpr int RPW = RPI * WKB_NI;    // rows per wavefront
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int total = a.n_head * a.d_v;
    const int row0 = gw * RPW;
    if (row0 >= total) return;
    const int h = row0 / a.d_v;          // d_v % RPW == 0 (host-checked): one head per wavefront
    const int sub = lane / LPR, li = lane % LPR;

    f32x4 wv[WKB_NI];
#pragma unroll
    for (int i = 0; i < WKB_NI; ++i) {
        const int row = row0 + i * RPI + sub;
        wv[i] = ld16f_stream(a.w + (size_t)row * DN + 4 * li);
    }
    for (int t = 0; t < a.nt; ++t) {
        const float4 qv = *(reinterpret_cast<const float4 *>(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 + (size_t)h * a.q_nb1) + li);
        float p[WKB_NI];
#pragma unroll
        for (int i = 0; i < WKB_NI; ++i) {
            float v = wv[i][0] * qv.x;
            v = fmaf(wv[i][1], qv.y, v);
            v = fmaf(wv[i][2], qv.z, v);
            v = fmaf(wv[i][3], qv.w, v);
            p[i] = v;
        }
        // sum over the row's LPR lanes: the 16-lane rows by DPP, then (d_n = 128) the row pair
#pragma unroll
        for (int i = 0; i < WKB_NI; ++i) {
            p[i] += dpp_xor<8>(p[i]);
            p[i] += dpp_xor<4>(p[i]);
            p[i] += dpp_xor<2>(p[i]);
            p[i] += dpp_xor<1>(p[i]);
            if constexpr (LPR == 32) {
                float e, o;
                rows_pair16(p[i], e, o);
                p[i] = e + o;
            }
        }
        if (li == 0) {
            char * drow = reinterpret_cast<char *>(a.dst) + (size_t)t * a.d_nb2 + (size_t)h * a.d_nb1;
#pragma unroll
            for (int i = 0; i < WKB_NI; ++i) {
                const int c = row0 + i * RPI + sub - h * a.d_v;
                reinterpret_cast<float *>(drow)[c] = p[i];
            }
        }
    }
}

// Many tokens (chunked prefill): per head a GEMM dst_h[t][c] = sum_d q_h[t][d] W_h[c][d] with f32
// operands, run on the 16-bit MFMA: each operand value x is split into two f16 pieces,
// hi = f16(x) and lo = f16(2^11 (x - hi)) (x - hi is exact in f32), which carry 22 bits of x, and
// x.y = hi.hi + 2^-11 (hi.lo + lo.hi) up to lo.lo (below 2^-22 of the product).  Three
// v_mfma_f32_32x32x16_f16 per 16-d step, f32 accumulation (hi.hi on one accumulator, the cross
// terms on a second, added at the end): 5.3x the operand throughput of v_mfma_f32_32x32x2_f32 for
// results within a few f32 ulps of the f32 product.  A 16-d step of a wave whose largest operand
// magnitude is 2^15 or more (hi would overflow f16) or below 2^-8 (its values would sit in f16's
// subnormal range) runs on v_mfma_f32_32x32x2_f32 instead, on the same accumulator.
// With two waves per SIMD the kernel is bound by the VALU work of the split, not by the MFMAs (32
// values per lane per 16-d step against 12 MFMAs), so the split is written out instruction by
// instruction: 3 VALU instructions per value with the range check (split_pair, v_max3_f32 on
// absolute values), where the compiler's own f32 -> f16 -> f32 round trip and canonicalising max
// took about 7.
// A workgroup computes a 128-token x 128-column tile of one head, each wave a 64 x 64 quarter
// (2 x 2 tiles of 32 x 32).  The operands pass through LDS in d-chunks of 32 (128 bytes of every
// row): the chunk's q rows (A) and W rows (B) arrive by LDS DMA, 8 lanes fetching one row's whole
// 128-byte line, in a two-stage ring (64 KB), the next chunk's DMA in flight while the MFMAs run on
// this one.  Row r of a stage keeps its 8 16-byte chunks at slot c ^ (r & 7), so the fragment reads
// (32 rows at one chunk) cover every bank once per 8 lanes.  A lane reads 8 consecutive d of its
// row per 16-d step, the k index of the f16 MFMA (or, on the f32 path, d = 16 ks + 8 (lane >> 5) + e
// is k-step e, in A and B alike: the k order inside an MFMA is free as long as both operands
// agree).  Tiles are ordered so that the tiles of a head run on one XCD (workgroup i is dispatched
// to XCD i mod 8), which keeps each head's q and W rows in one L2.  Two workgroups share a CU
// (LDS-bound), so the kernel is held to 256 registers per lane.  The result leaves through the
// ring once it is free: each wave's 64 x 64 quarter as rows in LDS, then 16-byte row chunks (16
// stores of 1 KB per wave instead of 64 single-value stores, each with its own row address);
// an output view whose rows are not 16-byte aligned takes the single-value stores.
constexpr int WKB_GEMM_MIN_TOKENS = 16;
constexpr int WG_T = 128;                   // tile rows (tokens) and columns
constexpr int WG_DC = 32;                   // d per chunk
constexpr int WG_STAGE = WG_T * WG_DC * 4;  // bytes of one operand in one stage (16 KB)

// x = hi + 2^-11 lo for a pair of f32 values: hi = f16(x) (round to nearest even, v_cvt_pk_f16_f32),
// d = x - hi exactly in f32 (v_fma_mix_f32 takes hi's f16 half as it is), lo = f16(2^11 d) rounded
// once (v_fma_mixlo / mixhi_f16 write the low / high half): 2.5 VALU instructions per value.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t & hi, uint32_t & lo) {
    uint32_t h, l;
    float d0, d1;
    const float two11 = 2048.0f;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(h) : "v"(x0), "v"(x1));
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d0) : "v"(h), "v"(x0));
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d1) : "v"(h), "v"(x1));
    asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(l) : "v"(d0), "s"(two11));
    asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(l) : "v"(d1), "s"(two11));
    hi = h;
    lo = l;
}
// the f16 pieces of 8 values (x0, then x1), in MFMA operand order
__device__ __forceinline__ void split8(const f32x4 & x0, const f32x4 & x1, half8 & hi, half8 & lo) {
    uint32_t h[4], l[4];
    split_pair(x0[0], x0[1], h[0], l[0]);
    split_pair(x0[2], x0[3], h[1], l[1]);
    split_pair(x1[0], x1[1], h[2], l[2]);
    split_pair(x1[2], x1[3], h[3], l[3]);
    hi = __builtin_bit_cast(half8, u32x4{h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(half8, u32x4{l[0], l[1], l[2], l[3]});
}

struct WkbGemmLds {
    __attribute__((aligned(16))) char a[2][WG_STAGE];
    __attribute__((aligned(16))) char b[2][WG_STAGE];
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void wkb_gemm_kernel(WkbArgs a) {
    __shared__ WkbGemmLds sh;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ntb = (a.nt + WG_T - 1) / WG_T, ncb = (a.d_v + WG_T - 1) / WG_T;
    const int per_head = ntb * ncb;
    const int total = a.n_head * per_head;
    int lt = blockIdx.x;
    if ((total & 7) == 0) lt = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int h = lt / per_head;
    const int tb = (lt - h * per_head) / ncb;
    const int cb = lt - h * per_head - tb * ncb;
    const int t0 = tb * WG_T, c0 = cb * WG_T;

    // DMA plan: wave w fetches rows 8 i .. 8 i + 7 (i = 4 w .. 4 w + 3) of both operands; lane l
    // takes row 8 i + (l >> 3), logical chunk (l & 7) ^ (row & 7), into slot l of the 1 KB block i.
    // Each instruction's resource starts at its first row, so the lane offsets stay below 8 rows.
    const int lr = lane >> 3;
    const uint32_t lchunk = 16u * (uint32_t)((lane & 7) ^ lr);      // row & 7 == lr
    const char * qh = reinterpret_cast<const char *>(a.q) + (size_t)h * a.q_nb1;
    const char * wh = reinterpret_cast<const char *>(a.w) + (size_t)h * a.d_v * a.d_n * 4;
    const int rowb = a.d_n * 4;
    i32x4 ars[4], brs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r0 = 8 * (4 * w + u);
        const int ra = min(a.nt - t0 - r0, 8), rb = min(a.d_v - c0 - r0, 8);     // rows that exist
        ars[u] = make_rsrc(qh + (size_t)(t0 + r0) * a.q_nb2, ra > 0 ? (uint32_t)((int64_t)(ra - 1) * a.q_nb2 + rowb) : 0u);
        brs[u] = make_rsrc(wh + (size_t)(c0 + r0) * rowb, rb > 0 ? (uint32_t)(rb * rowb) : 0u);
    }
    const uint32_t avo = (uint32_t)(lr * a.q_nb2) + lchunk, bvo = (uint32_t)(lr * rowb) + lchunk;
    auto dma_chunk = [&](int kc, int st) {
        const uint32_t la = lds_addr(sh.a[st]), lb = lds_addr(sh.b[st]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t blk = 1024u * (uint32_t)(4 * w + u);
            dma16(ars[u], avo + (uint32_t)(WG_DC * 4 * kc), 0u, la + blk);
            dma16(brs[u], bvo + (uint32_t)(WG_DC * 4 * kc), 0u, lb + blk);
        }
    };

    // fragment addresses: A rows 64 (w >> 1) + 32 i + (lane & 31), B rows 64 (w & 1) + 32 j + (lane & 31)
    const int r32 = lane & 31, hh = lane >> 5;
    const int sw = r32 & 7;
    const int apitch = WG_DC * 4;            // a stage row: 128 bytes
    const int aoff = apitch * (64 * (w >> 1) + r32), boff = apitch * (64 * (w & 1) + r32);

    // acc: the f32 sum; accx: the cross terms of the f16 split, in units of 2^-11
    f32x16 acc[2][2], accx[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[i][j][r] = 0.0f;
                accx[i][j][r] = 0.0f;
            }

    const int nch = a.d_n / WG_DC;
    dma_chunk(0, 0);
    for (int kc = 0; kc < nch; ++kc) {
        const int st = kc & 1;
        wait_vm<0>();                        // this wave's part of chunk kc has landed
        __syncthreads();                     // every wave's part; every wave is past chunk kc - 1
        if (kc + 1 < nch) dma_chunk(kc + 1, st ^ 1);
        const char * sa = sh.a[st];
        const char * sb = sh.b[st];
        // per 16-d k-step ks: the wave's operands, row 32 i + (lane & 31) of its A / B rows,
        // d = 16 ks + 8 hh .. + 7 (logical 16-byte chunks 4 ks + 2 hh, + 1)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f32x4 af[2][2], bf[2][2];            // [tile][half]
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int slot = 16 * ((4 * ks + 2 * hh + u) ^ sw);
                    af[i][u] = *reinterpret_cast<const f32x4 *>(sa + aoff + apitch * 32 * i + slot);
                    bf[i][u] = *reinterpret_cast<const f32x4 *>(sb + boff + apitch * 32 * i + slot);
                }
            // the largest magnitude among the wave's operands of this step: v_max3_f32 on absolute
            // values, two per instruction (no canonicalisation of the loaded values), in two chains;
            // the s_nop covers the VALU -> DPP read distance of the wave reduction
            float mx = 0.0f, my = 0.0f;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int e = 0; e < 4; e += 2) {
                        asm("v_max3_f32 %0, |%1|, |%2|, %0" : "+v"(mx) : "v"(af[i][u][e]), "v"(af[i][u][e + 1]));
                        asm("v_max3_f32 %0, |%1|, |%2|, %0" : "+v"(my) : "v"(bf[i][u][e]), "v"(bf[i][u][e + 1]));
                    }
            asm("v_max_f32 %0, %0, %1\n\ts_nop 1" : "+v"(mx) : "v"(my));
            mx = wave_max(mx);
            if (mx < 32768.0f && (mx >= 0.00390625f || mx == 0.0f)) {
                // x = hi + 2^-11 lo with hi = f16(x), lo = f16(2^11 (x - hi)) (x - hi exact in f32):
                // 22 bits of x.  hi.hi on one accumulator, hi.lo + lo.hi on the other (lo.lo, below
                // 2^-22 of the product, is dropped)
                half8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    split8(af[i][0], af[i][1], ah[i], al[i]);
                    split8(bf[i][0], bf[i][1], bh[i], bl[i]);
                }
                // 3 wait states between the VALU writes above (inline asm, outside the compiler's
                // hazard tracking) and the MFMAs that read them
                asm volatile("s_nop 2" : "+v"(ah[0]), "+v"(ah[1]), "+v"(al[0]), "+v"(al[1]), "+v"(bh[0]), "+v"(bh[1]),
                             "+v"(bl[0]), "+v"(bl[1]));
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                        accx[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], accx[i][j], 0, 0, 0);
                        accx[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], accx[i][j], 0, 0, 0);
                    }
            } else {
                // values the f16 pieces cannot carry (|x| >= 2^15) or a step of tiny values: f32
                // MFMA, its k-step e taking d = 16 ks + 8 hh + e in A and B alike
#pragma unroll
                for (int e = 0; e < 8; ++e)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][e >> 2][e & 3], bf[j][e >> 2][e & 3],
                                                                            acc[i][j], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(accx[i][j][r], 1.0f / 2048.0f, acc[i][j][r]);
    // C tile (i, j): lane column c = c0 + 64 (w & 1) + 32 j + (lane & 31), rows
    // t = t0 + 64 (w >> 1) + 32 i + 8 (r / 4) + 4 (lane >> 5) + (r & 3)
    char * db = reinterpret_cast<char *>(a.dst) + (size_t)h * a.d_nb1;
    const int tw = t0 + 64 * (w >> 1), cw = c0 + 64 * (w & 1);
    const bool rows16 = ((reinterpret_cast<uintptr_t>(db) | (uintptr_t)a.d_nb2) & 15) == 0 && (a.d_v & 3) == 0;
    if (rows16) {
        // through LDS (the ring is free once every wave is past the last chunk): the wave's 64 x 64
        // quarter as [64 rows][64 columns] in its own 16 KB, then out in 16-byte row chunks, four
        // rows of 256 bytes per store instruction
        __syncthreads();
        float * qs = reinterpret_cast<float *>(&sh) + w * 64 * 64;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    qs[(32 * i + 8 * (r >> 2) + 4 * hh + (r & 3)) * 64 + 32 * j + r32] = acc[i][j][r];
        const int ch = lane & 15, rq = lane >> 4;
        const int col = cw + 4 * ch;
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int row = 4 * it + rq;
            const f32x4 v = *reinterpret_cast<const f32x4 *>(qs + row * 64 + 4 * ch);
            const int t = tw + row;
            if (t < a.nt && col < a.d_v) *reinterpret_cast<f32x4 *>(db + (size_t)t * a.d_nb2 + 4 * col) = v;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = cw + 32 * j + r32;
            if (c >= a.d_v) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = tw + 32 * i + 8 * (r >> 2) + 4 * hh + (r & 3);
                if (t < a.nt) reinterpret_cast<float *>(db + (size_t)t * a.d_nb2)[c] = acc[i][j][r];
            }
        }
}

}  // namespace

hipError_t launch_wkb_f32(const WkbArgs & a, hipStream_t stream) {
    if (a.nt >= WKB_GEMM_MIN_TOKENS && a.d_n % WG_DC == 0) {
        // one 8-row DMA window of q must stay within the buffer's 32-bit offsets
        if (a.q_nb2 > (int64_t)(UINT32_MAX / 8)) return hipErrorInvalidValue;
        const int64_t tiles = (int64_t)a.n_head * ((a.nt + WG_T - 1) / WG_T) * ((a.d_v + WG_T - 1) / WG_T);
        if (tiles > INT32_MAX) return hipErrorInvalidValue;
        hipLaunchKernelGGL(wkb_gemm_kernel, dim3((unsigned)tiles), dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    const int total = a.n_head * a.d_v;
    if (a.d_n == 128) {
        const int rpb = 4 * (64 / 32) * WKB_NI;
        hipLaunchKernelGGL(wkb_f32_kernel<128>, dim3((total + rpb - 1) / rpb), dim3(256), 0, stream, a);
    } else if (a.d_n == 64) {
        const int rpb = 4 * (64 / 16) * WKB_NI;
        hipLaunchKernelGGL(wkb_f32_kernel<64>, dim3((total + rpb - 1) / rpb), dim3(256), 0, stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mla

// wkb.hip -- GGML_OP_M4_WKB on gfx950: the MLA absorption of q's nope half into the latent space,
// dst[t][h][c] = sum_d W_kb[h][c][d] * q_nope[t][h][d], f32 throughout (ggml-cpu's F32 mul_mat
// converts nothing).  Reference: patches/ggml-m4/m4-wkb.cu:55-86 (a fixed Q8_0 gemv); this kernel
// takes the geometry from the tensors and streams the f32 weight.
//
// Decode is a pure HBM stream of W_kb (8 MiB at d_n = 128, D_v = 512, H = 32): each wavefront
// owns 8 (d_n = 128) or 16 (d_n = 64) consecutive rows of one head, issues all its 16-byte row
// loads before the first use, and reduces each row over its d_n/4 lanes with xor shuffles.  For
// a few tokens the rows stay in registers while the tokens stream past; from 16 tokens on the op
// is a batched GEMM and runs on f32 MFMA (wkb_gemm_kernel).
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

// Many tokens (chunked prefill): per head a GEMM dst_h[t][c] = sum_d q_h[t][d] W_h[c][d], on
// v_mfma_f32_32x32x2_f32 (f32 products and sums, as the f32 mul_mat).  A workgroup computes 128
// tokens x 128 columns of one head, each wave a 64 x 64 quarter (2 x 2 tiles of 32 x 32).  Both
// operands have d contiguous, so a lane reads 4 consecutive d of its row (16 bytes) and spends them
// on 4 MFMA k-steps: step j uses d = 8 p + 4 (lane >> 5) + j in A and B alike (the k order inside
// an MFMA is free as long as both operands agree).  Operands come straight from global memory
// (L2-resident: each q tile is read by D_v/128 workgroups, each W tile by nt/128) one 8-d block
// ahead of their MFMAs.
constexpr int WKB_GEMM_MIN_TOKENS = 16;

__global__ __launch_bounds__(256) void wkb_gemm_kernel(WkbArgs a) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int h = blockIdx.z;
    const int tw = blockIdx.y * 128 + 64 * (w >> 1);     // this wave's first token
    const int cw = blockIdx.x * 128 + 64 * (w & 1);      // and first column
    const int r32 = lane & 31, hh = lane >> 5;
    const char * qb = reinterpret_cast<const char *>(a.q) + (size_t)h * a.q_nb1;
    const float * wb = a.w + (size_t)h * a.d_v * a.d_n;
    const float * arow[2];
    const float * brow[2];
    bool av[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int t = tw + 32 * i + r32;
        av[i] = t < a.nt;
        arow[i] = reinterpret_cast<const float *>(qb + (size_t)min(t, a.nt - 1) * a.q_nb2) + 4 * hh;
        const int c = min(cw + 32 * i + r32, a.d_v - 1);
        brow[i] = wb + (size_t)c * a.d_n + 4 * hh;
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const int np = a.d_n / 8;
    f32x4 an[2], bn[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        an[i] = av[i] ? *reinterpret_cast<const f32x4 *>(arow[i]) : f32x4{0.f, 0.f, 0.f, 0.f};
        bn[i] = *reinterpret_cast<const f32x4 *>(brow[i]);
    }
    for (int p = 0; p < np; ++p) {
        const f32x4 ac[2] = {an[0], an[1]};
        const f32x4 bc[2] = {bn[0], bn[1]};
        if (p + 1 < np) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                an[i] = av[i] ? *reinterpret_cast<const f32x4 *>(arow[i] + 8 * (p + 1)) : f32x4{0.f, 0.f, 0.f, 0.f};
                bn[i] = *reinterpret_cast<const f32x4 *>(brow[i] + 8 * (p + 1));
            }
        }
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ac[i][j4], bc[j][j4], acc[i][j], 0, 0, 0);
    }
    // C tile (i, j): lane column c = cw + 32 j + (lane & 31), rows t = tw + 32 i + 8 (r / 4) + 4 (lane >> 5) + (r & 3)
    char * db = reinterpret_cast<char *>(a.dst) + (size_t)h * a.d_nb1;
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
    if (a.nt >= WKB_GEMM_MIN_TOKENS && a.d_n % 8 == 0) {
        const dim3 grid((a.d_v + 127) / 128, (a.nt + 127) / 128, a.n_head);
        hipLaunchKernelGGL(wkb_gemm_kernel, grid, dim3(256), 0, stream, a);
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

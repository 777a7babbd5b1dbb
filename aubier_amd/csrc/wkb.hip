// wkb.hip -- GGML_OP_M4_WKB on gfx950: the MLA absorption of q's nope half into the latent space,
// dst[t][h][c] = sum_d W_kb[h][c][d] * q_nope[t][h][d], f32 throughout (ggml-cpu's F32 mul_mat
// converts nothing).  Reference: patches/ggml-m4/m4-wkb.cu:55-86 (a fixed Q8_0 gemv); this kernel
// takes the geometry from the tensors and streams the f32 weight.
//
// Decode is a pure HBM stream of W_kb (8 MiB at d_n = 128, D_v = 512, H = 32): each wavefront
// owns 8 (d_n = 128) or 16 (d_n = 64) consecutive rows of one head, issues all its 16-byte row
// loads before the first use, and reduces each row over its d_n/4 lanes with xor shuffles.  For
// nt > 1 the rows stay in registers while the tokens stream past.
#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

constexpr int WKB_NI = 4;   // row loads in flight per wavefront

template <int DN>
__global__ __launch_bounds__(256) void wkb_f32_kernel(WkbArgs a) {
    constexpr int LPR = DN / 4;          // lanes per row
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
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1)
#pragma unroll
            for (int i = 0; i < WKB_NI; ++i) p[i] += shfl_xor(p[i], off);
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

}  // namespace

hipError_t launch_wkb_f32(const WkbArgs & a, hipStream_t stream) {
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

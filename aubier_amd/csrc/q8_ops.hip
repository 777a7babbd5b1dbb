// q8_ops.hip -- the reference geometry's quantised ops on gfx950:
//   * GGML_OP_M4_WKB with a Q8_0 W_kb (patches/ggml-m4/m4-wkb.cu:14-86),
//   * GGML_OP_M4_PHASE phase 1, wv_b (m4-phase.cu:44-89, 209-224),
//   * GGML_OP_M4_PHASE phase 0, KV-write: wkv_a gemv, RMS norm, YaRN rope and the in-place f16
//     (or Q8_0) scatter into the cache (m4-phase.cu:91-200, 226-273).
// Numerics are the reference kernels' (the GPU MMVQ form, not ggml-cpu's): the f32 activation is
// quantised per 32-value block (d = amax / 127, an f16 scale, int8 quants by roundf(x / d) in
// WKB and roundf(x * (1 / d)) in the PHASE ops), block dots are exact int32 sums (v_dot4_i32_i8),
// and the f32 accumulation keeps the reference's order -- per row, or per lane and then the
// 32-lane xor butterfly of warp_reduce_sum -- so the integer paths match the CPU restatement bit
// for bit.  All three are small latency-bound launches (0.5 MiB, 1 MiB and 1.4 MiB of weights).
#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

__device__ __forceinline__ float f16_bits(uint32_t bits) { return (float)__builtin_bit_cast(half_t, (uint16_t)bits); }
__device__ __forceinline__ float round_to_f16(float x) { return (float)(half_t)x; }

// The 4 bytes of a row at byte offset B, from the row's dwords D (B folds to a constant once the
// caller's loops are unrolled; rows are 4-byte aligned, Q8_0 blocks only 2-byte aligned).
__device__ __forceinline__ uint32_t bytes4(const uint32_t * D, int B) {
    const int i = B >> 2, r = B & 3;
    return r == 0 ? D[i] : __builtin_amdgcn_alignbyte(D[i + 1], D[i], r);
}

// Block quantisation with one value per lane of a 32-lane half-wavefront (the xor offsets stay
// inside the half): returns the int8 quant, d16 = the block's f16 scale as f32.
template <bool DIV>
__device__ __forceinline__ int quant_lane(float x, float & d16) {
    const float amax = half_max(fabsf(x));
    const float d = amax / 127.0f;
    d16 = round_to_f16(d);
    if constexpr (DIV) return amax == 0.0f ? 0 : (int)roundf(x / d);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    return (int)roundf(x * id);
}

// The 32-lane butterfly of warp_reduce_sum (xor 16, 8, 4, 2, 1) inside a half-wavefront: the
// same additions in the same order (mla_common.h).
__device__ __forceinline__ float half_wave_sum(float v) { return half_sum(v); }

// ---- WKB, Q8_0 W_kb: one workgroup per (head, token); a thread per output row ----
// The head's d_n activations are quantised once into LDS (4 int8 per word); each row's blocks
// come in as dwords (17 per 2 blocks), the qs realigned with v_alignbyte, dotted with
// v_dot4_i32_i8, and acc = fma(wd * d16, sum, acc) over the blocks in order (m4-wkb.cu:30-52).
template <int NB>
__global__ __launch_bounds__(256) void wkb_q8_kernel(WkbArgs a) {
    static_assert(NB % 2 == 0, "rows of an even number of blocks are 4-byte aligned");
    constexpr int RW = NB * 17 / 2;      // dwords per row
    __shared__ uint32_t xq[NB * 8];
    __shared__ float xd[NB];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    if (tid < NB * 32) {                 // whole wavefronts: NB * 32 is a multiple of 64
        const float x = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 +
                                                        (size_t)h * a.q_nb1)[tid];
        float d16;
        const int q = quant_lane<true>(x, d16);
        reinterpret_cast<int8_t *>(xq)[tid] = (int8_t)q;
        if ((tid & 31) == 0) xd[tid >> 5] = d16;
    }
    __syncthreads();
    float * drow = reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + (size_t)t * a.d_nb2 + (size_t)h * a.d_nb1);
    for (int r = tid; r < a.d_v; r += 256) {
        const uint32_t * row = reinterpret_cast<const uint32_t *>(a.wq + ((size_t)h * a.d_v + r) * (NB * 34));
        uint32_t D[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) D[i] = row[i];
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int o = 34 * b;
            const float wd = f16_bits((D[o >> 2] >> (8 * (o & 3))) & 0xffffu);
            int s = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) s = __builtin_amdgcn_sdot4((int)bytes4(D, o + 2 + 4 * j), (int)xq[8 * b + j], s, false);
            acc = fmaf(wd * xd[b], (float)s, acc);
        }
        drow[r] = acc;
    }
}

// ---- PHASE 1, wv_b: 8 outputs per workgroup (one per 32-lane half), grid (d_out / 8, H, nt) ----
// Lane k of an output's half holds element k of every block: p_k = sum_b fma(wd_b * xd_b,
// q_w[b][k] * q_x[b][k], .), then the butterfly (m4-phase.cu:52-88).
template <int NB>
__global__ __launch_bounds__(256) void wvb_q8_kernel(WvbArgs a) {
    __shared__ int8_t xq[NB * 32];
    __shared__ float xd[NB];
    const int h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const float * xh = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.x) + (size_t)t * a.x_nb1 +
                                                       (size_t)h * a.x_nb2);
    static_assert((NB * 32) % 256 == 0, "whole rounds of the workgroup");
#pragma unroll
    for (int i0 = 0; i0 < NB * 32; i0 += 256) {
        const int i = i0 + tid;
        float d16;
        const int q = quant_lane<false>(xh[i], d16);
        xq[i] = (int8_t)q;
        if ((i & 31) == 0) xd[i >> 5] = d16;
    }
    __syncthreads();
    const int o = blockIdx.x * 8 + (tid >> 5);
    const int k = tid & 31;
    if (o >= a.d_out) return;                // whole halves leave together
    const uint8_t * row = a.w + ((size_t)h * a.d_out + o) * (NB * 34);
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float wd = f16_bits(*reinterpret_cast<const uint16_t *>(row + 34 * b));
        const int q = (int)reinterpret_cast<const int8_t *>(row + 34 * b + 2)[k];
        acc = fmaf(wd * xd[b], (float)(q * (int)xq[32 * b + k]), acc);
    }
    acc = half_wave_sum(acc);
    if (k == 0)
        reinterpret_cast<float *>(reinterpret_cast<char *>(a.dst) + (size_t)t * a.d_nb1 + (size_t)h * a.d_nb2)[o] = acc;
}

// ---- PHASE 0, KV-write ----
// gemv: a workgroup per output row, a thread per 32-value block of the input (m4-phase.cu:95-125):
// the thread quantises its block itself, acc = (wd * d16) * sum, the butterfly per 32 blocks, then
// the 32-block partials summed in order.
template <int NBE>
__global__ __launch_bounds__(NBE) void kvwrite_gemv_kernel(KvWriteArgs a) {
    // the reference's product (wd * d16) * sum and the butterfly's adds are separate statements;
    // without this the compiler fuses the first add with the product (one rounding instead of two)
#pragma clang fp contract(off)
    static_assert(NBE % 32 == 0 && NBE <= 1024, "whole 32-block groups");
    __shared__ float sv[NBE / 32];
    const int o = blockIdx.x, tid = threadIdx.x;
    const float * xb = a.cur + 32 * tid;
    float x[32];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        x[k] = xb[k];
        amax = fmaxf(amax, fabsf(x[k]));
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const float d16 = round_to_f16(d);
    uint32_t xqw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t wv = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) wv |= ((uint32_t)(uint8_t)(int8_t)(int)roundf(x[4 * j + e] * id)) << (8 * e);
        xqw[j] = wv;
    }
    // the block's 34 bytes: 2-byte aligned; read the 9 dwords around it and realign
    const size_t boff = ((size_t)o * (NBE * 34)) + 34 * (size_t)tid;
    const uint32_t * bw = reinterpret_cast<const uint32_t *>(a.w + (boff & ~(size_t)3));
    const int sh = (int)(boff & 3);          // 0 or 2
    // (at sh = 0 the last two bytes of the 9th dword are the next block's: read only the 16 bits
    // that belong to this one, so the last block of the tensor reads nothing past its end)
    uint32_t D[9];
#pragma unroll
    for (int i = 0; i < 8; ++i) D[i] = bw[i];
    D[8] = sh ? bw[8] : (uint32_t)*reinterpret_cast<const uint16_t *>(bw + 8);
    const float wd = f16_bits((D[0] >> (8 * sh)) & 0xffffu);
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t qw = sh ? D[j + 1] : __builtin_amdgcn_alignbyte(D[j + 1], D[j], 2);
        s = __builtin_amdgcn_sdot4((int)qw, (int)xqw[j], s, false);
    }
    float acc = (wd * d16) * (float)s;
    acc = half_wave_sum(acc);
    if ((tid & 31) == 0) sv[tid >> 5] = acc;
    __syncthreads();
    if (tid == 0) {
        float total = sv[0];
#pragma unroll
        for (int g = 1; g < NBE / 32; ++g) total += sv[g];
        a.dst[o] = total;
    }
}

// tail: one workgroup of n_out threads (m4-phase.cu:130-200).  Every thread reads its inputs
// (its row of the gemv output, and for a rope row both of its pair), the squares of the latent
// rows are reduced (butterfly per 32 rows, then the partials in order), and each thread writes its
// final value to dst and, as f16, to cache row kidx -- read on the device from the graph's
// tensors; a row outside [0, n_kv) is not written (the reference trusts the engine; this
// implementation refuses to scatter out of bounds).  With a Q8_0 cache (kc_q8) each 32-thread
// half-wavefront holds one block of the row and stores it as ggml's f32 -> q8_0 copy does
// (quantize_row_q8_0_ref, ggml-quants.c:276-299): d = amax / 127, q = roundf(x * (1 / d)), the
// f16 scale by the block's first lane, one int8 per lane.  n_out is a multiple of 32, so a
// half-wavefront is either all inside the row or all past it.
__global__ __launch_bounds__(1024) void kvwrite_tail_kernel(KvWriteArgs a) {
    __shared__ float sred[32];
    const int tid = threadIdx.x;
    const int n_out = a.d_lat + a.n_rope;
    const int64_t row = a.kidx[0];
    const int pos = a.pos[0];
    const bool lat = tid < a.d_lat;
    const bool rope = !lat && tid < n_out;
    const float v = tid < n_out ? a.dst[tid] : 0.0f;
    float x0 = 0.0f, x1 = 0.0f;
    const int p = (tid - a.d_lat) >> 1;     // the rope pair of a rope row
    if (rope) {
        x0 = a.dst[a.d_lat + 2 * p];
        x1 = a.dst[a.d_lat + 2 * p + 1];
    }
    const float sq = lat ? v * v : 0.0f;
    const float part = half_wave_sum(sq);
    if ((tid & 31) == 0) sred[tid >> 5] = part;
    __syncthreads();                         // (also: every input of dst has been read)
    float s = 0.0f;
    for (int g = 0; g < (n_out + 31) / 32; ++g) s += sred[g];
    float out = 0.0f;
    if (lat) {
        const float scale = rsqrtf(s / (float)a.d_lat + a.eps);
        out = scale * v * a.nw[tid];
    } else if (rope) {
        const float theta_extrap = (float)pos * powf(a.theta_scale, (float)p);
        float mscale = a.attn_factor;
        float theta = a.freq_scale * theta_extrap;
        if (a.ext_factor != 0.0f) {
            const float y = ((float)p - a.corr0) / fmaxf(0.001f, a.corr1 - a.corr0);
            const float ramp_mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * a.ext_factor;
            theta = theta * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / a.freq_scale);
        }
        const float co = cosf(theta) * mscale, si = sinf(theta) * mscale;
        out = ((tid - a.d_lat) & 1) ? x0 * si + x1 * co : x0 * co - x1 * si;
    }
    if (a.kc_q8) {
        float d16;
        const int q = quant_lane<false>(out, d16);   // every lane takes part in the block max
        if (tid < n_out) {
            a.dst[tid] = out;
            if (row >= 0 && row < a.n_kv) {
                char * blk = reinterpret_cast<char *>(a.kcache) + (size_t)row * a.kc_nb1 + (size_t)(tid >> 5) * 34;
                if ((tid & 31) == 0) *reinterpret_cast<half_t *>(blk) = (half_t)d16;
                reinterpret_cast<int8_t *>(blk + 2)[tid & 31] = (int8_t)q;
            }
        }
        return;
    }
    if (tid < n_out) {
        a.dst[tid] = out;
        if (row >= 0 && row < a.n_kv)
            reinterpret_cast<half_t *>(reinterpret_cast<char *>(a.kcache) + (size_t)row * a.kc_nb1)[tid] = (half_t)out;
    }
}

}  // namespace

hipError_t launch_wkb_q8(const WkbArgs & a, hipStream_t stream) {
    const dim3 grid(a.n_head, a.nt);
    if (a.d_n == 64) hipLaunchKernelGGL(wkb_q8_kernel<2>, grid, dim3(256), 0, stream, a);
    else if (a.d_n == 128) hipLaunchKernelGGL(wkb_q8_kernel<4>, grid, dim3(256), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_wvb_q8(const WvbArgs & a, hipStream_t stream) {
    const dim3 grid((a.d_out + 7) / 8, a.n_head, a.nt);
    if (a.d_in == 256) hipLaunchKernelGGL(wvb_q8_kernel<8>, grid, dim3(256), 0, stream, a);
    else if (a.d_in == 512) hipLaunchKernelGGL(wvb_q8_kernel<16>, grid, dim3(256), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_kvwrite(const KvWriteArgs & a, hipStream_t stream) {
    const int n_out = a.d_lat + a.n_rope;
    if (n_out > 1024) return hipErrorInvalidValue;
    if (a.n_embd == 4096) hipLaunchKernelGGL(kvwrite_gemv_kernel<128>, dim3(n_out), dim3(128), 0, stream, a);
    else if (a.n_embd == 7168) hipLaunchKernelGGL(kvwrite_gemv_kernel<224>, dim3(n_out), dim3(224), 0, stream, a);
    else return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kvwrite_tail_kernel, dim3(1), dim3((n_out + 63) / 64 * 64), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla

// mla_common.h -- device-side helpers shared by the gfx950 MLA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// v_exp_f32: 2^x (the kernels keep scores in log2 units)
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// f32 -> f16 round-to-nearest-even (v_cvt_f16_f32 under the default round mode), the
// conversion ggml-cpu's mul_mat applies to src1 when src0 is F16.
__device__ __forceinline__ half_t to_half(float x) { return (half_t)x; }

// Cross-lane shuffles over the full 64-lane wavefront.
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, WAVE); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor(v, o);
    return v;
}

// gfx950 LDS transpose read (ds_read_b64_tr_b16).  In each 16-lane group, lane j supplies the
// address of 4 consecutive 16-bit elements; the 16 addresses form a 4 x 16 block (lane j holds row
// j >> 2, columns 4 (j & 3) .. +3) and lane j receives column j of that block, rows 0..3.
typedef short short4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ half4 lds_read_tr16(const half_t * p) {
    const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4v *)(__attribute__((address_space(3))) void *)p);
    return __builtin_bit_cast(half4, v);
}

// 16-byte global load/store helpers
__device__ __forceinline__ u32x4 ld16(const void * p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ __forceinline__ u32x4 ld16_stream(const void * p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ f32x4 ld16f_stream(const void * p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}

}  // namespace mla

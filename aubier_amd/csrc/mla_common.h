// mla_common.h -- device-side helpers shared by the gfx950 MLA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// v_exp_f32: 2^x (the kernels keep scores in log2 units)
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
// exp2_fast(x), or 0 where zero holds (a masked key, an empty accumulator), without a branch: the
// exponential is taken unconditionally (x may then be NaN) and the result selected
__device__ __forceinline__ float exp2_unless(bool zero, float x) {
    const float e = exp2_fast(x);
    return zero ? 0.0f : e;
}

// f32 -> f16 round-to-nearest-even (v_cvt_f16_f32 under the default round mode), the
// conversion ggml-cpu's mul_mat applies to src1 when src0 is F16.
__device__ __forceinline__ half_t to_half(float x) { return (half_t)x; }


// Max / sum over the four 16-lane rows of a wavefront (lanes j, j + 16, j + 32, j + 48) with the
// gfx950 row-swap instructions: v_permlane16_swap(x, x) leaves (row 0 | row 0 | row 2 | row 2) and
// (row 1 | row 1 | row 3 | row 3), v_permlane32_swap(x, x) (low half | low half) and (high | high):
// two VALU ops per step instead of an LDS permute round trip.
__device__ __forceinline__ float rows4_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// the value of lane l ^ 32 added to lane l's (the two 32-lane halves summed)
__device__ __forceinline__ float halves_sum(float v) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Lane l's partner l ^ k within rows of 16 lanes, by DPP (a VALU operand modifier, no LDS round
// trip): k = 1, 2 quad_perm [1,0,3,2] / [2,3,0,1]; k = 4 row_half_mirror (l -> 7 - l within 8) then
// quad_perm [3,2,1,0]; k = 8 row_ror:8.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int K>
__device__ __forceinline__ float dpp_xor(float v) {
    static_assert(K == 1 || K == 2 || K == 4 || K == 8, "row-local partners only");
    if constexpr (K == 1) return dpp_mov<0xB1>(v);
    else if constexpr (K == 2) return dpp_mov<0x4E>(v);
    else if constexpr (K == 4) return dpp_mov<0x1B>(dpp_mov<0x141>(v));
    else return dpp_mov<0x128>(v);
}
// (x of the even row, x of the odd row) of each pair of 16-lane rows / (low half, high half) of the
// wavefront, at every lane: the operands of a symmetric combine of lanes l and l ^ 16 / l ^ 32
__device__ __forceinline__ void rows_pair16(float v, float & even, float & odd) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    even = __uint_as_float(a[0]);
    odd = __uint_as_float(a[1]);
}
__device__ __forceinline__ void halves_pair(float v, float & lo, float & hi) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(b[0]);
    hi = __uint_as_float(b[1]);
}

// Butterflies over a 32-lane half (xor 16, 8, 4, 2, 1) and the whole wavefront (xor 32 first):
// every step adds / maxes the partner's current value, as the LDS-permute loops would, on the VALU
__device__ __forceinline__ float half_sum(float v) {
    float e, o;
    rows_pair16(v, e, o);
    v = e + o;
    v += dpp_xor<8>(v);
    v += dpp_xor<4>(v);
    v += dpp_xor<2>(v);
    return v + dpp_xor<1>(v);
}
__device__ __forceinline__ float half_max(float v) {
    float e, o;
    rows_pair16(v, e, o);
    v = fmaxf(e, o);
    v = fmaxf(v, dpp_xor<8>(v));
    v = fmaxf(v, dpp_xor<4>(v));
    v = fmaxf(v, dpp_xor<2>(v));
    return fmaxf(v, dpp_xor<1>(v));
}
__device__ __forceinline__ float wave_max(float v) {
    float lo, hi;
    halves_pair(v, lo, hi);
    return half_max(fmaxf(lo, hi));
}
__device__ __forceinline__ float wave_sum(float v) {
    float lo, hi;
    halves_pair(v, lo, hi);
    return half_sum(lo + hi);
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

// LDS DMA through a raw buffer resource (gfx950 buffer_load_dword{,x4} ... lds).  Lane l's 4 (or
// 16) bytes at rsrc.base + voff + soff land in LDS at lds_base + l * 4 (or * 16); lds_base is
// wave-uniform (it goes through M0).  The hardware range check of the resource makes a read at
// or past num_records return zeros, so tails need no clamping.  Issued from inline asm so that
// the compiler does not track them (its conservative handling of LDS DMA would wait for every DMA
// in flight before any LDS read): the caller owns the waits (s_waitcnt vmcnt).
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_rsrc(const void * base, uint32_t num_records) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    i32x4 r;
    r[0] = (int32_t)(uint32_t)b;
    r[1] = (int32_t)((uint32_t)(b >> 32) & 0xffffu);     // stride 0
    r[2] = (int32_t)num_records;
    r[3] = 0x00020000;                                  // gfx9 dword 3: DATA_FORMAT 32
    return r;
}
// 16-byte load through a buffer resource over [base, base + num_records): an offset at or past
// num_records reads zeros without a memory access -- a per-lane "or zero" with no branch.  NT: the
// non-temporal policy (buffer_load ... nt), for data read once.
template <bool NT = false>
__device__ __forceinline__ u32x4 buf_ld16(const void * base, uint32_t num_records, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)num_records, 0x00020000);
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, NT ? 2 : 0));
}
__device__ __forceinline__ uint32_t lds_addr(const void * p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" :: "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_base) : "memory");
}
// the same with the non-temporal policy: for data read once (a streamed cache), so that it does
// not displace reused data from the caches
__device__ __forceinline__ void dma16_nt(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds" :: "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_base) : "memory");
}
__device__ __forceinline__ void dma4(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds" :: "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_base) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }
// s_waitcnt vmcnt(n) for an n that folds to a constant once the caller's loop is unrolled
template <int N = 0>
__device__ __forceinline__ void wait_vm_le(int n) {
    if constexpr (N >= 63) {
        wait_vm<63>();
    } else {
        if (n <= N) { wait_vm<N>(); return; }
        wait_vm_le<N + 1>(n);
    }
}

// 16-byte streaming (non-temporal) global load
__device__ __forceinline__ f32x4 ld16f_stream(const void * p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}

}  // namespace mla

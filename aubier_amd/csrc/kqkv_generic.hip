// kqkv_generic.hip -- the VALU attention kernel (f32 caches and geometries outside the MFMA
// instantiations) and the split-K merge.
//
// Generic kernel: one workgroup (4 waves) per (split, head, token).  Splits are balanced runs of
// 16-key granules (GRAN_KEYS; finer than the MFMA kernels' 64-key tiles, so that a short window
// still spreads over ~256 workgroups), walked in 64-key tiles clipped to the split.  Per tile:
//   * scores: wave w takes keys 16 w .. 16 w + 15 of the tile, four lanes per key, each lane a
//     quarter of the row in 16-byte chunks (chunk 4 i + lane & 3), so the whole tile's loads of a
//     wave are in flight together (one memory latency per tile, not one per key); the four lanes
//     of a key are summed by two DPP steps;
//   * wave 0 does the online-softmax bookkeeping of the tile;
//   * P.V: thread t owns a 4-column chunk (t mod D_v/4) of the output and the keys of one residue
//     class (t div D_v/4) of the tile, 16-byte V loads; the classes are summed once at the end.
// F32 caches run in f32 end to end, like ggml-cpu's F32 mul_mat; with an F16 cache q and P are
// rounded to f16 first (the F16 vec_dot_type conversion), matching the MFMA path.
//
// Merge kernel (GGML_OP_M4_PHASE phase 2; the combine of patches/ggml-m4/m4-kqkv.cu:314-338)
// over the partial blocks of mla_kernels.h.
#include "mla_common.h"
#include "mla_kernels.h"
#include "mla_merge.h"

namespace mla {

namespace {

constexpr int GTK = 64;
constexpr int GMAX_DK = 1024;
constexpr int GMAX_DV = 1024;

template <bool F16>
__global__ __launch_bounds__(256) void kqkv_generic_kernel(DecodeArgs a, int dk, int dv) {
    constexpr int EPC = F16 ? 8 : 4;                 // elements per 16-byte chunk
    constexpr int ES = F16 ? 2 : 4;
    __shared__ __attribute__((aligned(16))) float qs[GMAX_DK];
    __shared__ float sc[GTK];
    __shared__ float ps[GTK];
    __shared__ float st[3];          // m_new, alpha, tile sum
    __shared__ __attribute__((aligned(16))) f32x4 ored[256];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int sp = blockIdx.x, h = blockIdx.y, t = blockIdx.z;

    const float * qrow = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 + (size_t)h * a.q_nb1);
    for (int k = tid; k < dk; k += 256) {
        const float x = qrow[k];
        qs[k] = F16 ? (float)to_half(x) : x;
    }
    const float * mrow = a.mask ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1) : nullptr;

    // this split's keys [k0, k1): a balanced run of whole granules
    const int n_gran = (a.n_kv + GRAN_KEYS - 1) / GRAN_KEYS;
    const int base_g = n_gran / a.n_split, rem_g = n_gran % a.n_split;
    const int g0 = sp * base_g + min(sp, rem_g);
    const int k0 = g0 * GRAN_KEYS;
    const int k1 = min((g0 + base_g + (sp < rem_g ? 1 : 0)) * GRAN_KEYS, a.n_kv);

    // scores: this lane's key (4 lanes per key) and quarter of the row
    const int kq = lane >> 2, qq = lane & 3;
    const int n_chunks = dk / EPC;                   // whole 16-byte chunks of a row
    // P.V: this thread's 4-column chunk and key class
    const int n_cc = dv / 4;
    const int n_kg = n_cc >= 256 ? 1 : 256 / n_cc;
    const int cc = tid % n_cc, kg = tid / n_cc;
    const bool pv_on = kg < n_kg && 4 * cc < dv;

    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;
    __syncthreads();

    for (int kb = k0; kb < k1; kb += GTK) {
        {
            const int key = kb + 16 * w + kq;
            const bool live_key = key < k1;
            const char * row = a.kc + (size_t)min(key, a.n_kv - 1) * a.kc_nb1;
            float d0 = 0.f, d1 = 0.f;
            // chunks qq, qq + 4, ... of the row, QB at a time: every load of a batch is issued
            // before the first use (one memory latency per batch; 576-wide rows take 2 batches)
            constexpr int QB = 18;
            for (int c0 = qq; c0 < n_chunks; c0 += 4 * QB) {
                u32x4 raw[QB];
#pragma unroll
                for (int b = 0; b < QB; ++b) {
                    const int c = c0 + 4 * b;
                    raw[b] = c < n_chunks ? *reinterpret_cast<const u32x4 *>(row + 16 * c) : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int b = 0; b < QB; ++b) {
                    const int c = min(c0 + 4 * b, n_chunks - 1);      // past the row: raw is zero
                    f32x4 lo, hi;
                    if constexpr (F16) {
                        const half8 hv = __builtin_bit_cast(half8, raw[b]);
                        lo = f32x4{(float)hv[0], (float)hv[1], (float)hv[2], (float)hv[3]};
                        hi = f32x4{(float)hv[4], (float)hv[5], (float)hv[6], (float)hv[7]};
                    } else {
                        lo = __builtin_bit_cast(f32x4, raw[b]);
                    }
                    const f32x4 qa = *reinterpret_cast<const f32x4 *>(&qs[EPC * c]);
                    d0 = fmaf(lo[0], qa[0], d0);
                    d1 = fmaf(lo[1], qa[1], d1);
                    d0 = fmaf(lo[2], qa[2], d0);
                    d1 = fmaf(lo[3], qa[3], d1);
                    if constexpr (F16) {
                        const f32x4 qb = *reinterpret_cast<const f32x4 *>(&qs[EPC * c + 4]);
                        d0 = fmaf(hi[0], qb[0], d0);
                        d1 = fmaf(hi[1], qb[1], d1);
                        d0 = fmaf(hi[2], qb[2], d0);
                        d1 = fmaf(hi[3], qb[3], d1);
                    }
                }
            }
            // elements past the whole chunks (dk not a multiple of EPC)
            for (int e = n_chunks * EPC + qq; e < dk; e += 4) {
                const float kv = F16 ? (float)reinterpret_cast<const half_t *>(row)[e] : reinterpret_cast<const float *>(row)[e];
                d0 = fmaf(kv, qs[e], d0);
            }
            float d = d0 + d1;
            d += dpp_xor<1>(d);
            d += dpp_xor<2>(d);
            if (qq == 0)
                sc[16 * w + kq] = live_key ? d * a.scale_log2 + (mrow ? mrow[key] * LOG2E : 0.0f) : -INFINITY;
        }
        __syncthreads();
        if (w == 0) {
            const float s = sc[lane];
            const float tmax = wave_max(s);
            const float m_new = fmaxf(m_run, tmax);
            const float p = exp2_unless(s == -INFINITY, s - m_new);
            ps[lane] = F16 ? (float)to_half(p) : p;
            const float tsum = wave_sum(p);
            if (lane == 0) {
                st[0] = m_new;
                st[1] = exp2_unless(m_run == -INFINITY, m_run - m_new);
                st[2] = tsum;
            }
        }
        __syncthreads();
        const float alpha = st[1];
        m_run = st[0];
        l_run = alpha * l_run + st[2];
        if (pv_on) {
            const int nk = min(GTK, k1 - kb);
            f32x4 acc = o * alpha;
            const char * vcol = a.kc + (size_t)kb * a.kc_nb1 + (size_t)(4 * cc) * ES;
            // keys kg, kg + n_kg, ... of the tile, VB at a time (loads issued before use)
            constexpr int VB = 16;
            for (int j0 = kg; j0 < nk; j0 += n_kg * VB) {
                // raw 16 (f32) or 8 (f16) bytes per key, selected to zero past the tile's keys;
                // converted only in the use loop, so that the loads stay one batch
                typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
                u32x4 v4[F16 ? 1 : VB];
                u32x2 v2[F16 ? VB : 1];
#pragma unroll
                for (int b = 0; b < VB; ++b) {
                    const int j = j0 + n_kg * b;
                    const char * pv = vcol + (size_t)min(j, nk - 1) * a.kc_nb1;
                    if constexpr (F16) {
                        const u32x2 x = *reinterpret_cast<const u32x2 *>(pv);
                        v2[b] = j < nk ? x : u32x2{0u, 0u};
                    } else {
                        const u32x4 x = *reinterpret_cast<const u32x4 *>(pv);
                        v4[b] = j < nk ? x : u32x4{0u, 0u, 0u, 0u};
                    }
                }
                f32x4 v[VB];
#pragma unroll
                for (int b = 0; b < VB; ++b) {
                    if constexpr (F16) {
                        const half4 hv = __builtin_bit_cast(half4, v2[b]);
                        v[b] = f32x4{(float)hv[0], (float)hv[1], (float)hv[2], (float)hv[3]};
                    } else {
                        v[b] = __builtin_bit_cast(f32x4, v4[b]);
                    }
                }
#pragma unroll
                for (int b = 0; b < VB; ++b) {
                    const float p = ps[min(j0 + n_kg * b, GTK - 1)];     // past nk: v is zero
                    acc[0] = fmaf(p, v[b][0], acc[0]);
                    acc[1] = fmaf(p, v[b][1], acc[1]);
                    acc[2] = fmaf(p, v[b][2], acc[2]);
                    acc[3] = fmaf(p, v[b][3], acc[3]);
                }
            }
            o = acc;
        }
        __syncthreads();
    }
    // the key classes' partial outputs summed (class 0 keeps the result)
    if (n_kg > 1) {
        ored[tid] = o;
        __syncthreads();
        if (kg == 0 && pv_on) {
            for (int g2 = 1; g2 < n_kg; ++g2) o += ored[g2 * n_cc + cc];
        }
    }
    const bool writer = kg == 0 && pv_on;

    if (a.dst != nullptr) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        if (writer) *reinterpret_cast<f32x4 *>(a.dst + ((size_t)h * a.nt + t) * dv + 4 * cc) = o * inv;
        return;
    }
    constexpr int OB = F16 ? 2 : 4;
    char * rec = part_record(a.part, h / PART_HEADS, a.nt, t, a.n_split, dv, OB);
    const int hh = h % PART_HEADS;
    char * blk = rec + part_o_off(a.n_split, sp, dv, OB);
    if (tid == 0)
        *reinterpret_cast<f32x2 *>(rec + part_ml_off(a.n_split, hh, sp)) = f32x2{(m_run == -INFINITY) ? -INFINITY : m_run * LN2, l_run};
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    if (writer) {
        const f32x4 r = o * inv;
        if (F16) *reinterpret_cast<half4 *>(reinterpret_cast<half_t *>(blk) + (size_t)hh * dv + 4 * cc) =
                     half4{to_half(r[0]), to_half(r[1]), to_half(r[2]), to_half(r[3])};
        else *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(blk) + (size_t)hh * dv + 4 * cc) = r;
    }
}

// The PHASE merge: one workgroup per (64 output columns, head, token).
template <typename OT>
__global__ __launch_bounds__(256) void merge_kernel(const char * __restrict__ part, int dv, int n_split,
                                                    int nt, float * __restrict__ dst) {
    __shared__ MergeScratch sc;
    merge_unit<OT>(part, dv, n_split, nt, blockIdx.x, blockIdx.y, blockIdx.z, dst, sc);
}

}  // namespace

hipError_t launch_kqkv_generic(int dk, int dv, int kc_is_f16, const DecodeArgs & a, hipStream_t stream) {
    if (dk > GMAX_DK || dv > GMAX_DV || dv % 4 != 0) return hipErrorInvalidValue;
    dim3 grid(a.n_split, a.n_head, a.nt);
    if (kc_is_f16)
        hipLaunchKernelGGL((kqkv_generic_kernel<true>), grid, dim3(256), 0, stream, a, dk, dv);
    else
        hipLaunchKernelGGL((kqkv_generic_kernel<false>), grid, dim3(256), 0, stream, a, dk, dv);
    return hipGetLastError();
}

// The PHASE merge for a few splits (chunked prefill: many tokens, S <= MERGE_FEW): one thread per
// (token, head, 8 output columns) folding the S partials in order -- a wavefront covers 64 chunks
// of one head's row, so every split's o / l is read as contiguous 1 KB (f16) and the header as a
// broadcast.  The same combine as merge_unit: m* = max m_s, l* = sum l_s e^(m_s - m*),
// out = sum l_s e^(m_s - m*) (o_s / l_s) / l*, 0 when every split is empty.
constexpr int MERGE_FEW = 16;

template <typename OT>
__global__ __launch_bounds__(256) void merge_few_kernel(const char * __restrict__ part, int dv, int n_split, int nt,
                                                        int n_head, float * __restrict__ dst) {
    const int c8n = dv / 8;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)nt * n_head * c8n) return;
    const int c8 = (int)(idx % c8n);
    const int h = (int)((idx / c8n) % n_head);
    const int t = (int)(idx / ((int64_t)c8n * n_head));
    const int hh = h % PART_HEADS;
    const char * rec = part_record(part, h / PART_HEADS, nt, t, n_split, dv, (int)sizeof(OT));
    float ms[MERGE_FEW], ls[MERGE_FEW];
    float m = -INFINITY;
    for (int s = 0; s < n_split; ++s) {
        const f32x2 ml = *reinterpret_cast<const f32x2 *>(rec + part_ml_off(n_split, hh, s));
        ms[s] = ml[0];
        ls[s] = ml[1];
        m = fmaxf(m, ms[s]);
    }
    float L = 0.0f;
    float O[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < n_split; ++s) {
        const float f = ls[s] * exp2_unless(ms[s] == -INFINITY, (ms[s] - m) * LOG2E);
        L += f;
        if (ms[s] == -INFINITY) continue;   // an empty split's o block is never written
        const OT * src = reinterpret_cast<const OT *>(rec + part_o_off(n_split, s, dv, (int)sizeof(OT))) + (size_t)hh * dv + 8 * c8;
        if constexpr (sizeof(OT) == 2) {
            const half8 v = *reinterpret_cast<const half8 *>(src);
#pragma unroll
            for (int k = 0; k < 8; ++k) O[k] += f * (float)v[k];
        } else {
            const f32x4 v0 = *reinterpret_cast<const f32x4 *>(src);
            const f32x4 v1 = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
            for (int k = 0; k < 4; ++k) { O[k] += f * v0[k]; O[4 + k] += f * v1[k]; }
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    float * d = dst + ((size_t)h * nt + t) * dv + 8 * c8;
    *reinterpret_cast<f32x4 *>(d) = f32x4{O[0] * inv, O[1] * inv, O[2] * inv, O[3] * inv};
    *reinterpret_cast<f32x4 *>(d + 4) = f32x4{O[4] * inv, O[5] * inv, O[6] * inv, O[7] * inv};
}

hipError_t launch_merge(const char * part, int dv, int o_bytes, int n_split, int nt, int n_head, float * dst,
                        hipStream_t stream) {
    if (dv % 8 != 0) return hipErrorInvalidValue;
    // few splits over many (token, head) rows: a thread per 8 columns; otherwise (decode: hundreds
    // of splits, one token) a workgroup per 64 columns with the splits across its lanes
    if (n_split <= MERGE_FEW && (int64_t)nt * n_head >= 256) {
        const int64_t threads = (int64_t)nt * n_head * (dv / 8);
        const dim3 grid((unsigned)((threads + 255) / 256));
        if (o_bytes == 2)
            hipLaunchKernelGGL(merge_few_kernel<half_t>, grid, dim3(256), 0, stream, part, dv, n_split, nt, n_head, dst);
        else if (o_bytes == 4)
            hipLaunchKernelGGL(merge_few_kernel<float>, grid, dim3(256), 0, stream, part, dv, n_split, nt, n_head, dst);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    }
    dim3 grid((dv + 63) / 64, n_head, nt);
    if (o_bytes == 2)
        hipLaunchKernelGGL(merge_kernel<half_t>, grid, dim3(256), 0, stream, part, dv, n_split, nt, dst);
    else if (o_bytes == 4)
        hipLaunchKernelGGL(merge_kernel<float>, grid, dim3(256), 0, stream, part, dv, n_split, nt, dst);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace mla

// kqkv_generic.hip -- the VALU attention kernel (f32 caches and geometries outside the MFMA
// instantiations) and the split-K merge.
//
// Generic kernel: one workgroup (4 waves) per (split, head, token).  Per 64-key tile, each wave
// scores 16 keys with a lane-strided dot over D_k and a wavefront sum; wave 0 then does the
// online-softmax bookkeeping for the tile; every thread accumulates its output columns against the
// coalesced V rows.  F32 caches run in f32 end to end, like ggml-cpu's F32 mul_mat; with an F16
// cache q and P are rounded to f16 first (the F16 vec_dot_type conversion), matching the MFMA path.
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
constexpr int GMAX_OPT = 4;     // output columns per thread (D_v <= 1024)

template <bool F16>
__global__ __launch_bounds__(256) void kqkv_generic_kernel(DecodeArgs a, int dk, int dv) {
    __shared__ float qs[GMAX_DK];
    __shared__ float sc[GTK];
    __shared__ float ps[GTK];
    __shared__ float st[3];          // m_new, alpha, tile sum

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int sp = blockIdx.x, h = blockIdx.y, t = blockIdx.z;

    const float * qrow = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 + (size_t)h * a.q_nb1);
    for (int k = tid; k < dk; k += 256) {
        const float x = qrow[k];
        qs[k] = F16 ? (float)to_half(x) : x;
    }
    const float * mrow = a.mask ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1) : nullptr;

    const int base_t = a.n_tiles / a.n_split, rem = a.n_tiles % a.n_split;
    const int t0 = sp * base_t + min(sp, rem);
    const int t1 = t0 + base_t + (sp < rem ? 1 : 0);

    float o[GMAX_OPT];
#pragma unroll
    for (int i = 0; i < GMAX_OPT; ++i) o[i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    __syncthreads();

    for (int tile = t0; tile < t1; ++tile) {
        const int kb = tile * GTK;
        // scores: wave w -> keys kb + 16 w .. +15
        for (int j = 0; j < 16; ++j) {
            const int key = kb + 16 * w + j;
            float d = 0.0f;
            if (key < a.n_kv) {
                const char * row = a.kc + (size_t)key * a.kc_nb1;
                for (int k = lane; k < dk; k += 64) {
                    const float kv = F16 ? (float)reinterpret_cast<const half_t *>(row)[k] : reinterpret_cast<const float *>(row)[k];
                    d += kv * qs[k];
                }
            }
            d = wave_sum(d);
            if (lane == 0)
                sc[16 * w + j] = (key < a.n_kv) ? d * a.scale_log2 + (mrow ? mrow[key] * LOG2E : 0.0f) : -INFINITY;
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
        const int nk = min(GTK, a.n_kv - kb);
#pragma unroll
        for (int i = 0; i < GMAX_OPT; ++i) {
            const int c = tid + 256 * i;
            if (c >= dv) break;
            float acc = o[i] * alpha;
            for (int j = 0; j < nk; ++j) {
                const char * row = a.kc + (size_t)(kb + j) * a.kc_nb1;
                const float vv = F16 ? (float)reinterpret_cast<const half_t *>(row)[c] : reinterpret_cast<const float *>(row)[c];
                acc += ps[j] * vv;
            }
            o[i] = acc;
        }
        __syncthreads();
    }

    if (a.dst != nullptr) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        float * drow = a.dst + ((size_t)h * a.nt + t) * dv;
#pragma unroll
        for (int i = 0; i < GMAX_OPT; ++i) {
            const int c = tid + 256 * i;
            if (c < dv) drow[c] = o[i] * inv;
        }
        return;
    }
    constexpr int OB = F16 ? 2 : 4;
    char * rec = part_record(a.part, h / PART_HEADS, a.nt, t, a.n_split, dv, OB);
    const int hh = h % PART_HEADS;
    char * blk = rec + part_o_off(a.n_split, sp, dv, OB);
    if (tid == 0)
        *reinterpret_cast<f32x2 *>(rec + part_ml_off(a.n_split, hh, sp)) = f32x2{(m_run == -INFINITY) ? -INFINITY : m_run * LN2, l_run};
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
    for (int i = 0; i < GMAX_OPT; ++i) {
        const int c = tid + 256 * i;
        if (c >= dv) continue;
        if (F16) reinterpret_cast<half_t *>(blk)[(size_t)hh * dv + c] = to_half(o[i] * inv);
        else reinterpret_cast<float *>(blk)[(size_t)hh * dv + c] = o[i] * inv;
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
    if (dk > GMAX_DK || dv > 256 * GMAX_OPT) return hipErrorInvalidValue;
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

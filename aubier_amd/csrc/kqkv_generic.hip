// kqkv_generic.hip -- the VALU attention kernel (f32 caches and geometries outside the MFMA
// instantiations) and the split-K merge.
//
// Generic kernel: one workgroup (4 waves) per (split, head, token).  Per 64-key tile, each wave
// scores 16 keys with a lane-strided dot over D_k and a wavefront sum; wave 0 then does the
// online-softmax bookkeeping for the tile; every thread accumulates its output columns against the
// coalesced V rows.  F32 caches run in f32 end to end, like ggml-cpu's F32 mul_mat; with an F16
// cache q and P are rounded to f16 first (the F16 vec_dot_type conversion), matching the MFMA path.
//
// Merge kernel (GGML_OP_M4_PHASE phase 2; the combine of patches/ggml-m4/m4-kqkv.cu:314-338):
// 16 column-lanes x 16 split-lanes per workgroup, each split-lane folding its splits with the
// online LSE rule, then one fold across split-lanes through LDS.
#include "mla_common.h"
#include "mla_kernels.h"

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
            const float p = (s == -INFINITY) ? 0.0f : exp2_fast(s - m_new);
            ps[lane] = F16 ? (float)to_half(p) : p;
            const float tsum = wave_sum(p);
            if (lane == 0) {
                st[0] = m_new;
                st[1] = (m_run == -INFINITY) ? 0.0f : exp2_fast(m_run - m_new);
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
    float * rec = a.part + (((size_t)h * a.nt + t) * a.n_split + sp) * (size_t)(4 + dv);
    if (tid == 0) {
        rec[0] = (m_run == -INFINITY) ? -INFINITY : m_run * LN2;
        rec[1] = l_run;
        rec[2] = 0.0f;
        rec[3] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < GMAX_OPT; ++i) {
        const int c = tid + 256 * i;
        if (c < dv) rec[4 + c] = o[i];
    }
}

__global__ __launch_bounds__(256) void merge_kernel(const float * __restrict__ part, int dv, int n_split,
                                                    int nt, float * __restrict__ dst) {
    __shared__ float sm[16][16];
    __shared__ float sl[16][16];
    __shared__ float4 so[16][16];
    const int tid = threadIdx.x;
    const int cl = tid & 15, sl_i = tid >> 4;
    const int c = blockIdx.x * 64 + 4 * cl;
    const int t = blockIdx.y, h = blockIdx.z;
    const size_t rs = (size_t)(4 + dv);
    const float * base = part + ((size_t)h * nt + t) * n_split * rs;

    float m = -INFINITY, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = sl_i; s < n_split; s += 16) {
        const float * r = base + (size_t)s * rs;
        const float ms = r[0];
        if (ms == -INFINITY) continue;
        const float ls = r[1];
        const float4 os = (c < dv) ? *reinterpret_cast<const float4 *>(r + 4 + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (ms > m) {
            const float f = (m == -INFINITY) ? 0.0f : exp2_fast((m - ms) * LOG2E);
            l *= f; o.x *= f; o.y *= f; o.z *= f; o.w *= f;
            m = ms;
        }
        const float f = exp2_fast((ms - m) * LOG2E);
        l += ls * f;
        o.x += os.x * f; o.y += os.y * f; o.z += os.z * f; o.w += os.w * f;
    }
    sm[sl_i][cl] = m;
    sl[sl_i][cl] = l;
    so[sl_i][cl] = o;
    __syncthreads();
    if (sl_i == 0 && c < dv) {
        float M = -INFINITY;
        for (int i = 0; i < 16; ++i) M = fmaxf(M, sm[i][cl]);
        float4 out = make_float4(0.f, 0.f, 0.f, 0.f);
        if (M > -INFINITY) {
            float L = 0.0f;
            float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int i = 0; i < 16; ++i) {
                const float mi = sm[i][cl];
                if (mi == -INFINITY) continue;
                const float f = exp2_fast((mi - M) * LOG2E);
                L += sl[i][cl] * f;
                const float4 oi = so[i][cl];
                O.x += oi.x * f; O.y += oi.y * f; O.z += oi.z * f; O.w += oi.w * f;
            }
            const float inv = 1.0f / L;
            out = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
        }
        *reinterpret_cast<float4 *>(dst + ((size_t)h * nt + t) * dv + c) = out;
    }
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

hipError_t launch_merge(const float * part, int dv, int n_split, int nt, int n_head, float * dst,
                        hipStream_t stream) {
    dim3 grid((dv + 63) / 64, nt, n_head);
    hipLaunchKernelGGL(merge_kernel, grid, dim3(256), 0, stream, part, dv, n_split, nt, dst);
    return hipGetLastError();
}

}  // namespace mla

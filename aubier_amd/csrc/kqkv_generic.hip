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
    char * blk = a.part + (((size_t)(h / PART_HEADS) * a.nt + t) * a.n_split + sp) * part_block_bytes(dv, F16 ? 2 : 4);
    const int hh = h % PART_HEADS;
    if (tid == 0) {
        float * hdr = reinterpret_cast<float *>(blk);
        hdr[hh] = (m_run == -INFINITY) ? -INFINITY : m_run * LN2;
        hdr[PART_HEADS + hh] = l_run;
    }
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
    for (int i = 0; i < GMAX_OPT; ++i) {
        const int c = tid + 256 * i;
        if (c >= dv) continue;
        if (F16) reinterpret_cast<half_t *>(blk + 256)[(size_t)hh * dv + c] = to_half(o[i] * inv);
        else reinterpret_cast<float *>(blk + 256)[(size_t)hh * dv + c] = o[i] * inv;
    }
}

// One workgroup per (64 output columns, head, token): 8 column-lanes (8 f16 columns = 16 bytes
// each) x 32 split-lanes.  Split-lane sl takes splits sl, sl + 32, ...: the loads of a 256-split
// chunk (16 bytes of o/l plus m, l) all issue before the first use, then the chunk is folded with
// the max taken first.  Split-lanes are combined with wavefront shuffles, then across the four
// wavefronts through LDS.  Accumulators: (m, L = sum l_s e^(m_s - m), O = sum l_s e^(m_s - m) o_s).
template <typename OT>
__global__ __launch_bounds__(256) void merge_kernel(const char * __restrict__ part, int dv, int n_split,
                                                    int nt, float * __restrict__ dst) {
    constexpr int J = 8;
    __shared__ float sm[4][8];
    __shared__ float sL[4][8];
    __shared__ f32x4 sO[4][8][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c8 = tid & 7, sl_i = tid >> 3;               // column lane, split lane (0..31)
    const int c = blockIdx.x * 64 + 8 * c8;
    const int h = blockIdx.y, t = blockIdx.z;
    const int hh = h % PART_HEADS;
    const size_t bb = part_block_bytes(dv, (int)sizeof(OT));
    const char * base = part + ((size_t)(h / PART_HEADS) * nt + t) * n_split * bb;
    const int cc = min(c, dv - 8);

    float m = -INFINITY, L = 0.0f;
    float O[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_split; s0 += 32 * J) {
        float ms[J], ls[J];
        float os[J][8];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int s = s0 + 32 * j + sl_i;
            const char * blk = base + (size_t)min(s, n_split - 1) * bb;
            const float mv = reinterpret_cast<const float *>(blk)[hh];
            ms[j] = (s < n_split) ? mv : -INFINITY;
            ls[j] = reinterpret_cast<const float *>(blk)[PART_HEADS + hh];
            const OT * src = reinterpret_cast<const OT *>(blk + 256) + (size_t)hh * dv + cc;
            if constexpr (sizeof(OT) == 2) {
                const half8 v = *reinterpret_cast<const half8 *>(src);
#pragma unroll
                for (int k = 0; k < 8; ++k) os[j][k] = (float)v[k];
            } else {
                const f32x4 v0 = *reinterpret_cast<const f32x4 *>(src);
                const f32x4 v1 = *reinterpret_cast<const f32x4 *>(src + 4);
#pragma unroll
                for (int k = 0; k < 4; ++k) { os[j][k] = v0[k]; os[j][4 + k] = v1[k]; }
            }
        }
        float mx = m;
#pragma unroll
        for (int j = 0; j < J; ++j) mx = fmaxf(mx, ms[j]);
        const float f0 = (m == -INFINITY) ? 0.0f : exp2_fast((m - mx) * LOG2E);
        L *= f0;
#pragma unroll
        for (int k = 0; k < 8; ++k) O[k] *= f0;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float f = (ms[j] == -INFINITY) ? 0.0f : ls[j] * exp2_fast((ms[j] - mx) * LOG2E);
            L += f;
#pragma unroll
            for (int k = 0; k < 8; ++k) O[k] += f * os[j][k];
        }
        m = mx;
    }
    // fold the 8 split-lanes of this wavefront (lane bits 3..5)
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
        const float m2 = shfl_xor(m, off);
        const float L2 = shfl_xor(L, off);
        const float M = fmaxf(m, m2);
        const float f1 = (m == -INFINITY) ? 0.0f : exp2_fast((m - M) * LOG2E);
        const float f2 = (m2 == -INFINITY) ? 0.0f : exp2_fast((m2 - M) * LOG2E);
        L = L * f1 + L2 * f2;
#pragma unroll
        for (int k = 0; k < 8; ++k) O[k] = O[k] * f1 + shfl_xor(O[k], off) * f2;
        m = M;
    }
    if (lane < 8) {
        sm[w][c8] = m;
        sL[w][c8] = L;
        sO[w][c8][0] = f32x4{O[0], O[1], O[2], O[3]};
        sO[w][c8][1] = f32x4{O[4], O[5], O[6], O[7]};
    }
    __syncthreads();
    if (tid < 8 && c < dv) {
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) M = fmaxf(M, sm[i][c8]);
        f32x4 r0 = {0.f, 0.f, 0.f, 0.f}, r1 = {0.f, 0.f, 0.f, 0.f};
        if (M > -INFINITY) {
            float LL = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float f = (sm[i][c8] == -INFINITY) ? 0.0f : exp2_fast((sm[i][c8] - M) * LOG2E);
                LL += sL[i][c8] * f;
                r0 += sO[i][c8][0] * f;
                r1 += sO[i][c8][1] * f;
            }
            const float inv = 1.0f / LL;
            r0 *= inv;
            r1 *= inv;
        }
        float * d = dst + ((size_t)h * nt + t) * dv + c;
        *reinterpret_cast<f32x4 *>(d) = r0;
        *reinterpret_cast<f32x4 *>(d + 4) = r1;
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

hipError_t launch_merge(const char * part, int dv, int o_bytes, int n_split, int nt, int n_head, float * dst,
                        hipStream_t stream) {
    if (dv % 8 != 0) return hipErrorInvalidValue;
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

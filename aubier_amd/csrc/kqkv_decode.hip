// kqkv_decode.hip -- split-K MLA decode attention over an f16 latent+rope KV cache, on MFMA.
//
// The pass-1 kernel of GGML_OP_M4_KQKV (reference: patches/ggml-m4/m4-kqkv.cu:201-312), designed
// for gfx950 rather than translated:
//   * ALL heads of a 32-head group live in one workgroup, so every KV byte is fetched from HBM
//     exactly once per token (MLA's single latent row serves every head).
//   * Q.K^T and P.V are dense contractions ([32 x D_k].[D_k x keys] and [32 x keys].[keys x D_v],
//     60 FLOP per cache byte): they run on v_mfma_f32_16x16x32_f16 / v_mfma_f32_32x32x16_f16 with
//     f32 accumulation.  q and P enter the MFMA as f16 -- the same rounding points as the unfused
//     ggml-cpu graph, whose mul_mat converts src1 to F16 for an F16 src0.
//   * The cache streams through 64-key tiles: coalesced 16-byte global loads into registers for
//     tile i+1 while tile i is computed out of LDS (rows padded by 16 bytes so the MFMA operand
//     reads are bank-conflict free).
//   * Online softmax in log2 units (v_exp_f32), rescaling the accumulators only by the per-tile
//     factor; all-masked prefixes are guarded (no exp(-inf - -inf)).
//
// Work split: grid = (n_split, ceil(H/32), nt), 512 threads = 8 waves.
//   QK role:  wave w -> key group kg = w & 3 (16 keys of the tile), head tile ht = w >> 2 (16 heads)
//   PV role:  wave w -> output columns [w*D_v/8, (w+1)*D_v/8), all 32 heads
// Output: one partial record per (head, token, split) = {m (natural log), l, 0, 0, o[D_v]}
// (unnormalised), or -- when the launch has a single split -- the final o/l written to dst.
#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

constexpr int TK = 64;          // keys per tile
constexpr int NTHR = 512;       // threads per workgroup
constexpr int HG = 32;          // heads per workgroup

template <int DK, int DV>
struct DecodeCfg {
    static_assert(DK % 32 == 0 && DV % 256 == 0 && DV <= DK, "geometry");
    static constexpr int KROW = DK + 8;                 // LDS row pitch in halves (+16 bytes)
    static constexpr int CH = DK * 2 / 16;              // 16-byte chunks per cache row
    static constexpr int NCHUNK = TK * CH;
    static constexpr int NPT = (NCHUNK + NTHR - 1) / NTHR;   // staged chunks per thread
    static constexpr int QSTEPS = DK / 32;              // K-steps of the 16x16x32 MFMA
    static constexpr int DVW = DV / 8;                  // output columns per wave
    static constexpr int NT_DV = DVW / 32;              // 32-wide MFMA tiles per wave
    static constexpr int PROW = TK + 8;                 // P row pitch in halves
};

template <int DK, int DV>
__global__ __launch_bounds__(NTHR, 1) void kqkv_decode_f16_kernel(DecodeArgs a) {
    using C = DecodeCfg<DK, DV>;
    __shared__ __attribute__((aligned(16))) half_t kt[TK * C::KROW];
    __shared__ __attribute__((aligned(16))) half_t pl[HG * C::PROW];
    __shared__ float red_max[4][HG];
    __shared__ float red_sum[4][HG];
    __shared__ __attribute__((aligned(16))) float alpha_s[HG];
    __shared__ __attribute__((aligned(16))) float l_fin[HG];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int sp = blockIdx.x;
    const int hg0 = blockIdx.y * HG;
    const int t = blockIdx.z;

    // ---- split range (balanced partition of whole tiles) ----
    const int base_t = a.n_tiles / a.n_split;
    const int rem = a.n_tiles % a.n_split;
    const int t0 = sp * base_t + min(sp, rem);
    const int t1 = t0 + base_t + (sp < rem ? 1 : 0);

    // ---- QK-role constants ----
    const int kg = w & 3;
    const int ht = w >> 2;
    const int qk_head = hg0 + 16 * ht + (lane & 15);     // this lane's head (B/C column)

    // q^T fragments (B operand), f32 -> f16 once: lane holds head qk_head, d = 32 s + 8 (lane>>4) .. +7
    half8 qreg[C::QSTEPS];
    {
        const bool hv = qk_head < a.n_head;
        const char * qrow = reinterpret_cast<const char *>(a.q) + (size_t)t * a.q_nb2 +
                            (size_t)(hv ? qk_head : 0) * a.q_nb1;
#pragma unroll
        for (int s = 0; s < C::QSTEPS; ++s) {
            const float4 * src = reinterpret_cast<const float4 *>(qrow) + (32 * s + 8 * (lane >> 4)) / 4;
            float4 x0 = hv ? src[0] : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 x1 = hv ? src[1] : make_float4(0.f, 0.f, 0.f, 0.f);
            half8 h;
            h[0] = to_half(x0.x); h[1] = to_half(x0.y); h[2] = to_half(x0.z); h[3] = to_half(x0.w);
            h[4] = to_half(x1.x); h[5] = to_half(x1.y); h[6] = to_half(x1.z); h[7] = to_half(x1.w);
            qreg[s] = h;
        }
    }

    const float * mrow = a.mask ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.mask) + (size_t)t * a.mask_nb1) : nullptr;

    // ---- running state ----
    float m_run = -INFINITY;   // log2 units, for head qk_head (replicated across the 4 kg waves)
    float l_run = 0.0f;
    f32x16 o[C::NT_DV];
#pragma unroll
    for (int i = 0; i < C::NT_DV; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;

    // ---- tile staging ----
    u32x4 stg[C::NPT];
    auto issue = [&](int tile) {
        const int kbase = tile * TK;
#pragma unroll
        for (int i = 0; i < C::NPT; ++i) {
            const int c = i * NTHR + tid;
            const int key = c / C::CH;
            const int cc = c - key * C::CH;
            const int gk = kbase + key;
            if (c < C::NCHUNK && gk < a.n_kv)
                stg[i] = ld16_stream(a.kc + (size_t)gk * a.kc_nb1 + (size_t)cc * 16);
            else
                stg[i] = u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < C::NPT; ++i) {
            const int c = i * NTHR + tid;
            if (c < C::NCHUNK) {
                const int key = c / C::CH;
                const int cc = c - key * C::CH;
                *reinterpret_cast<u32x4 *>(&kt[key * C::KROW + cc * 8]) = stg[i];
            }
        }
    };

    if (t0 < t1) issue(t0);

    for (int tile = t0; tile < t1; ++tile) {
        __syncthreads();                                  // (A) previous tile fully consumed
        commit();
        if (tile + 1 < t1) issue(tile + 1);
        __syncthreads();                                  // (B) tile in LDS

        // ---- S^T = K . Q^T : 16 keys x 16 heads per wave ----
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        {
            const half_t * arow = &kt[(16 * kg + (lane & 15)) * C::KROW + 8 * (lane >> 4)];
#pragma unroll
            for (int s = 0; s < C::QSTEPS; ++s) {
                const half8 av = *reinterpret_cast<const half8 *>(arow + 32 * s);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qreg[s], acc, 0, 0, 0);
            }
        }
        const int kbase = tile * TK;
        const int kl0 = 16 * kg + 4 * (lane >> 4);      // first of this lane's 4 keys (tile-local)
        float sc[4];
        float lmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int gk = kbase + kl0 + r;
            float v = -INFINITY;
            if (gk < a.n_kv) v = acc[r] * a.scale_log2 + (mrow ? mrow[gk] * LOG2E : 0.0f);
            sc[r] = v;
            lmax = fmaxf(lmax, v);
        }
        lmax = fmaxf(lmax, shfl_xor(lmax, 16));
        lmax = fmaxf(lmax, shfl_xor(lmax, 32));
        if (lane < 16) red_max[kg][16 * ht + lane] = lmax;
        __syncthreads();                                  // (C)

        const int hl = 16 * ht + (lane & 15);
        float tmax = fmaxf(fmaxf(red_max[0][hl], red_max[1][hl]), fmaxf(red_max[2][hl], red_max[3][hl]));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = (m_run == -INFINITY) ? 0.0f : exp2_fast(m_run - m_new);
        float psum = 0.0f;
        half4 ph;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float p = (sc[r] == -INFINITY) ? 0.0f : exp2_fast(sc[r] - m_new);
            psum += p;
            ph[r] = to_half(p);
        }
        *reinterpret_cast<half4 *>(&pl[hl * C::PROW + kl0]) = ph;
        psum += shfl_xor(psum, 16);
        psum += shfl_xor(psum, 32);
        if (lane < 16) {
            red_sum[kg][hl] = psum;
            if (kg == 0) alpha_s[hl] = alpha;
        }
        m_run = m_new;
        __syncthreads();                                  // (D)

        l_run = alpha * l_run + ((red_sum[0][hl] + red_sum[1][hl]) + (red_sum[2][hl] + red_sum[3][hl]));

        // ---- O[32 heads x DVW] = alpha * O + P . V ----
        {
            // lane's C rows: heads 8*(r/4) + 4*(lane>>5) + (r&3)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 al = *reinterpret_cast<const float4 *>(&alpha_s[8 * q4 + 4 * (lane >> 5)]);
#pragma unroll
                for (int i = 0; i < C::NT_DV; ++i) {
                    o[i][4 * q4 + 0] *= al.x;
                    o[i][4 * q4 + 1] *= al.y;
                    o[i][4 * q4 + 2] *= al.z;
                    o[i][4 * q4 + 3] *= al.w;
                }
            }
            const int dv0 = w * C::DVW + (lane & 31);
#pragma unroll
            for (int kk = 0; kk < TK / 16; ++kk) {
                const int key0 = 16 * kk + 8 * (lane >> 5);
                const half8 pa = *reinterpret_cast<const half8 *>(&pl[(lane & 31) * C::PROW + key0]);
#pragma unroll
                for (int i = 0; i < C::NT_DV; ++i) {
                    half8 vb;
#pragma unroll
                    for (int j = 0; j < 8; ++j) vb[j] = kt[(key0 + j) * C::KROW + dv0 + 32 * i];
                    o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, vb, o[i], 0, 0, 0);
                }
            }
        }
    }

    // ---- epilogue ----
    if (a.dst != nullptr) {
        // single split: normalise and write the final output dst [D_v, nt, H]
        __syncthreads();
        if (kg == 0 && lane < 16) l_fin[16 * ht + lane] = l_run;
        __syncthreads();
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int hloc = 8 * q4 + 4 * (lane >> 5) + r4;
                const int h = hg0 + hloc;
                if (h >= a.n_head) continue;
                const float l = l_fin[hloc];
                const float inv = l > 0.0f ? 1.0f / l : 0.0f;
                float * drow = a.dst + ((size_t)h * a.nt + t) * DV + w * C::DVW + (lane & 31);
#pragma unroll
                for (int i = 0; i < C::NT_DV; ++i) drow[32 * i] = o[i][4 * q4 + r4] * inv;
            }
        }
        return;
    }
    const size_t rs = (size_t)(4 + DV);
    if (kg == 0 && lane < 16) {
        const int h = hg0 + 16 * ht + lane;
        if (h < a.n_head) {
            float * rec = a.part + (((size_t)h * a.nt + t) * a.n_split + sp) * rs;
            const float m_nat = (m_run == -INFINITY) ? -INFINITY : m_run * LN2;
            *reinterpret_cast<float4 *>(rec) = make_float4(m_nat, l_run, 0.0f, 0.0f);
        }
    }
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int h = hg0 + 8 * q4 + 4 * (lane >> 5) + r4;
            if (h >= a.n_head) continue;
            float * rec = a.part + (((size_t)h * a.nt + t) * a.n_split + sp) * rs + 4 + w * C::DVW + (lane & 31);
#pragma unroll
            for (int i = 0; i < C::NT_DV; ++i) rec[32 * i] = o[i][4 * q4 + r4];
        }
    }
}

}  // namespace

template <int DK, int DV>
static hipError_t launch_decode(const DecodeArgs & a, int n_hgroups, hipStream_t stream) {
    dim3 grid(a.n_split, n_hgroups, a.nt);
    hipLaunchKernelGGL((kqkv_decode_f16_kernel<DK, DV>), grid, dim3(NTHR), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kqkv_decode_f16(int dk, int dv, const DecodeArgs & a, hipStream_t stream) {
    const int n_hgroups = (a.n_head + HG - 1) / HG;
    if (dk == 576 && dv == 512) return launch_decode<576, 512>(a, n_hgroups, stream);
    if (dk == 320 && dv == 256) return launch_decode<320, 256>(a, n_hgroups, stream);
    return hipErrorInvalidValue;
}

bool decode_f16_supported(int dk, int dv) {
    return (dk == 576 && dv == 512) || (dk == 320 && dv == 256);
}

}  // namespace mla

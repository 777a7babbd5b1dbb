// kqkv_flat.hip -- GGML_OP_M4_KQKV for short decode windows in ONE launch (the reference runs a window
// of up to 256 keys as a single flat launch, one block per head: patches/ggml-m4/m4-kqkv.cu:161-199,
// 363-367).  A launch in a graph costs ~1.85 us on this part, so for a 256-key window the split-K
// partial + merge pair spent more time launching than computing.
//
// Design (gfx950, not a translation): one workgroup per (split, head) of one token -- splits of at
// most FLAT_KEYS keys, so that a short window still spreads over ~256 workgroups -- and the merge
// folded into the same launch:
//   * every load the workgroup needs (q row, the split's K/V rows by LDS DMA, its mask values) is
//     issued at once: one memory round trip.  The rows land padded by 128 bytes, so that the 16-lane
//     groups of Q.K^T's reads hit distinct banks;
//   * Q.K^T: 8 threads per key, each a strided eighth of the row, summed by DPP; the exact softmax
//     of the split (all its keys are present); P.V: each thread owns 2 output columns;
//   * the split's record (m, l, unnormalised o, f32) goes to the workspace by device-coherent stores,
//     and once they are acknowledged thread 0 takes a ticket on the head's counter (agent-scope
//     atomic: the XCDs' L2s are not coherent with each other).  The workgroup that takes the last
//     ticket reads the head's records back by device-coherent loads, merges them (log-sum-exp)
//     into dst and resets the counter to zero for the next launch.  No workgroup ever waits for
//     another, so every launch drains whatever the scheduling.
// F32 caches run in f32 end to end (ggml-cpu's F32 mul_mat); with an F16 cache q and P are rounded
// to f16 first, as the other kernels do.
#include "mla_common.h"
#include "mla_kernels.h"

namespace mla {

namespace {

constexpr int FTHR = 256;

struct FlatLds {
    __attribute__((aligned(16))) char rows[FLAT_KEYS * FLAT_ROW_PITCH];   // K/V rows (padded), f32 or f16
    __attribute__((aligned(16))) float q[FLAT_DK_MAX];
    __attribute__((aligned(16))) float s[FLAT_KEYS];                    // scores, then P
    float ml[2];                                                        // split max (log2 units), l
    int last;
};

template <bool F16>
__global__ __launch_bounds__(FTHR) void kqkv_flat_kernel(FlatArgs a) {
    constexpr int ES = F16 ? 2 : 4;
    constexpr int EPC = 16 / ES;                       // elements per 16-byte chunk
    __shared__ FlatLds sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int sp = blockIdx.x, h = blockIdx.y;
    const int dk = a.dk, dv = a.dv;

    // ---- the split's keys [k0, k1) (balanced), everything loaded in one round trip ----
    const int base = a.n_kv / a.n_split, rem = a.n_kv % a.n_split;
    const int k0 = sp * base + min(sp, rem);
    const int nk = base + (sp < rem ? 1 : 0);
    const int cpr = dk / EPC;                          // 16-byte chunks per row (dk % EPC == 0)
    // K/V rows by LDS DMA straight into the padded layout: LDS chunk k = 64 i + lane of instruction i
    // is chunk k % PCH of row k / PCH; chunks past the row, rows past the split and anything past
    // n_kv come back as zeros from the buffer range check (no memory access)
    constexpr int PCH = FLAT_ROW_PITCH / 16;
    constexpr int NDMA = FLAT_KEYS * PCH / 64;        // DMA instructions per workgroup
    static_assert(FLAT_KEYS * PCH % 64 == 0 && NDMA % 4 == 0, "whole DMA instructions, even over the waves");
    {
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t nrec = nk > 0 ? (uint32_t)((int64_t)(nk - 1) * a.kc_nb1 + dk * ES) : 0u;
        const i32x4 rs = make_rsrc(a.kc + (int64_t)k0 * a.kc_nb1, nrec);
        const uint32_t lds0 = lds_addr(sh.rows);
#pragma unroll
        for (int i = 0; i < NDMA / 4; ++i) {
            const int ii = (NDMA / 4) * w + i;
            const int k = 64 * ii + lane;
            const int r = k / PCH, x = k - r * PCH;
            const uint32_t off = (x < cpr && r < nk) ? (uint32_t)((int64_t)r * a.kc_nb1) + 16u * (uint32_t)x : 0xFFFFFFE0u;   // (+12 stays out of range)
            dma16(rs, off, 0u, lds0 + (uint32_t)(1024 * ii));
        }
    }
    const float * qrow = a.q + (size_t)h * (a.q_nb1 / 4);
    constexpr int QPT = (FLAT_DK_MAX + FTHR - 1) / FTHR;     // q values per thread
    float qv[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const int k = tid + FTHR * i;
        qv[i] = k < dk ? qrow[k] : 0.0f;
    }
    const float mk = (a.mask != nullptr && tid < nk) ? a.mask[k0 + tid] : 0.0f;
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const int k = tid + FTHR * i;
        if (k < dk) sh.q[k] = F16 ? (float)to_half(qv[i]) : qv[i];
    }
    wait_vm<0>();                                      // this wave's DMA (and q loads) have landed
    __syncthreads();

    // ---- Q.K^T: thread (key j = tid >> 3, part p = tid & 7) sums chunks p, p + 8, ... of row j,
    // every LDS read of the row issued before the first product ----
    {
        constexpr int CPT = (FLAT_DK_MAX * ES / 16 + 7) / 8;      // chunks per thread at most
        const int j = tid >> 3, p = tid & 7;
        const char * row = sh.rows + j * FLAT_ROW_PITCH;
        u32x4 kv[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) kv[i] = *reinterpret_cast<const u32x4 *>(row + 16 * min(p + 8 * i, PCH - 1));
        // the chunks past the row (c >= cpr) are the zeros the DMA wrote into the row's padding, so
        // no lane needs a guard: their q index is clamped and their products are 0 (a guard
        // depending on the lane kept every q read in its own round trip)
        f32x4 qv4[CPT][EPC / 4];
#pragma unroll
        for (int i = 0; i < CPT; ++i)
#pragma unroll
            for (int hq = 0; hq < EPC / 4; ++hq)
                qv4[i][hq] = *reinterpret_cast<const f32x4 *>(&sh.q[EPC * min(p + 8 * i, cpr - 1) + 4 * hq]);
        f32x4 dacc = {0.0f, 0.0f, 0.0f, 0.0f};       // four independent product chains
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            if constexpr (F16) {
                const half8 hv = __builtin_bit_cast(half8, kv[i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) dacc[e] = fmaf((float)hv[e], qv4[i][0][e], dacc[e]);
#pragma unroll
                for (int e = 0; e < 4; ++e) dacc[e] = fmaf((float)hv[4 + e], qv4[i][1][e], dacc[e]);
            } else {
                const f32x4 fv = __builtin_bit_cast(f32x4, kv[i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) dacc[e] = fmaf(fv[e], qv4[i][0][e], dacc[e]);
            }
        }
        const float d0 = dacc[0] + dacc[2], d1 = dacc[1] + dacc[3];
        float d = d0 + d1;
        d += dpp_xor<1>(d);
        d += dpp_xor<2>(d);
        d += dpp_xor<4>(d);
        if (p == 0 && j < FLAT_KEYS) sh.s[j] = j < nk ? d * a.scale_log2 : -INFINITY;
    }
    __syncthreads();
    // ---- the split's softmax (wave 0): its exact max, P = 2^(s - m), l = sum P ----
    if (tid < 64) {
        const float s = tid < FLAT_KEYS ? sh.s[tid] + (tid < nk ? mk * LOG2E : 0.0f) : -INFINITY;
        const float m = wave_max(s);
        const float pr = exp2_unless(s == -INFINITY, s - m);      // m = -inf only if s is -inf too
        const float p = F16 ? (float)to_half(pr) : pr;
        const float l = wave_sum(p);
        if (tid < FLAT_KEYS) sh.s[tid] = p;
        if (tid == 0) {
            sh.ml[0] = m;
            sh.ml[1] = l;
        }
    }
    __syncthreads();
    // ---- P.V: thread t owns columns 2 t, 2 t + 1; the split's rows past nk are zeros in LDS and
    // their P is 0, so all FLAT_KEYS rows are read, every read before the first product ----
    float o0 = 0.0f, o1 = 0.0f;
    const int col = 2 * tid;
    if (col < dv) {
        f32x2 v[FLAT_KEYS];
#pragma unroll
        for (int j = 0; j < FLAT_KEYS; ++j) {
            const char * vr = sh.rows + j * FLAT_ROW_PITCH + col * ES;
            if constexpr (F16) {
                const half2 hv = *reinterpret_cast<const half2 *>(vr);
                v[j] = f32x2{(float)hv[0], (float)hv[1]};
            } else {
                v[j] = *reinterpret_cast<const f32x2 *>(vr);
            }
        }
        f32x4 pv[FLAT_KEYS / 4];
#pragma unroll
        for (int j4 = 0; j4 < FLAT_KEYS / 4; ++j4) pv[j4] = *reinterpret_cast<const f32x4 *>(&sh.s[4 * j4]);
        float oa = 0.0f, ob = 0.0f;                   // two chains per column
#pragma unroll
        for (int j = 0; j < FLAT_KEYS; j += 2) {
            const float p0 = pv[j / 4][j & 3], p1 = pv[j / 4][(j & 3) + 1];
            o0 = fmaf(p0, v[j][0], o0);
            o1 = fmaf(p0, v[j][1], o1);
            oa = fmaf(p1, v[j + 1][0], oa);
            ob = fmaf(p1, v[j + 1][1], ob);
        }
        o0 += oa;
        o1 += ob;
    }
    // ---- the record: (m in natural-log units or -inf, l, o unnormalised) ----
    // Written and read back with agent-scope relaxed atomic accesses (global_store / global_load
    // ... sc1: device-coherent, past the XCDs' own L2s, which are not coherent with each other),
    // and no fence: an agent-scope release or acquire fence writes back or invalidates this XCD's
    // whole L2, and 256 workgroups doing that serialised to ~0.13 us each (34 us for a 256-key
    // window).  Ordering instead: each wave waits for its record stores to be acknowledged
    // (s_waitcnt vmcnt(0)) before the barrier after which thread 0 takes the ticket, so every
    // record of a head is at the coherence point before its last ticket is taken; the last
    // workgroup issues its record loads only after its ticket has returned.
    uint64_t * rec = reinterpret_cast<uint64_t *>(a.rec + ((size_t)h * a.n_split + sp) * (size_t)(dv + 4));
    if (tid == 0) {
        const float m = sh.ml[0];
        const f32x2 ml = {(m == -INFINITY) ? -INFINITY : m * LN2, sh.ml[1]};
        __hip_atomic_store(rec, __builtin_bit_cast(uint64_t, ml), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (col < dv)
        __hip_atomic_store(rec + 2 + tid, __builtin_bit_cast(uint64_t, f32x2{o0, o1}), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.ticket + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.last = prev == (unsigned)(a.n_split - 1);
    }
    __syncthreads();
    if (!sh.last) return;
    // ---- the last workgroup of head h: merge its records (log-sum-exp) into dst ----
    const uint64_t * hrec = reinterpret_cast<const uint64_t *>(a.rec + (size_t)h * a.n_split * (size_t)(dv + 4));
    const size_t rstride = (size_t)(dv + 4) / 2;       // 8-byte words per record
    float ms[FLAT_MAX_SPLITS], ls[FLAT_MAX_SPLITS];
    f32x2 ov[FLAT_MAX_SPLITS];
    float M = -INFINITY;
#pragma unroll
    for (int s2 = 0; s2 < FLAT_MAX_SPLITS; ++s2) {       // every load issued before the first use
        ms[s2] = -INFINITY;
        ls[s2] = 0.0f;
        ov[s2] = f32x2{0.0f, 0.0f};
        if (s2 < a.n_split) {
            const f32x2 ml = __builtin_bit_cast(f32x2, __hip_atomic_load(hrec + s2 * rstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            ms[s2] = ml[0];
            ls[s2] = ml[1];
            if (col < dv)
                ov[s2] = __builtin_bit_cast(f32x2, __hip_atomic_load(hrec + s2 * rstride + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
    }
#pragma unroll
    for (int s2 = 0; s2 < FLAT_MAX_SPLITS; ++s2) M = fmaxf(M, ms[s2]);
    float L = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < FLAT_MAX_SPLITS; ++s2) {
        const float f = (ms[s2] == -INFINITY) ? 0.0f : expf(ms[s2] - M);
        L = fmaf(f, ls[s2], L);
        r0 = fmaf(f, ov[s2][0], r0);
        r1 = fmaf(f, ov[s2][1], r1);
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (col < dv) *reinterpret_cast<f32x2 *>(a.dst + (size_t)h * dv + col) = f32x2{r0 * inv, r1 * inv};
    if (tid == 0) __hip_atomic_store(a.ticket + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_kqkv_flat(int kc_is_f16, const FlatArgs & a, hipStream_t stream) {
    if (a.n_split < 1 || a.n_kv > a.n_split * FLAT_KEYS || a.dk > FLAT_DK_MAX || a.dv > 2 * FTHR || (a.dv & 1) ||
        a.dk % (kc_is_f16 ? 8 : 4) != 0 || a.dk * (kc_is_f16 ? 2 : 4) > FLAT_ROW_PITCH)
        return hipErrorInvalidValue;
    const dim3 grid(a.n_split, a.n_head);
    if (kc_is_f16)
        hipLaunchKernelGGL(kqkv_flat_kernel<true>, grid, dim3(FTHR), 0, stream, a);
    else
        hipLaunchKernelGGL(kqkv_flat_kernel<false>, grid, dim3(FTHR), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla

// mla_kernels.h -- host-visible launch interface of the gfx950 kernels (internal to the library;
// the public boundary is include/mla_m4.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

// Split-K partials of one (32-head group g, token t) form a record of n_split * part_block_bytes
// bytes at part + (g * nt + t) * n_split * part_block_bytes, records ordered [group][token]:
//   float2 ml[32][n_split]       (m, l) of head hh, split s at [hh][s]: one head's pairs are
//                                contiguous, so the merge reads them as a few whole lines
//   T      o[n_split][32][D_v]   split s's o / l
// with
//   m      a reference for the split's scores, natural-log units: the exact max (VALU kernel) or a
//          running reference at most 15 ln 2 below it (MFMA kernels); -inf if the split is empty.
//          The merge only uses m + ln l.
//   l      sum_j exp(s_j - m)
//   o / l  the split's normalised softmax output.  T is the cache's element type: f16 for an f16
//          cache (|o / l| <= max|V|, so it cannot overflow), f32 for f32.  A split with no live
//          key (m = -inf) may leave its block unwritten; the merge never reads it.
constexpr int PART_HEADS = 32;
__host__ __device__ constexpr size_t part_block_bytes(int dv, int o_bytes) {
    return 256 + (size_t)PART_HEADS * (size_t)o_bytes * (size_t)dv;
}
__host__ __device__ inline char * part_record(char * part, int g, int nt, int t, int n_split, int dv, int o_bytes) {
    return part + ((size_t)g * nt + t) * (size_t)n_split * part_block_bytes(dv, o_bytes);
}
__host__ __device__ inline const char * part_record(const char * part, int g, int nt, int t, int n_split, int dv, int o_bytes) {
    return part + ((size_t)g * nt + t) * (size_t)n_split * part_block_bytes(dv, o_bytes);
}
// byte offsets within a record: the (m, l) pair of (head hh, split s); split s's o block
__host__ __device__ constexpr size_t part_ml_off(int n_split, int hh, int s) { return ((size_t)hh * n_split + s) * 8; }
__host__ __device__ constexpr size_t part_o_off(int n_split, int s, int dv, int o_bytes) {
    return (size_t)n_split * 256 + (size_t)s * PART_HEADS * (size_t)dv * (size_t)o_bytes;
}

// Split-K decode / generic attention launch arguments (byte strides throughout).
struct DecodeArgs {
    const char * kc;        // cache base
    int64_t kc_nb1;         // cache row stride
    const float * q;        // Qcur
    int64_t q_nb1, q_nb2;   // head, token strides
    const float * mask;     // may be null
    int64_t mask_nb1;       // token stride
    float scale_log2;       // kq_scale * log2(e)
    int n_kv;
    int n_head;
    int nt;
    int n_split;
    int n_tiles;            // ceil(n_kv / 64)
    char * part;            // partial blocks (when dst == null)
    float * dst;            // final output (single-split launches), contiguous [D_v, nt, H]
};

hipError_t launch_kqkv_decode_f16(int dk, int dv, const DecodeArgs & a, hipStream_t stream);
// several query tokens (nt >= PREFILL_MIN_TOKENS, chunked prefill): 4 tokens per workgroup sharing
// each K / V tile; grid (n_split, ceil(H/32), ceil(nt/4)); same outputs and geometries as the
// decode kernel.  Fewer rows (batch-of-N decode, often over disjoint per-sequence regions) stay on
// the decode kernels, whose workgroups skip the rows a split holds no live key of.
constexpr int PREFILL_MIN_TOKENS = 16;
constexpr int PREFILL_TOKENS_PER_WG = 4;
hipError_t launch_kqkv_prefill_f16(int dk, int dv, const DecodeArgs & a, hipStream_t stream);
bool decode_f16_supported(int dk, int dv);
// An 8-bit cache (ggml block_q8_0 rows, contiguous): the decode kernel of kqkv_decode_q8.hip, grid
// (n_split, ceil(H/32), row groups) as the f16 decode kernel, the f16 path's partial records (f16 o)
// and direct output.
hipError_t launch_kqkv_decode_q8(int dk, int dv, const DecodeArgs & a, hipStream_t stream);
inline bool decode_q8_supported(int dk, int dv) { return (dk == 576 && dv == 512) || (dk == 320 && dv == 256); }
// The cache's values as f16 rows (f16(q d), the 8-bit kernel's own), dst [n_kv][dk] contiguous:
// the chunked-prefill path over an 8-bit cache runs the f16 prefill kernel on that copy.
hipError_t launch_q8_rows_to_f16(int dk, const char * src, int n_kv, void * dst, hipStream_t stream);

// Generic VALU path (f32 or f16 cache, any D_k <= 1024, D_v <= D_k): one workgroup per
// (split, head, token).  round16 applies the f16 rounding of q and P (F16 cache semantics).
// Its splits are balanced runs of GRAN_KEYS-key granules.
constexpr int GRAN_KEYS = 16;
hipError_t launch_kqkv_generic(int dk, int dv, int kc_is_f16, const DecodeArgs & a, hipStream_t stream);

// Short decode windows in one launch (kqkv_flat.hip): one workgroup per (split of <= FLAT_KEYS keys,
// head) of one token; each writes a record (m, l, unnormalised o: dv + 4 floats) to rec
// [head][split], and the last workgroup of each head (an agent-scope ticket per head, ticket[h],
// zero before the launch and left zero after it) merges the head's records into dst.
constexpr int FLAT_KEYS = 32;
constexpr int FLAT_DK_MAX = 576;
constexpr int FLAT_ROW_PITCH = FLAT_DK_MAX * 4 + 128;    // LDS row pitch: 128 mod 256, distinct banks
constexpr int FLAT_MAX_SPLITS = 16;                      // windows up to 512 keys
struct FlatArgs {
    const char * kc;        // cache base (f32 or f16 rows)
    int64_t kc_nb1;
    const float * q;        // token 0's q, head h at q + h * q_nb1 bytes
    int64_t q_nb1;
    const float * mask;     // token 0's mask row, or null
    float scale_log2;       // kq_scale * log2(e)
    int n_kv, n_head, n_split, dk, dv;
    float * rec;            // n_head * n_split * (dv + 4) floats
    unsigned * ticket;      // n_head counters
    float * dst;            // [H][dv]
};
hipError_t launch_kqkv_flat(int kc_is_f16, const FlatArgs & a, hipStream_t stream);

// Split-K merge: partial blocks [group][token][split] (o of o_bytes = 2 or 4) -> dst [dv, nt, H]
hipError_t launch_merge(const char * part, int dv, int o_bytes, int n_split, int nt, int n_head, float * dst,
                        hipStream_t stream);

// WKB: dst[t][h][c] = sum_d w[h][c][d] * q[t][h][d]
struct WkbArgs {
    const float * w;        // F32 W_kb, contiguous [d_n, D_v, H]
    const uint8_t * wq;     // or Q8_0 W_kb: rows of d_n / 32 blocks of 34 bytes
    const float * q;        // q_nope
    int64_t q_nb1, q_nb2;
    float * dst;
    int64_t d_nb1, d_nb2;
    int d_n, d_v, n_head, nt;
};
hipError_t launch_wkb_f32(const WkbArgs & a, hipStream_t stream);
hipError_t launch_wkb_q8(const WkbArgs & a, hipStream_t stream);     // d_n in {64, 128}

// PHASE 1 (wv_b): dst[(o, t, h)] = Q8_0 w[h][o] . Q8_1(x[(:, t, h)])
struct WvbArgs {
    const uint8_t * w;      // Q8_0 rows [H][d_out] of d_in / 32 blocks
    const float * x;        // element (i, t, h) at x + t x_nb1 + h x_nb2 (bytes) + 4 i
    int64_t x_nb1, x_nb2;
    float * dst;            // element (o, t, h) at dst + t d_nb1 + h d_nb2 + 4 o
    int64_t d_nb1, d_nb2;
    int d_in, d_out, n_head, nt;
};
hipError_t launch_wvb_q8(const WvbArgs & a, hipStream_t stream);     // d_in in {256, 512}

// PHASE 0 (KV-write): gemv of cur through Q8_0 wkv_a [n_embd -> d_lat + n_rope], RMS norm of the
// latent rows, YaRN rope of the last n_rope rows, dst = the row, cache row kidx[0] = f16(row).
struct KvWriteArgs {
    const float * cur;
    const uint8_t * w;      // Q8_0 rows [d_lat + n_rope] of n_embd / 32 blocks
    const float * nw;       // [d_lat]
    void * kcache;          // F16 rows of kc_nb1 bytes, or Q8_0 rows (kc_q8) of 34-byte blocks
    int64_t kc_nb1;
    int kc_q8;
    int64_t n_kv;
    const int64_t * kidx;
    const int32_t * pos;
    float * dst;            // [d_lat + n_rope]
    int n_embd, d_lat, n_rope;
    float eps, theta_scale, freq_scale, ext_factor, attn_factor, corr0, corr1;
};
hipError_t launch_kvwrite(const KvWriteArgs & a, hipStream_t stream);  // n_embd in {4096, 7168}

}  // namespace mla

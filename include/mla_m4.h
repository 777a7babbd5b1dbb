/*
 * mla_m4.h -- the C ABI of the MI355X (gfx950) MLA attention kernels behind aubier's three
 * custom ggml ops GGML_OP_M4_WKB, GGML_OP_M4_KQKV and GGML_OP_M4_PHASE.
 *
 * The ggml HIP backend's launchers (ggml_cuda_m4_wkb / ggml_cuda_m4_kqkv / ggml_cuda_m4_phase,
 * dispatched from ggml_cuda_compute_forward) fill the tensor views below from their ggml_tensor
 * arguments and call these entry points on ctx.stream().  Every entry point:
 *   - is a plain asynchronous launch on `stream` (a hipStream_t): no allocation, no stream or
 *     device synchronisation, no host read of device memory -- legal inside hipGraph capture;
 *   - validates the whole shape/type/stride contract on the host BEFORE launching and returns a
 *     negative MLA_M4_ERR_* code on a violation (the ggml glue turns that into GGML_ABORT, which
 *     keeps the reference's FATAL semantics);
 *   - reports a failed launch through hipGetLastError as MLA_M4_ERR_LAUNCH.
 * Thread-compatible: one stream per call; concurrent streams need separate workspaces.
 *
 * Axis order is ggml's (ne[0] fastest).  Geometry is taken from ne[]/nb[]: the kernels are
 * instantiated for the two MLA geometries in use -- (D_k, D_v, d_n) = (576, 512, 128) and
 * (320, 256, 64) -- and any head count.
 */
#ifndef MLA_M4_H
#define MLA_M4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types.  The values are ggml's enum ggml_type numbers, so the glue passes
 * tensor->type through unchanged. */
enum {
    MLA_M4_TYPE_F32  = 0,
    MLA_M4_TYPE_F16  = 1,
    MLA_M4_TYPE_Q8_0 = 8,
    MLA_M4_TYPE_I32  = 26,
    MLA_M4_TYPE_I64  = 27
};

/* Status codes. */
enum {
    MLA_M4_OK             =  0,
    MLA_M4_ERR_NULL       = -1,  /* a required pointer is NULL */
    MLA_M4_ERR_TYPE       = -2,  /* unsupported element type */
    MLA_M4_ERR_SHAPE      = -3,  /* ne[] violates the op contract */
    MLA_M4_ERR_STRIDE     = -4,  /* nb[] violates the op contract (alignment, overlap, permutation) */
    MLA_M4_ERR_WORKSPACE  = -5,  /* workspace missing or smaller than mla_m4_kqkv_workspace_bytes() */
    MLA_M4_ERR_ARG        = -6,  /* a scalar argument is out of range (split count, phase id, ...) */
    MLA_M4_ERR_LAUNCH     = -7,  /* the HIP launch failed (hipGetLastError) */
    MLA_M4_ERR_UNSUPPORTED = -8, /* a legal ggml shape these kernels do not implement */
    MLA_M4_ERR_SCRATCH    = -9   /* mla_m4_kqkv_noalloc: the partials exceed its static scratch, or
                                    the scratch address could not be resolved */
};

/* A device tensor view: the data/type/ne/nb fields of a ggml_tensor (ggml.h struct ggml_tensor). */
typedef struct mla_m4_tensor {
    void *  data;    /* device pointer */
    int32_t type;    /* MLA_M4_TYPE_* */
    int32_t pad_;
    int64_t ne[4];   /* elements per axis, fastest first */
    size_t  nb[4];   /* byte strides per axis */
} mla_m4_tensor;

/* GGML_OP_M4_PHASE selectors (op_params[0]).  0 and 1 keep the reference's meaning
 * (patches/ggml-m4/m4-phase.cuh:3-14): KV-write and wv_b; 2 is the split-K merge. */
enum {
    MLA_M4_PHASE_KVWRITE = 0,
    MLA_M4_PHASE_WVB     = 1,
    MLA_M4_PHASE_MERGE   = 2
};

/* Split-K partials.  One record per (32-head group g, token t), records ordered [g][t], of
 * n_split * W words (W = MLA_M4_PART_FLOATS(D_v) for an F16 cache, MLA_M4_PART_FLOATS_F32(D_v)
 * for an F32 cache):
 *   float2 ml[32][n_split]      (m, l) of head h, split s at [h][s]:
 *                               m  a reference for the split's scaled, masked scores (natural-log
 *                                  units, at most 15 ln 2 below their max; -INFINITY for a split
 *                                  with no live key) -- the merge only uses m + ln l
 *                               l  sum over the split's keys of exp(score - m)
 *   T      o[n_split][32][D_v]  o / l: the split's normalised softmax output; T = f16 for an
 *                               F16 cache, f32 for an F32 cache.  A split with no live key
 *                               (m = -INFINITY) may leave its block unwritten: the merge never
 *                               reads it
 * As a tensor: F32 ne [W, n_split, nt, ceil(H / 32)], contiguous (its size; the words of a
 * record are laid out as above). */
#define MLA_M4_PART_HEADS 32
#define MLA_M4_PART_FLOATS(dv) (64 + 16 * (dv))
#define MLA_M4_PART_FLOATS_F32(dv) (64 + 32 * (dv))

/* Largest split count mla_m4_kqkv_partial accepts. */
#define MLA_M4_MAX_SPLITS 1024

const char * mla_m4_version(void);
const char * mla_m4_status_str(int status);

/* -------------------------------------------------------------------------------------------
 * GGML_OP_M4_WKB -- the MLA absorption of the query's nope half into the latent space.
 * Replaces ggml_cuda_m4_wkb (patches/ggml-m4/m4-wkb.cu:71-86); builder contract ggml_m4_wkb
 * (vendor/llama.cpp/ggml/src/ggml.c:3405-3426), generalised from the fixed Q8_0 [64,256,32]:
 *   w      F32  ne [d_n, D_v, H]     contiguous (W_kb: W[h][c][d]), d_n in {64, 128}
 *          or Q8_0 ne [d_n, D_v, H]  rows of d_n / 32 blocks (nb[0] = 34), 4-byte aligned --
 *                                     the reference's own form
 *   q_nope F32  ne [d_n, H, nt]      nb[0] = 4, any 16-byte-aligned (4-byte for Q8_0) head/token
 *                                     strides (the engine's view of q with a (d_n + d_r)-float
 *                                     head stride)
 *   dst    F32  ne [D_v, H, nt]      nb[0] = 4, 16-byte-aligned strides (may be a view into Qcur)
 *   F32:  dst[t][h][c] = sum_d w[h][c][d] * q_nope[t][h][d]         (f32 throughout, as ggml-cpu)
 *   Q8_0: the reference kernel's numerics (m4-wkb.cu:21-53): per 32-block b the activation is
 *         quantised to int8 with q = roundf(x / d), d = amax / 127 stored as f16 (d16), and
 *         dst = sum_b fma(wd_b * d16_b, (float) sum_k qw * qx, .) over the blocks in order.
 * ------------------------------------------------------------------------------------------- */
int mla_m4_wkb(const mla_m4_tensor * w, const mla_m4_tensor * q_nope,
               const mla_m4_tensor * dst, void * stream);

/* -------------------------------------------------------------------------------------------
 * GGML_OP_M4_KQKV -- fused Q.K^T over the latent+rope KV cache, masked softmax, then .V.
 * Replaces ggml_cuda_m4_kqkv (patches/ggml-m4/m4-kqkv.cu:340-378); builder contract
 * ggml_m4_kqkv (ggml.c:3429-3460), generalised:
 *   kcache F16|F32 ne [D_k, n_kv]    nb[0] = elsize, row stride nb[1] a multiple of 16 bytes;
 *                                     K = all D_k columns, V = columns [0, D_v) of the same row
 *          or Q8_0 ne [D_k, n_kv]    an 8-bit cache (no counterpart in the reference, whose KQKV
 *                                     asserts F16): ggml block_q8_0 rows (per 32 values an f16
 *                                     scale d and 32 int8 q, value q d), contiguous (nb[1] =
 *                                     D_k / 32 * 34), at (D_k, D_v) = (576, 512) or (320, 256);
 *                                     computed as the F16 cache f16(q d) (the f32 product rounded
 *                                     once), with the F16 path's numerics and f16 partials
 *   q      F32     ne [D_k, H, nt]   nb[0] = 4 (Qcur: absorbed nope part, then the rope part)
 *   mask   F32     ne [n_kv, >= nt]  nb[0] = 4 (0 / -INFINITY per key and token), or data NULL
 *   dst    F32     ne [D_v, nt, H]   contiguous
 *   kq_scale = op_params[0]
 *   dst[h][t][:] = softmax_j(kq_scale * q[t][h].K[j] + mask[t][j]) . V[j][:]
 * An F16 cache runs on MFMA with q rounded to f16 where the unfused ggml-cpu graph rounds it (its
 * mul_mat converts src1 to F16 for an F16 src0) and P rounded to f16 UNNORMALISED (exp2 of the
 * score minus a running reference max, at most 2^15) -- ggml-cpu rounds the normalised P instead,
 * which is subnormal in f16 at long context, so results differ from the oracle by more than one
 * rounding there (and are closer to exact arithmetic); an F32 cache runs in f32.
 * One token over a short window (an F32 cache of at most 512 keys, an F16 cache of at most 256,
 * D_k <= 576) runs in one launch: splits of at most 32 keys, one workgroup per (split, head), and
 * the last workgroup of each head (a ticket counter per head) merges the head's splits into dst.
 * Its tickets live in a static device array with one slot per (device, stream) -- 32 such pairs
 * per process; a stream beyond them takes the split-K path.  Otherwise up to 15 tokens (nt) run
 * the decode kernels, split-K (partial + merge, two launches); from 16 tokens the prefill kernel
 * (4 tokens per workgroup sharing each K/V tile).
 * `workspace` (device memory, >= mla_m4_kqkv_workspace_bytes()) holds the split-K partials (or the
 * one-launch kernel's per-split records: (m, l, o) in D_v + 4 floats per head and split), and,
 * for 16 or more tokens over a Q8_0 cache, first the cache's f16 values (n_kv x D_k x 2 bytes,
 * rounded up to 256), which the f16 prefill kernel then reads (a third launch before it).
 * ------------------------------------------------------------------------------------------- */
int mla_m4_kqkv(const mla_m4_tensor * kcache, const mla_m4_tensor * q,
                const mla_m4_tensor * mask, float kq_scale, const mla_m4_tensor * dst,
                void * workspace, size_t workspace_bytes, void * stream);

/* Workspace bytes mla_m4_kqkv needs for these shapes: the split-K partials, plus the f16 copy of a
 * Q8_0 cache for 16 or more tokens (0 when neither is used). */
size_t mla_m4_kqkv_workspace_bytes(const mla_m4_tensor * kcache, const mla_m4_tensor * q,
                                   const mla_m4_tensor * dst);

/* -------------------------------------------------------------------------------------------
 * mla_m4_kqkv without a workspace argument -- no counterpart in the reference's interface; for
 * callers that cannot allocate (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same operands, launches and results as mla_m4_kqkv (bit for bit); the
 * split-K partials live in a static device array of MLA_M4_NOALLOC_SCRATCH_BYTES (32 MiB) that
 * each GPU the library runs on holds until the process ends.  With an f16 cache a 32-head group
 * at 256 splits (>= 16K keys) needs 8.45 MB per token, so decode of up to 3 tokens at H <= 32
 * fits; the f32-cache kernel uses ~256 / (H nt) splits (0.53 MB at H = 32, one token).  The
 * workspace a shape needs (mla_m4_kqkv_workspace_bytes, including a Q8_0 cache's f16 copy for
 * prefill) must fit the array; larger shapes (long prefill, more heads) return MLA_M4_ERR_SCRATCH.
 * Allocates nothing and calls no allocating routine; the first call on each device resolves the
 * array's address (hipGetSymbolAddress), so make that first call outside graph capture.  Every
 * call on a GPU uses that GPU's one array: calls that overlap on one GPU (concurrent streams) race.
 * ------------------------------------------------------------------------------------------- */
#define MLA_M4_NOALLOC_SCRATCH_BYTES (32u << 20)
int mla_m4_kqkv_noalloc(const mla_m4_tensor * kcache, const mla_m4_tensor * q,
                        const mla_m4_tensor * mask, float kq_scale, const mla_m4_tensor * dst, void * stream);

/* Split count mla_m4_kqkv uses for a decode window of n_kv keys (a function of the window): about
 * one workgroup per CU, at most one split per 64-key tile (one token over an f16 cache: one tile per
 * split up to 256 tiles, then 256 splits -- also the fastest choice for the whole op, partial then
 * merge, measured over 2K-64K keys). */
int mla_m4_kqkv_default_splits(int64_t n_kv, int64_t n_head, int32_t kcache_type);

/* -------------------------------------------------------------------------------------------
 * Split-K pass 1 on its own: the partial kernel of patches/ggml-m4/m4-kqkv.cu:201-312 with an
 * explicit split count (1 .. MLA_M4_MAX_SPLITS).  Keys are partitioned into n_split contiguous
 * ranges of whole units, balanced (the first n_units % n_split ranges get one more unit): 64-key
 * tiles on the MFMA path (F16 cache, the two instantiated geometries; a Q8_0 cache), 16-key
 * granules on the VALU path (F32 cache, other geometries).  With a Q8_0 cache this entry point
 * always runs the 8-bit decode kernel, one pass over the window per token, also for 16 and more
 * tokens, where mla_m4_kqkv instead writes the cache's f16 values into its workspace and runs the
 * chunked-prefill kernel on them: the two agree within the f16-cache bar, not bit for bit.
 *   part F32 ne [MLA_M4_PART_FLOATS(D_v) (F16 cache) or MLA_M4_PART_FLOATS_F32(D_v) (F32 cache),
 *                n_split, nt, ceil(H / 32)] contiguous (layout above);
 *   D_v is the V width the partials are for (512 for the 576-wide cache, 256 for the 320-wide).
 * Followed by mla_m4_phase_merge this is mla_m4_kqkv's split-K path: bit for bit where mla_m4_kqkv
 * takes that path with the same split count (F16 and F32 caches below 16 tokens, except a short
 * window's one-launch kernel, which agrees within the cache type's bar).
 * ------------------------------------------------------------------------------------------- */
int mla_m4_kqkv_partial(const mla_m4_tensor * kcache, const mla_m4_tensor * q,
                        const mla_m4_tensor * mask, float kq_scale, int n_split, int64_t d_v,
                        const mla_m4_tensor * part, void * stream);

/* -------------------------------------------------------------------------------------------
 * GGML_OP_M4_PHASE, phase MLA_M4_PHASE_MERGE -- the split-K merge (the combine kernel of
 * patches/ggml-m4/m4-kqkv.cu:314-338): m* = max m_s; l* = sum l_s e^(m_s - m*);
 * o* = sum o_s e^(m_s - m*) over splits with m_s > -inf; dst = o* / l*, or 0 if every split is
 * empty.
 *   part F32 ne [MLA_M4_PART_FLOATS(D_v) or MLA_M4_PART_FLOATS_F32(D_v), n_split, nt, ceil(H / 32)]
 *   dst  F32 ne [D_v, nt, H] contiguous (H and D_v are taken from dst; the o type from ne[0])
 * ------------------------------------------------------------------------------------------- */
int mla_m4_phase_merge(const mla_m4_tensor * part, const mla_m4_tensor * dst, void * stream);

/* -------------------------------------------------------------------------------------------
 * GGML_OP_M4_PHASE, phase MLA_M4_PHASE_WVB -- the MLA value absorption (kqv_mla): replaces the
 * phase-1 branch of ggml_cuda_m4_phase (patches/ggml-m4/m4-phase.cu:52-88, 209-224); builder
 * ggml_m4_phase_wvb (vendor/llama.cpp/ggml/src/ggml.c:3520-3539), generalised from [256,128,32]:
 *   w    Q8_0 ne [d_in, d_out, H]   rows of d_in / 32 blocks, d_in in {256, 512}
 *   x    F32  ne [d_in, nt, H]      nb[0] = 4 (the KQKV output), 4-byte-aligned strides
 *   dst  F32  ne [d_out, nt, H]     nb[0] = 4
 * Numerics of the reference kernel: x quantised per 32-block (id = 1 / d, q = roundf(x * id),
 * f16 scale); lane k of 32 accumulates fma(wd_b * xd_b, qw[b][k] * qx[b][k], .) over the blocks
 * in order, then the xor butterfly 16, 8, 4, 2, 1 of warp_reduce_sum.
 * ------------------------------------------------------------------------------------------- */
int mla_m4_phase_wvb(const mla_m4_tensor * w, const mla_m4_tensor * x, const mla_m4_tensor * dst,
                     void * stream);

/* The rope / norm scalars of phase 0, op_params[1..9] of ggml_m4_phase_kvwrite in order
 * (ggml.c:3462-3468: an int32 array, f32 values bit-cast). */
typedef struct mla_m4_rope_params {
    float   freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow;
    float   eps;
    int32_t n_dims, n_ctx_orig;
} mla_m4_rope_params;

/* -------------------------------------------------------------------------------------------
 * GGML_OP_M4_PHASE, phase MLA_M4_PHASE_KVWRITE -- the step that writes the row KQKV streams:
 * replaces the phase-0 branch of ggml_cuda_m4_phase (patches/ggml-m4/m4-phase.cu:95-200, 226-273);
 * builder ggml_m4_phase_kvwrite (ggml.c:3469-3517), generalised from 4096 -> 256 + 64:
 *   cur     F32  ne [n_embd, 1]               the attn_norm output, n_embd in {4096, 7168}
 *   wkv_a   Q8_0 ne [n_embd, d_lat + n_dims]  rows of n_embd / 32 blocks
 *   kv_norm F32  ne [d_lat]                   attn_kv_a_norm weight
 *   kcache  F16  ne [d_lat + n_dims, n_kv]    WRITTEN IN PLACE at row kidx[0] (as ggml_set_rows)
 *           or Q8_0 (an extension: the reference's cache is F16 only; rows of (d_lat + n_dims) / 32
 *           blocks, nb[0] = 34, nb[1] even) -- the row is quantised as ggml's f32 -> q8_0 copy
 *           does (quantize_row_q8_0_ref, ggml-quants.c:276-299: per 32 values d = amax / 127,
 *           q = roundf(x * (1 / d)), d stored as f16), the cache KQKV reads as an 8-bit cache
 *   kidx    I64  ne [1], pos I32 ne [1]       read on the device (no host read of device memory);
 *                                             a row outside [0, n_kv) is not written
 *   dst     F32  ne [d_lat + n_dims]          Kcur: the values the cache row received
 * Two launches: the gemv (the reference's Q8_1 numerics: per input block q = roundf(x * (1/d)),
 * (wd * d16) * sum, butterfly per 32 blocks, partials in order), then one workgroup that
 * RMS-norms rows [0, d_lat) (1 / sqrt(mean of squares + eps) * kv_norm), ropes rows
 * [d_lat, d_lat + n_dims) (NORMAL mode, YaRN: theta = pos * theta_scale^p with the ramp mix when
 * ext_factor != 0, cos / sin scaled by attn_factor (1 + 0.1 ln(1 / freq_scale))), and scatters.
 * n_dims even, d_lat a multiple of 32, d_lat + n_dims <= 1024.
 * ------------------------------------------------------------------------------------------- */
int mla_m4_phase_kvwrite(const mla_m4_tensor * cur, const mla_m4_tensor * wkv_a,
                         const mla_m4_tensor * kv_norm, const mla_m4_tensor * kcache,
                         const mla_m4_tensor * kidx, const mla_m4_tensor * pos,
                         const mla_m4_rope_params * rope, const mla_m4_tensor * dst, void * stream);

/* -------------------------------------------------------------------------------------------
 * supports_op mirrors (ggml-cuda.cu:5848-5885): 1 if the entry point above accepts these
 * tensors, 0 otherwise.  They run the same host-side contract checks as the launch, without
 * launching, so the backend's supports_op and the launcher cannot disagree.  Data pointers may
 * be null (supports_op runs during graph planning, before allocation): only type, ne, nb and
 * the alignment of pointers that are set are checked.  A mask descriptor with ne[0] > 0 counts
 * as present.
 * ------------------------------------------------------------------------------------------- */
int mla_m4_supports_wkb(const mla_m4_tensor * w, const mla_m4_tensor * q_nope,
                        const mla_m4_tensor * dst);
int mla_m4_supports_kqkv(const mla_m4_tensor * kcache, const mla_m4_tensor * q,
                         const mla_m4_tensor * mask, const mla_m4_tensor * dst);
int mla_m4_supports_phase(int32_t phase, const mla_m4_tensor * src0, const mla_m4_tensor * dst);
/* phases 0 and 1 take more sources than (src0, dst): their own mirrors (mla_m4_supports_phase
 * returns 0 for them) */
int mla_m4_supports_phase_wvb(const mla_m4_tensor * w, const mla_m4_tensor * x, const mla_m4_tensor * dst);
int mla_m4_supports_phase_kvwrite(const mla_m4_tensor * cur, const mla_m4_tensor * wkv_a,
                                  const mla_m4_tensor * kv_norm, const mla_m4_tensor * kcache,
                                  const mla_m4_tensor * kidx, const mla_m4_tensor * pos,
                                  const mla_m4_rope_params * rope, const mla_m4_tensor * dst);

/* -------------------------------------------------------------------------------------------
 * The tri-state enable flag of each op (engine/m1_session.h:152-166, resolved at
 * engine/m1_engine.cpp:2178-2197): flag -1 = AUTO (on iff the attention core runs on the GPU),
 * 0 = off (the reference op sequence), 1 = explicit on, which requires gpu_core.  Returns 1/0
 * for on/off, or MLA_M4_ERR_ARG for an explicit 1 without gpu_core or a flag outside {-1,0,1}
 * (the engine CHECK-fails on that).
 * ------------------------------------------------------------------------------------------- */
int mla_m4_resolve_flag(int flag, int gpu_core);

#ifdef __cplusplus
}
#endif

#endif /* MLA_M4_H */

// mla_m4_abi.cpp -- the C ABI of include/mla_m4.h: host-side contract checks, path selection and
// launches.  Nothing here allocates, synchronises or reads device memory, so every entry point is
// legal inside hipGraph capture (the reference's plain-launch contract,
// patches/ggml-m4/m4-kqkv.cuh:3-7).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

#include "../../include/mla_m4.h"
#include "mla_kernels.h"

namespace {

constexpr int TILE_KEYS = 64;        // the decode kernels' tile (whole tiles per split)
constexpr int DECODE_HEADS = 32;     // heads per MFMA decode workgroup
constexpr int TARGET_WG = 256;       // one wave of workgroups over the 256 CUs

bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

size_t elsize(int32_t type) {
    switch (type) {
        case MLA_M4_TYPE_F32: return 4;
        case MLA_M4_TYPE_F16: return 2;
        default: return 0;
    }
}

bool is_contiguous(const mla_m4_tensor * t) {
    const size_t es = elsize(t->type);
    if (es == 0) return false;
    size_t expect = es;
    for (int i = 0; i < 4; ++i) {
        if (t->ne[i] != 1 && t->nb[i] != expect) return false;
        expect *= (size_t)t->ne[i];
    }
    return true;
}

// Q8_0 (ggml block_q8_0: f16 scale + 32 int8, 34 bytes): ne[0] a multiple of 32, nb[0] = the block
// size, rows of ne[0] / 32 blocks packed, higher axes packed.
constexpr size_t Q8_BLOCK = 34;
bool is_q8_rows(const mla_m4_tensor * t) {
    if (t->type != MLA_M4_TYPE_Q8_0 || t->ne[0] % 32 != 0 || t->nb[0] != Q8_BLOCK) return false;
    size_t expect = Q8_BLOCK * (size_t)(t->ne[0] / 32);
    for (int i = 1; i < 4; ++i) {
        if (t->ne[i] != 1 && t->nb[i] != expect) return false;
        expect *= (size_t)t->ne[i];
    }
    return true;
}

// ---------------------------------------------------------------- KQKV contract
struct KqkvShape {
    int64_t dk, dv, n_kv, n_head, nt;
    int64_t kc_nb1;
    int32_t kc_type;
    bool has_mask;
};

// plan = true: the supports_op mirrors, called on descriptors whose data may not be allocated yet
// (graph planning); only type/ne/nb are checked, and a data pointer only when it is set.
bool has_data(const mla_m4_tensor * t, bool plan) { return t && (plan || t->data); }
bool al16(const void * p, bool plan) { return (plan && !p) || aligned16(p); }
bool al4(const void * p, bool plan) { return (plan && !p) || (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

int check_kqkv(const mla_m4_tensor * kc, const mla_m4_tensor * q, const mla_m4_tensor * mask,
               const mla_m4_tensor * dst, KqkvShape * s, bool plan = false) {
    if (!has_data(kc, plan) || !has_data(q, plan) || !has_data(dst, plan)) return MLA_M4_ERR_NULL;
    const bool q8 = kc->type == MLA_M4_TYPE_Q8_0;
    if (kc->type != MLA_M4_TYPE_F16 && kc->type != MLA_M4_TYPE_F32 && !q8) return MLA_M4_ERR_TYPE;
    if (q->type != MLA_M4_TYPE_F32 || dst->type != MLA_M4_TYPE_F32) return MLA_M4_ERR_TYPE;
    // kcache ne [D_k, n_kv, 1, 1]
    if (kc->ne[0] < 1 || kc->ne[1] < 1 || kc->ne[2] != 1 || kc->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (q8) {
        // ggml block_q8_0 rows (34-byte blocks of 32 values), contiguous
        if (kc->ne[0] % 32) return MLA_M4_ERR_SHAPE;
        if (kc->nb[0] != 34 || kc->nb[1] != (size_t)(kc->ne[0] / 32 * 34) || !al16(kc->data, plan)) return MLA_M4_ERR_STRIDE;
    } else {
        const size_t es = elsize(kc->type);
        if (kc->nb[0] != es || kc->nb[1] < (size_t)kc->ne[0] * es || (kc->nb[1] & 15u) || !al16(kc->data, plan))
            return MLA_M4_ERR_STRIDE;
    }
    // q ne [D_k, H, nt, 1]
    if (q->ne[0] != kc->ne[0] || q->ne[1] < 1 || q->ne[2] < 1 || q->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (q->nb[0] != 4 || (q->nb[1] & 15u) || (q->nb[2] & 15u) || !al16(q->data, plan)) return MLA_M4_ERR_STRIDE;
    if (q->nb[1] < (size_t)q->ne[0] * 4) return MLA_M4_ERR_STRIDE;
    // dst ne [D_v, nt, H, 1] contiguous
    const int64_t dv = dst->ne[0];
    if (dv < 4 || (dv & 3) || dv > kc->ne[0]) return MLA_M4_ERR_SHAPE;
    if (dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (!is_contiguous(dst) || !al16(dst->data, plan)) return MLA_M4_ERR_STRIDE;
    // mask ne [n_kv, >= nt, 1, 1] (optional: a null descriptor, or null data outside planning)
    const bool has_mask = mask && (mask->data || (plan && mask->ne[0] > 0));
    if (has_mask) {
        if (mask->type != MLA_M4_TYPE_F32) return MLA_M4_ERR_TYPE;
        if (mask->ne[0] != kc->ne[1] || mask->ne[1] < q->ne[2] || mask->ne[2] != 1 || mask->ne[3] != 1)
            return MLA_M4_ERR_SHAPE;
        if (mask->nb[0] != 4 || mask->nb[1] < (size_t)mask->ne[0] * 4) return MLA_M4_ERR_STRIDE;
    }
    if (kc->ne[1] > INT32_MAX || q->ne[1] > 65535 || q->ne[2] > 65535) return MLA_M4_ERR_UNSUPPORTED;
    if (kc->ne[0] > 1024 || dv > 1024) return MLA_M4_ERR_UNSUPPORTED;
    // the 8-bit cache runs on its MFMA kernel only: its two geometries, rows within 4 GiB
    if (q8 && !(mla::decode_q8_supported((int)kc->ne[0], (int)dv) &&
                (uint64_t)kc->ne[1] * (uint64_t)kc->nb[1] <= 0xFFFFFFFFull))
        return MLA_M4_ERR_UNSUPPORTED;
    s->dk = kc->ne[0];
    s->dv = dv;
    s->n_kv = kc->ne[1];
    s->n_head = q->ne[1];
    s->nt = q->ne[2];
    s->kc_nb1 = (int64_t)kc->nb[1];
    s->kc_type = kc->type;
    s->has_mask = has_mask;
    return MLA_M4_OK;
}

// The MFMA kernel addresses the cache through a buffer resource with 32-bit byte offsets, so the
// rows it reads must end within 4 GiB of the cache base (n_kv <= 3.7M keys of a 576-wide f16
// cache); larger caches take the generic kernel.
bool use_mfma(const KqkvShape & s) {
    const uint64_t span = (uint64_t)(s.n_kv - 1) * (uint64_t)s.kc_nb1 + (uint64_t)s.dk * 2u;
    return s.kc_type == MLA_M4_TYPE_F16 && mla::decode_f16_supported((int)s.dk, (int)s.dv) && span <= 0xFFFFFFFFull;
}

// several tokens on the MFMA path: the prefill kernel (4 tokens per workgroup share each tile)
bool use_prefill(const KqkvShape & s) { return use_mfma(s) && s.nt >= mla::PREFILL_MIN_TOKENS; }

// an 8-bit (Q8_0) cache: its own MFMA kernel, one workgroup per (split, head group), shared by the
// split's rows as in the f16 decode kernel
bool use_q8(const KqkvShape & s) { return s.kc_type == MLA_M4_TYPE_Q8_0; }

// Chunked prefill over an 8-bit cache: a pre-pass writes the cache's f16 values (f16(q d), the
// 8-bit kernel's own) into the workspace and the f16 prefill kernel runs on that copy, 4 tokens
// sharing every K / V tile, instead of one 8-bit decode pass over the whole window per token.
bool use_q8_prefill(const KqkvShape & s) {
    return use_q8(s) && s.nt >= mla::PREFILL_MIN_TOKENS && mla::decode_f16_supported((int)s.dk, (int)s.dv) &&
           (uint64_t)s.n_kv * (uint64_t)s.dk * 2u <= 0xFFFFFFFFull;
}
// bytes of that copy at the head of the workspace (the partials follow it)
size_t q8_copy_bytes(const KqkvShape & s) {
    return use_q8_prefill(s) ? (((size_t)s.n_kv * (size_t)s.dk * 2u + 255u) & ~(size_t)255u) : 0;
}

int64_t n_tiles_of(int64_t n_kv) { return (n_kv + TILE_KEYS - 1) / TILE_KEYS; }

int default_splits(const KqkvShape & s) {
    // the unit a split is made of: 64-key tiles (MFMA kernels), 16-key granules (VALU kernel)
    const int64_t tiles = (use_mfma(s) || use_q8(s)) ? n_tiles_of(s.n_kv) : (s.n_kv + mla::GRAN_KEYS - 1) / mla::GRAN_KEYS;
    int64_t groups;   // workgroups per split
    if (use_prefill(s) || use_q8_prefill(s))
        groups = ((s.n_head + DECODE_HEADS - 1) / DECODE_HEADS) *
                 ((s.nt + mla::PREFILL_TOKENS_PER_WG - 1) / mla::PREFILL_TOKENS_PER_WG);
    // decode kernels: the rows of a split share its workgroup (the launch adds row groups only
    // when there are few splits), so the split count is the single-row one
    else if (use_mfma(s) || use_q8(s)) groups = (s.n_head + DECODE_HEADS - 1) / DECODE_HEADS;
    else groups = s.n_head * s.nt;
    // About one workgroup per CU.  For the single-token decode over an f16 cache this is also the
    // best split count for the whole op (partial, then the merge reading the records back), measured
    // on the MI355X over 2,048-65,536 keys (WKB + partial + merge, COLD): e.g. 32,768 keys 18.90 us
    // at 256 splits against 19.32 at 192 and 20.50 at 128; one tile per split below 256 tiles.
    // (With the records' o read by default-policy loads, which left them in the merge's L2s, fewer
    // and longer splits had won: 192 at 32,768 keys.)
    int64_t sp = (TARGET_WG + groups - 1) / groups;
    if (sp > tiles) sp = tiles;
    if (sp > MLA_M4_MAX_SPLITS) sp = MLA_M4_MAX_SPLITS;
    if (sp < 1) sp = 1;
    return (int)sp;
}

int64_t n_groups_of(int64_t n_head) { return (n_head + MLA_M4_PART_HEADS - 1) / MLA_M4_PART_HEADS; }

int part_o_bytes(const KqkvShape & s) { return s.kc_type == MLA_M4_TYPE_F32 ? 4 : 2; }     // f16 o for F16 and Q8_0 caches

int64_t part_floats(const KqkvShape & s) { return (int64_t)(mla::part_block_bytes((int)s.dv, part_o_bytes(s)) / 4); }

size_t part_bytes(const KqkvShape & s, int n_split) {
    return (size_t)n_groups_of(s.n_head) * (size_t)s.nt * (size_t)n_split * mla::part_block_bytes((int)s.dv, part_o_bytes(s));
}

mla::DecodeArgs make_args(const mla_m4_tensor * kc, const mla_m4_tensor * q, const mla_m4_tensor * mask,
                          float kq_scale, const KqkvShape & s, int n_split) {
    mla::DecodeArgs a{};
    a.kc = static_cast<const char *>(kc->data);
    a.kc_nb1 = (int64_t)kc->nb[1];
    a.q = static_cast<const float *>(q->data);
    a.q_nb1 = (int64_t)q->nb[1];
    a.q_nb2 = (int64_t)q->nb[2];
    a.mask = s.has_mask ? static_cast<const float *>(mask->data) : nullptr;
    a.mask_nb1 = s.has_mask ? (int64_t)mask->nb[1] : 0;
    a.scale_log2 = kq_scale * 1.4426950408889634f;
    a.n_kv = (int)s.n_kv;
    a.n_head = (int)s.n_head;
    a.nt = (int)s.nt;
    a.n_split = n_split;
    a.n_tiles = (int)n_tiles_of(s.n_kv);
    a.part = nullptr;
    a.dst = nullptr;
    return a;
}

// f16_copy: a's cache is the f16 copy of an 8-bit cache (use_q8_prefill)
int launch_attn(const KqkvShape & s, const mla::DecodeArgs & a, hipStream_t stream, bool f16_copy = false) {
    hipError_t e;
    if (f16_copy || use_prefill(s)) e = mla::launch_kqkv_prefill_f16((int)s.dk, (int)s.dv, a, stream);
    else if (use_q8(s)) e = mla::launch_kqkv_decode_q8((int)s.dk, (int)s.dv, a, stream);
    else if (use_mfma(s)) e = mla::launch_kqkv_decode_f16((int)s.dk, (int)s.dv, a, stream);
    else e = mla::launch_kqkv_generic((int)s.dk, (int)s.dv, s.kc_type == MLA_M4_TYPE_F16, a, stream);
    return e == hipSuccess ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

// ---------------------------------------------------------------- merge contract
int check_merge(const mla_m4_tensor * part, const mla_m4_tensor * dst, bool plan = false) {
    if (!has_data(part, plan) || !has_data(dst, plan)) return MLA_M4_ERR_NULL;
    if (part->type != MLA_M4_TYPE_F32 || dst->type != MLA_M4_TYPE_F32) return MLA_M4_ERR_TYPE;
    const int64_t dv = dst->ne[0];
    if (dv < 8 || (dv & 7) || dst->ne[1] < 1 || dst->ne[2] < 1 || dst->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if ((part->ne[0] != MLA_M4_PART_FLOATS(dv) && part->ne[0] != MLA_M4_PART_FLOATS_F32(dv)) ||
        part->ne[1] < 1 || part->ne[1] > MLA_M4_MAX_SPLITS ||
        part->ne[2] != dst->ne[1] || part->ne[3] != n_groups_of(dst->ne[2]))
        return MLA_M4_ERR_SHAPE;
    if (dst->ne[1] > 65535 || dst->ne[2] > 65535) return MLA_M4_ERR_UNSUPPORTED;
    if (!is_contiguous(part) || !is_contiguous(dst) || !al16(part->data, plan) || !al16(dst->data, plan))
        return MLA_M4_ERR_STRIDE;
    return MLA_M4_OK;
}

// ---------------------------------------------------------------- WKB contract
int check_wkb(const mla_m4_tensor * w, const mla_m4_tensor * x, const mla_m4_tensor * dst, bool plan = false) {
    if (!has_data(w, plan) || !has_data(x, plan) || !has_data(dst, plan)) return MLA_M4_ERR_NULL;
    if ((w->type != MLA_M4_TYPE_F32 && w->type != MLA_M4_TYPE_Q8_0) || x->type != MLA_M4_TYPE_F32 ||
        dst->type != MLA_M4_TYPE_F32)
        return MLA_M4_ERR_TYPE;
    const int64_t dn = w->ne[0], dv = w->ne[1], nh = w->ne[2];
    if (dn < 1 || dv < 1 || nh < 1 || w->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (x->ne[0] != dn || x->ne[1] != nh || x->ne[2] < 1 || x->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (dst->ne[0] != dv || dst->ne[1] != nh || dst->ne[2] != x->ne[2] || dst->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (w->type == MLA_M4_TYPE_Q8_0) {       // the reference's own form: rows of d_n / 32 blocks
        if (!is_q8_rows(w) || !al4(w->data, plan)) return MLA_M4_ERR_STRIDE;
        if (x->nb[0] != 4 || (x->nb[1] & 3u) || (x->nb[2] & 3u) || !al4(x->data, plan)) return MLA_M4_ERR_STRIDE;
        if (dst->nb[0] != 4 || (dst->nb[1] & 3u) || (dst->nb[2] & 3u) || dst->nb[1] < (size_t)dv * 4)
            return MLA_M4_ERR_STRIDE;
        if (dn != 64 && dn != 128) return MLA_M4_ERR_UNSUPPORTED;
        if (nh > 65535 || x->ne[2] > 65535) return MLA_M4_ERR_UNSUPPORTED;
        return MLA_M4_OK;
    }
    if (!is_contiguous(w) || !al16(w->data, plan)) return MLA_M4_ERR_STRIDE;
    if (x->nb[0] != 4 || (x->nb[1] & 15u) || (x->nb[2] & 15u) || !al16(x->data, plan)) return MLA_M4_ERR_STRIDE;
    if (dst->nb[0] != 4 || (dst->nb[1] & 3u) || (dst->nb[2] & 3u)) return MLA_M4_ERR_STRIDE;
    if (dst->nb[1] < (size_t)dv * 4) return MLA_M4_ERR_STRIDE;
    if (dn != 64 && dn != 128) return MLA_M4_ERR_UNSUPPORTED;
    if (dv % 16 != 0 || nh * dv > INT32_MAX || x->ne[2] > INT32_MAX) return MLA_M4_ERR_UNSUPPORTED;
    // the GEMM path (16 tokens and more) addresses 8 token rows of q from one buffer base
    if (x->ne[2] >= 16 && x->nb[2] > UINT32_MAX / 8) return MLA_M4_ERR_UNSUPPORTED;
    return MLA_M4_OK;
}

// ---------------------------------------------------------------- PHASE 1 (wv_b) contract
// w Q8_0 ne [d_in, d_out, H]; x F32 ne [d_in, nt, H] (the KQKV dst layout); dst F32 ne [d_out, nt, H]
int check_wvb(const mla_m4_tensor * w, const mla_m4_tensor * x, const mla_m4_tensor * dst, bool plan = false) {
    if (!has_data(w, plan) || !has_data(x, plan) || !has_data(dst, plan)) return MLA_M4_ERR_NULL;
    if (w->type != MLA_M4_TYPE_Q8_0 || x->type != MLA_M4_TYPE_F32 || dst->type != MLA_M4_TYPE_F32) return MLA_M4_ERR_TYPE;
    const int64_t din = w->ne[0], dout = w->ne[1], nh = w->ne[2];
    if (din < 32 || dout < 1 || nh < 1 || w->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (x->ne[0] != din || x->ne[1] < 1 || x->ne[2] != nh || x->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (dst->ne[0] != dout || dst->ne[1] != x->ne[1] || dst->ne[2] != nh || dst->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (!is_q8_rows(w) || !al4(w->data, plan)) return MLA_M4_ERR_STRIDE;
    if (x->nb[0] != 4 || (x->nb[1] & 3u) || (x->nb[2] & 3u) || !al4(x->data, plan)) return MLA_M4_ERR_STRIDE;
    if (dst->nb[0] != 4 || (dst->nb[1] & 3u) || (dst->nb[2] & 3u) || !al4(dst->data, plan)) return MLA_M4_ERR_STRIDE;
    if (din != 256 && din != 512) return MLA_M4_ERR_UNSUPPORTED;
    if (x->ne[1] > 65535 || nh > 65535) return MLA_M4_ERR_UNSUPPORTED;
    return MLA_M4_OK;
}

// ---------------------------------------------------------------- PHASE 0 (KV-write) contract
// cur F32 ne [n_embd, 1]; wkv_a Q8_0 ne [n_embd, d_lat + n_dims]; kv_norm F32 ne [d_lat];
// kcache F16 ne [d_lat + n_dims, n_kv] (rows of nb[1] bytes); kidx I64 ne [1]; pos I32 ne [1];
// dst F32 ne [d_lat + n_dims]
int check_kvwrite(const mla_m4_tensor * cur, const mla_m4_tensor * w, const mla_m4_tensor * nw,
                  const mla_m4_tensor * kc, const mla_m4_tensor * kidx, const mla_m4_tensor * pos,
                  const mla_m4_rope_params * rp, const mla_m4_tensor * dst, bool plan = false) {
    if (!has_data(cur, plan) || !has_data(w, plan) || !has_data(nw, plan) || !has_data(kc, plan) ||
        !has_data(kidx, plan) || !has_data(pos, plan) || !has_data(dst, plan) || !rp)
        return MLA_M4_ERR_NULL;
    if (cur->type != MLA_M4_TYPE_F32 || w->type != MLA_M4_TYPE_Q8_0 || nw->type != MLA_M4_TYPE_F32 ||
        (kc->type != MLA_M4_TYPE_F16 && kc->type != MLA_M4_TYPE_Q8_0) || kidx->type != MLA_M4_TYPE_I64 ||
        pos->type != MLA_M4_TYPE_I32 ||
        dst->type != MLA_M4_TYPE_F32)
        return MLA_M4_ERR_TYPE;
    const int64_t n_embd = cur->ne[0], n_out = w->ne[1], n_dims = rp->n_dims, d_lat = n_out - n_dims;
    if (cur->ne[1] != 1 || cur->ne[2] != 1 || cur->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (w->ne[0] != n_embd || w->ne[2] != 1 || w->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (n_dims < 2 || n_dims % 2 || d_lat < 32 || d_lat % 32 || nw->ne[0] != d_lat || nw->ne[1] != 1)
        return MLA_M4_ERR_SHAPE;
    if (kc->ne[0] != n_out || kc->ne[1] < 1 || kc->ne[2] != 1 || kc->ne[3] != 1) return MLA_M4_ERR_SHAPE;
    if (kidx->ne[0] != 1 || pos->ne[0] != 1 || dst->ne[0] != n_out || dst->ne[1] != 1) return MLA_M4_ERR_SHAPE;
    if (!is_q8_rows(w) || !al4(w->data, plan)) return MLA_M4_ERR_STRIDE;
    if (!is_contiguous(cur) || !is_contiguous(nw) || !is_contiguous(dst) || !al4(cur->data, plan) ||
        !al4(nw->data, plan) || !al4(dst->data, plan))
        return MLA_M4_ERR_STRIDE;
    if (kc->type == MLA_M4_TYPE_F16) {
        if (kc->nb[0] != 2 || kc->nb[1] < (size_t)n_out * 2 || (kc->nb[1] & 1u)) return MLA_M4_ERR_STRIDE;
    } else {
        // Q8_0 rows: whole blocks (n_out is a multiple of 32, checked below), 2-byte aligned scales
        if (n_out % 32 || kc->nb[0] != 34 || kc->nb[1] < (size_t)(n_out / 32) * 34 || (kc->nb[1] & 1u) ||
            (reinterpret_cast<uintptr_t>(kc->data) & 1u))
            return MLA_M4_ERR_STRIDE;
    }
    if (!(rp->freq_base > 0.0f) || !(rp->freq_scale > 0.0f) || !(rp->eps >= 0.0f) || rp->n_ctx_orig < 1 ||
        !std::isfinite(rp->ext_factor) || !std::isfinite(rp->attn_factor) || !(rp->beta_fast > 0.0f) ||
        !(rp->beta_slow > 0.0f))
        return MLA_M4_ERR_ARG;
    if ((n_embd != 4096 && n_embd != 7168) || n_out % 32 || n_out > 1024) return MLA_M4_ERR_UNSUPPORTED;
    return MLA_M4_OK;
}

// YaRN correction dims (the host-side ggml_rope_yarn_corr_dims, vendor/llama.cpp/ggml/src/ggml.c:4632-4643)
void rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow, float dims[2]) {
    const float pi = 3.14159265358979323846f;
    auto corr_dim = [&](float n_rot) {
        return (float)n_dims * logf((float)n_ctx_orig / (n_rot * 2.0f * pi)) / (2.0f * logf(freq_base));
    };
    const float start = floorf(corr_dim(beta_fast));
    const float end = ceilf(corr_dim(beta_slow));
    dims[0] = start > 0.0f ? start : 0.0f;
    dims[1] = end < (float)(n_dims - 1) ? end : (float)(n_dims - 1);
}

// ---------------------------------------------------------------- static scratch (no-alloc entry)
// The split-K partials of mla_m4_kqkv_noalloc: a fixed device array that each GPU the library
// runs on holds until the process ends.  Host code uses only the address hipGetSymbolAddress
// returns for the current device (the array's name in host code is a host-side stand-in, not a
// device address), resolved once per device on that device's first call and kept.
static __device__ __align__(256) unsigned char scratch[MLA_M4_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void * g_scratch_ptr[MAX_DEVICES] = {};

void * scratch_ptr() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void * p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

// ---------------------------------------------------------------- one-launch short windows
// One decode token over a short window runs kqkv_flat.hip's kernel: splits of <= 32 keys, the merge
// by the last workgroup of each head, one launch.  Measured on the MI355X (WKB + KQKV, COLD, 32
// heads, D_k 576): F32 cache 64 / 256 / 512 keys 9.85 / 11.46 / 15.10 us against 14.11 / 14.40 /
// 15.50 us for split-K partial + merge; F16 cache 64 / 256 keys 10.37 / 11.51 us against
// 12.73 / 13.18 us, but 512 keys 14.78 against 13.46 (every head's workgroups re-read the split's
// rows, and the MFMA kernel reads them once), hence the F16 bound.
constexpr int FLAT_MAX_HEADS = 256;
constexpr int FLAT_F16_MAX_KEYS = 256;
bool flat_eligible(const KqkvShape & s) {
    if (s.nt != 1 || (s.kc_type != MLA_M4_TYPE_F32 && s.kc_type != MLA_M4_TYPE_F16)) return false;
    const bool f16 = s.kc_type == MLA_M4_TYPE_F16;
    const int64_t es = f16 ? 2 : 4;
    const int64_t max_keys = f16 ? FLAT_F16_MAX_KEYS : (int64_t)mla::FLAT_KEYS * mla::FLAT_MAX_SPLITS;
    return s.n_kv <= max_keys && s.dk <= mla::FLAT_DK_MAX && s.dk % (16 / es) == 0 && s.dv <= 512 && s.dv % 2 == 0 &&
           s.n_head <= FLAT_MAX_HEADS;
}
int flat_splits(const KqkvShape & s) { return (int)((s.n_kv + mla::FLAT_KEYS - 1) / mla::FLAT_KEYS); }
size_t flat_bytes(const KqkvShape & s) { return (size_t)s.n_head * (size_t)flat_splits(s) * (size_t)(s.dv + 4) * 4u; }

// The flat kernel's per-head tickets: a static device array, zero when the library loads; every
// launch leaves its tickets zero again.  Launches that overlap on one GPU must not share tickets,
// so each (device, stream) pair gets a slot of its own on its first call, kept for the process
// (FLAT_SLOTS pairs; past that, a new stream takes the split-K path).  As with the scratch array,
// host code uses only the address hipGetSymbolAddress returns for the current device.
constexpr int FLAT_SLOTS = 32;
static __device__ __align__(256) unsigned flat_tickets[FLAT_SLOTS * FLAT_MAX_HEADS];
struct FlatSlot {
    int dev;
    hipStream_t st;
};
std::mutex g_flat_mu;
FlatSlot g_flat_slot[FLAT_SLOTS];
int g_flat_n = 0;
unsigned * g_flat_base[MAX_DEVICES] = {};

unsigned * flat_ticket_slot(hipStream_t st) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_flat_mu);
    if (g_flat_base[dev] == nullptr) {
        void * p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(flat_tickets)) != hipSuccess || p == nullptr) return nullptr;
        g_flat_base[dev] = static_cast<unsigned *>(p);
    }
    for (int i = 0; i < g_flat_n; ++i)
        if (g_flat_slot[i].dev == dev && g_flat_slot[i].st == st) return g_flat_base[dev] + (size_t)i * FLAT_MAX_HEADS;
    if (g_flat_n == FLAT_SLOTS) return nullptr;
    g_flat_slot[g_flat_n] = FlatSlot{dev, st};
    return g_flat_base[dev] + (size_t)(g_flat_n++) * FLAT_MAX_HEADS;
}

int flat_launch(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * mask, float kq_scale,
                const mla_m4_tensor * dst, const KqkvShape & s, char * work, unsigned * tickets, hipStream_t st) {
    mla::FlatArgs a{};
    a.kc = static_cast<const char *>(kcache->data);
    a.kc_nb1 = (int64_t)kcache->nb[1];
    a.q = static_cast<const float *>(q->data);
    a.q_nb1 = (int64_t)q->nb[1];
    a.mask = s.has_mask ? static_cast<const float *>(mask->data) : nullptr;
    a.scale_log2 = kq_scale * 1.4426950408889634f;
    a.n_kv = (int)s.n_kv;
    a.n_head = (int)s.n_head;
    a.n_split = flat_splits(s);
    a.dk = (int)s.dk;
    a.dv = (int)s.dv;
    a.rec = reinterpret_cast<float *>(work);
    a.ticket = tickets;
    a.dst = static_cast<float *>(dst->data);
    return mla::launch_kqkv_flat(s.kc_type == MLA_M4_TYPE_F16, a, st) == hipSuccess ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

// Workspace bytes of mla_m4_kqkv at split count sp: the f16 copy of an 8-bit cache for chunked
// prefill, then the split-K partials; a short window needs room for the flat kernel's records too
// (or its split-K fallback).
size_t kqkv_work_bytes(const KqkvShape & s, int sp) {
    const size_t split_k = q8_copy_bytes(s) + (sp > 1 ? part_bytes(s, sp) : 0);
    if (!flat_eligible(s)) return split_k;
    const size_t flat = flat_bytes(s);
    return flat > split_k ? flat : split_k;
}

// The KQKV launch sequence shared by mla_m4_kqkv and mla_m4_kqkv_noalloc, over `work` (>=
// kqkv_work_bytes(s, sp)): for chunked prefill over an 8-bit cache, its f16 copy first; then with
// one split the attention kernel writes dst, otherwise partials and the merge.
int kqkv_launch(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * mask, float kq_scale,
                const mla_m4_tensor * dst, const KqkvShape & s, int sp, char * work, hipStream_t st) {
    if (flat_eligible(s)) {
        unsigned * tickets = flat_ticket_slot(st);
        if (tickets != nullptr) return flat_launch(kcache, q, mask, kq_scale, dst, s, work, tickets, st);
    }
    mla::DecodeArgs a = make_args(kcache, q, mask, kq_scale, s, sp);
    const bool f16_copy = use_q8_prefill(s);
    if (f16_copy) {
        if (mla::launch_q8_rows_to_f16((int)s.dk, a.kc, (int)s.n_kv, work, st) != hipSuccess) return MLA_M4_ERR_LAUNCH;
        a.kc = work;
        a.kc_nb1 = s.dk * 2;
    }
    char * part = work + q8_copy_bytes(s);
    if (sp == 1) {
        a.dst = static_cast<float *>(dst->data);
        return launch_attn(s, a, st, f16_copy);
    }
    a.part = part;
    const int rc = launch_attn(s, a, st, f16_copy);
    if (rc != MLA_M4_OK) return rc;
    return mla::launch_merge(a.part, (int)s.dv, part_o_bytes(s), sp, (int)s.nt, (int)s.n_head, static_cast<float *>(dst->data), st) == hipSuccess
               ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

}  // namespace

extern "C" {

const char * mla_m4_version(void) { return "mla-m4-gfx950 0.1"; }

const char * mla_m4_status_str(int status) {
    switch (status) {
        case MLA_M4_OK: return "ok";
        case MLA_M4_ERR_NULL: return "null tensor or data pointer";
        case MLA_M4_ERR_TYPE: return "unsupported element type";
        case MLA_M4_ERR_SHAPE: return "shape violates the op contract";
        case MLA_M4_ERR_STRIDE: return "strides/alignment violate the op contract";
        case MLA_M4_ERR_WORKSPACE: return "workspace missing or too small";
        case MLA_M4_ERR_ARG: return "scalar argument out of range";
        case MLA_M4_ERR_LAUNCH: return "HIP launch failed";
        case MLA_M4_ERR_UNSUPPORTED: return "shape not implemented by these kernels";
        case MLA_M4_ERR_SCRATCH: return "needs more than the static scratch holds (or its address is unavailable)";
        default: return "unknown status";
    }
}

int mla_m4_wkb(const mla_m4_tensor * w, const mla_m4_tensor * q_nope, const mla_m4_tensor * dst, void * stream) {
    const int rc = check_wkb(w, q_nope, dst);
    if (rc != MLA_M4_OK) return rc;
    mla::WkbArgs a{};
    const bool q8 = w->type == MLA_M4_TYPE_Q8_0;
    a.w = q8 ? nullptr : static_cast<const float *>(w->data);
    a.wq = q8 ? static_cast<const uint8_t *>(w->data) : nullptr;
    a.q = static_cast<const float *>(q_nope->data);
    a.q_nb1 = (int64_t)q_nope->nb[1];
    a.q_nb2 = (int64_t)q_nope->nb[2];
    a.dst = static_cast<float *>(dst->data);
    a.d_nb1 = (int64_t)dst->nb[1];
    a.d_nb2 = (int64_t)dst->nb[2];
    a.d_n = (int)w->ne[0];
    a.d_v = (int)w->ne[1];
    a.n_head = (int)w->ne[2];
    a.nt = (int)q_nope->ne[2];
    const hipError_t e = q8 ? mla::launch_wkb_q8(a, static_cast<hipStream_t>(stream))
                            : mla::launch_wkb_f32(a, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

size_t mla_m4_kqkv_workspace_bytes(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * dst) {
    KqkvShape s{};
    if (check_kqkv(kcache, q, nullptr, dst, &s) != MLA_M4_OK) return 0;
    const int sp = (s.dv & 7) ? 1 : default_splits(s);
    return kqkv_work_bytes(s, sp);
}

int mla_m4_kqkv_default_splits(int64_t n_kv, int64_t n_head, int32_t kcache_type) {
    if (n_kv < 1 || n_head < 1) return MLA_M4_ERR_ARG;
    KqkvShape s{};
    s.dk = 576; s.dv = 512; s.n_kv = n_kv; s.n_head = n_head; s.nt = 1; s.kc_type = kcache_type;
    return default_splits(s);
}

int mla_m4_kqkv(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * mask, float kq_scale,
                const mla_m4_tensor * dst, void * workspace, size_t workspace_bytes, void * stream) {
    KqkvShape s{};
    const int rc = check_kqkv(kcache, q, mask, dst, &s);
    if (rc != MLA_M4_OK) return rc;
    if (!std::isfinite(kq_scale)) return MLA_M4_ERR_ARG;
    const int sp = (s.dv & 7) ? 1 : default_splits(s);     // the merge reads 8 columns at a time
    const size_t need = kqkv_work_bytes(s, sp);
    if (need > 0 && (!workspace || !aligned16(workspace) || workspace_bytes < need)) return MLA_M4_ERR_WORKSPACE;
    return kqkv_launch(kcache, q, mask, kq_scale, dst, s, sp, static_cast<char *>(workspace), static_cast<hipStream_t>(stream));
}

int mla_m4_kqkv_noalloc(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * mask, float kq_scale,
                        const mla_m4_tensor * dst, void * stream) {
    KqkvShape s{};
    const int rc = check_kqkv(kcache, q, mask, dst, &s);
    if (rc != MLA_M4_OK) return rc;
    if (!std::isfinite(kq_scale)) return MLA_M4_ERR_ARG;
    const int sp = (s.dv & 7) ? 1 : default_splits(s);
    const size_t need = kqkv_work_bytes(s, sp);
    char * work = nullptr;
    if (need > 0) {
        if (need > MLA_M4_NOALLOC_SCRATCH_BYTES) return MLA_M4_ERR_SCRATCH;
        work = static_cast<char *>(scratch_ptr());
        if (work == nullptr) return MLA_M4_ERR_SCRATCH;
    }
    return kqkv_launch(kcache, q, mask, kq_scale, dst, s, sp, work, static_cast<hipStream_t>(stream));
}

int mla_m4_kqkv_partial(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * mask,
                        float kq_scale, int n_split, int64_t d_v, const mla_m4_tensor * part, void * stream) {
    if (!part || !part->data) return MLA_M4_ERR_NULL;
    if (!q) return MLA_M4_ERR_NULL;
    // validate the attention operands against a dst view of the merged output
    mla_m4_tensor dview{};
    dview.data = part->data;
    dview.type = MLA_M4_TYPE_F32;
    dview.ne[0] = d_v;
    dview.ne[1] = q->ne[2];
    dview.ne[2] = q->ne[1];
    dview.ne[3] = 1;
    dview.nb[0] = 4;
    dview.nb[1] = 4 * (size_t)dview.ne[0];
    dview.nb[2] = dview.nb[1] * (size_t)dview.ne[1];
    dview.nb[3] = dview.nb[2] * (size_t)dview.ne[2];
    KqkvShape s{};
    int rc = check_kqkv(kcache, q, mask, &dview, &s);
    if (rc != MLA_M4_OK) return rc;
    if ((s.dv & 7) != 0) return MLA_M4_ERR_SHAPE;
    if (n_split < 1 || n_split > MLA_M4_MAX_SPLITS) return MLA_M4_ERR_ARG;
    if (!std::isfinite(kq_scale)) return MLA_M4_ERR_ARG;
    if (part->type != MLA_M4_TYPE_F32) return MLA_M4_ERR_TYPE;
    if (part->ne[0] != part_floats(s) || part->ne[1] != n_split || part->ne[2] != s.nt ||
        part->ne[3] != n_groups_of(s.n_head))
        return MLA_M4_ERR_SHAPE;
    if (!is_contiguous(part) || !aligned16(part->data)) return MLA_M4_ERR_STRIDE;
    mla::DecodeArgs a = make_args(kcache, q, mask, kq_scale, s, n_split);
    a.part = static_cast<char *>(part->data);
    return launch_attn(s, a, static_cast<hipStream_t>(stream));
}

int mla_m4_phase_merge(const mla_m4_tensor * part, const mla_m4_tensor * dst, void * stream) {
    const int rc = check_merge(part, dst);
    if (rc != MLA_M4_OK) return rc;
    const int o_bytes = part->ne[0] == MLA_M4_PART_FLOATS(dst->ne[0]) ? 2 : 4;
    return mla::launch_merge(static_cast<const char *>(part->data), (int)dst->ne[0], o_bytes, (int)part->ne[1],
                             (int)dst->ne[1], (int)dst->ne[2], static_cast<float *>(dst->data),
                             static_cast<hipStream_t>(stream)) == hipSuccess
               ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

int mla_m4_supports_wkb(const mla_m4_tensor * w, const mla_m4_tensor * q_nope, const mla_m4_tensor * dst) {
    return check_wkb(w, q_nope, dst, true) == MLA_M4_OK;
}

int mla_m4_supports_kqkv(const mla_m4_tensor * kcache, const mla_m4_tensor * q, const mla_m4_tensor * mask,
                         const mla_m4_tensor * dst) {
    KqkvShape s{};
    return check_kqkv(kcache, q, mask, dst, &s, true) == MLA_M4_OK;
}

int mla_m4_supports_phase(int32_t phase, const mla_m4_tensor * src0, const mla_m4_tensor * dst) {
    if (phase == MLA_M4_PHASE_MERGE) return check_merge(src0, dst, true) == MLA_M4_OK;
    return 0;   // phases 0 and 1 take more sources: mla_m4_supports_phase_kvwrite / _wvb
}

int mla_m4_phase_wvb(const mla_m4_tensor * w, const mla_m4_tensor * x, const mla_m4_tensor * dst, void * stream) {
    const int rc = check_wvb(w, x, dst);
    if (rc != MLA_M4_OK) return rc;
    mla::WvbArgs a{};
    a.w = static_cast<const uint8_t *>(w->data);
    a.x = static_cast<const float *>(x->data);
    a.x_nb1 = (int64_t)x->nb[1];
    a.x_nb2 = (int64_t)x->nb[2];
    a.dst = static_cast<float *>(dst->data);
    a.d_nb1 = (int64_t)dst->nb[1];
    a.d_nb2 = (int64_t)dst->nb[2];
    a.d_in = (int)w->ne[0];
    a.d_out = (int)w->ne[1];
    a.n_head = (int)w->ne[2];
    a.nt = (int)x->ne[1];
    return mla::launch_wvb_q8(a, static_cast<hipStream_t>(stream)) == hipSuccess ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

int mla_m4_supports_phase_wvb(const mla_m4_tensor * w, const mla_m4_tensor * x, const mla_m4_tensor * dst) {
    return check_wvb(w, x, dst, true) == MLA_M4_OK;
}

int mla_m4_phase_kvwrite(const mla_m4_tensor * cur, const mla_m4_tensor * wkv_a, const mla_m4_tensor * kv_norm,
                         const mla_m4_tensor * kcache, const mla_m4_tensor * kidx, const mla_m4_tensor * pos,
                         const mla_m4_rope_params * rope, const mla_m4_tensor * dst, void * stream) {
    const int rc = check_kvwrite(cur, wkv_a, kv_norm, kcache, kidx, pos, rope, dst);
    if (rc != MLA_M4_OK) return rc;
    mla::KvWriteArgs a{};
    a.cur = static_cast<const float *>(cur->data);
    a.w = static_cast<const uint8_t *>(wkv_a->data);
    a.nw = static_cast<const float *>(kv_norm->data);
    a.kcache = kcache->data;
    a.kc_nb1 = (int64_t)kcache->nb[1];
    a.kc_q8 = kcache->type == MLA_M4_TYPE_Q8_0;
    a.n_kv = kcache->ne[1];
    a.kidx = static_cast<const int64_t *>(kidx->data);
    a.pos = static_cast<const int32_t *>(pos->data);
    a.dst = static_cast<float *>(dst->data);
    a.n_embd = (int)cur->ne[0];
    a.n_rope = rope->n_dims;
    a.d_lat = (int)wkv_a->ne[1] - rope->n_dims;
    a.eps = rope->eps;
    a.theta_scale = powf(rope->freq_base, -2.0f / (float)rope->n_dims);
    a.freq_scale = rope->freq_scale;
    a.ext_factor = rope->ext_factor;
    a.attn_factor = rope->attn_factor;
    float corr[2];
    rope_yarn_corr_dims(rope->n_dims, rope->n_ctx_orig, rope->freq_base, rope->beta_fast, rope->beta_slow, corr);
    a.corr0 = corr[0];
    a.corr1 = corr[1];
    return mla::launch_kvwrite(a, static_cast<hipStream_t>(stream)) == hipSuccess ? MLA_M4_OK : MLA_M4_ERR_LAUNCH;
}

int mla_m4_supports_phase_kvwrite(const mla_m4_tensor * cur, const mla_m4_tensor * wkv_a, const mla_m4_tensor * kv_norm,
                                  const mla_m4_tensor * kcache, const mla_m4_tensor * kidx, const mla_m4_tensor * pos,
                                  const mla_m4_rope_params * rope, const mla_m4_tensor * dst) {
    return check_kvwrite(cur, wkv_a, kv_norm, kcache, kidx, pos, rope, dst, true) == MLA_M4_OK;
}

int mla_m4_resolve_flag(int flag, int gpu_core) {
    if (flag == -1) return gpu_core ? 1 : 0;
    if (flag == 0) return 0;
    if (flag == 1) return gpu_core ? 1 : MLA_M4_ERR_ARG;
    return MLA_M4_ERR_ARG;
}

}  // extern "C"

// m4-mla.cpp -- the ggml HIP backend's side of aubier's M4 ops: the three launchers and the
// supports_op hook, forwarding every GGML_OP_M4_* node to the gfx950 kernels of libmla_m4 through
// its C ABI (include/mla_m4.h).  Installed as ggml/src/ggml-cuda/m4-mla.cpp by ggml-glue/apply.sh;
// replaces the launchers of patches/ggml-m4/m4-wkb.cu:71-86, m4-kqkv.cu:340-378 and the phase
// dispatcher m4-phase.cu:205-277 (none of the reference's kernels stays in the build).
//
// This is the only translation unit that sees both ggml and mla_m4.h.  A ggml_tensor is handed over
// as its data/type/ne/nb fields; every check (type, shape, strides, alignment) is the library's,
// and the same checks answer supports_op, so planning and launching cannot disagree.  A launch
// that the library refuses aborts with its status, as the reference's GGML_ASSERTs do.
#include "m4-mla.cuh"

#include "mla_m4.h"

// the library's type codes are ggml_type's values
static_assert(MLA_M4_TYPE_F32 == GGML_TYPE_F32 && MLA_M4_TYPE_F16 == GGML_TYPE_F16 &&
              MLA_M4_TYPE_Q8_0 == GGML_TYPE_Q8_0 && MLA_M4_TYPE_I32 == GGML_TYPE_I32 &&
              MLA_M4_TYPE_I64 == GGML_TYPE_I64, "mla_m4 type codes must equal ggml_type");
static_assert(GGML_MAX_DIMS == 4, "mla_m4_tensor carries four axes");

static mla_m4_tensor m4_desc(const ggml_tensor * t) {
    mla_m4_tensor d{};
    if (t == nullptr) {
        return d;                         // absent source: null data, ne[0] = 0
    }
    d.data = t->data;
    d.type = (int32_t) t->type;
    for (int i = 0; i < GGML_MAX_DIMS; ++i) {
        d.ne[i] = t->ne[i];
        d.nb[i] = t->nb[i];
    }
    return d;
}

// op_params[1..9] of ggml_m4_phase_kvwrite (ggml.c:3462-3468 documents the int32-index layout)
static mla_m4_rope_params m4_rope(const ggml_tensor * op) {
    mla_m4_rope_params r{};
    r.freq_base   = ggml_get_op_params_f32(op, 1);
    r.freq_scale  = ggml_get_op_params_f32(op, 2);
    r.ext_factor  = ggml_get_op_params_f32(op, 3);
    r.attn_factor = ggml_get_op_params_f32(op, 4);
    r.beta_fast   = ggml_get_op_params_f32(op, 5);
    r.beta_slow   = ggml_get_op_params_f32(op, 6);
    r.eps         = ggml_get_op_params_f32(op, 7);
    r.n_dims      = ggml_get_op_params_i32(op, 8);
    r.n_ctx_orig  = ggml_get_op_params_i32(op, 9);
    return r;
}

static void m4_check(const char * op, const ggml_tensor * dst, int status) {
    if (status != MLA_M4_OK) {
        GGML_ABORT("%s (%s): %s (%d)", op, dst->name, mla_m4_status_str(status), status);
    }
}

void ggml_cuda_m4_wkb(ggml_backend_cuda_context & ctx, ggml_tensor * dst) {
    const mla_m4_tensor w = m4_desc(dst->src[0]);
    const mla_m4_tensor q = m4_desc(dst->src[1]);
    const mla_m4_tensor o = m4_desc(dst);
    m4_check("GGML_OP_M4_WKB", dst, mla_m4_wkb(&w, &q, &o, ctx.stream()));
}

void ggml_cuda_m4_kqkv(ggml_backend_cuda_context & ctx, ggml_tensor * dst) {
    const mla_m4_tensor k = m4_desc(dst->src[0]);
    const mla_m4_tensor q = m4_desc(dst->src[1]);
    const mla_m4_tensor m = m4_desc(dst->src[2]);
    const mla_m4_tensor o = m4_desc(dst);
    const float kq_scale = ggml_get_op_params_f32(dst, 0);

    // The split-K partials come from the context's pool, like every other temporary of this
    // backend: ggml captures its graphs in relaxed mode after uncaptured warm-up evaluations, and
    // the pool keeps (and re-hands) the memory a captured node was given.  Decode at 32 heads and
    // an F16 cache needs 8.45 MB per token (256 splits); one token of a short window (one launch)
    // needs D_v + 4 floats per head and 32-key split, 528 KB at 32 heads and 256 keys.
    const size_t need = mla_m4_kqkv_workspace_bytes(&k, &q, &o);
    ggml_cuda_pool_alloc<char> ws(ctx.pool());
    if (need > 0) {
        ws.alloc(need);
    }
    m4_check("GGML_OP_M4_KQKV", dst, mla_m4_kqkv(&k, &q, &m, kq_scale, &o, ws.ptr, need, ctx.stream()));
}

void ggml_cuda_m4_phase(ggml_backend_cuda_context & ctx, ggml_tensor * dst) {
    const int32_t phase = ggml_get_op_params_i32(dst, 0);
    const mla_m4_tensor o = m4_desc(dst);
    switch (phase) {
        case MLA_M4_PHASE_KVWRITE: {    // m4-phase.cu:226-273: cur, wkv_a, kv_norm, kcache, kidx, pos
            mla_m4_tensor s[6];
            for (int i = 0; i < 6; ++i) {
                s[i] = m4_desc(dst->src[i]);
            }
            const mla_m4_rope_params r = m4_rope(dst);
            m4_check("GGML_OP_M4_PHASE/kv-write", dst,
                     mla_m4_phase_kvwrite(&s[0], &s[1], &s[2], &s[3], &s[4], &s[5], &r, &o, ctx.stream()));
            break;
        }
        case MLA_M4_PHASE_WVB: {        // m4-phase.cu:209-224
            const mla_m4_tensor w = m4_desc(dst->src[0]);
            const mla_m4_tensor x = m4_desc(dst->src[1]);
            m4_check("GGML_OP_M4_PHASE/wv_b", dst, mla_m4_phase_wvb(&w, &x, &o, ctx.stream()));
            break;
        }
        case MLA_M4_PHASE_MERGE: {      // the split-K merge of ggml_m4_phase_merge
            const mla_m4_tensor p = m4_desc(dst->src[0]);
            m4_check("GGML_OP_M4_PHASE/merge", dst, mla_m4_phase_merge(&p, &o, ctx.stream()));
            break;
        }
        default:
            GGML_ABORT("GGML_OP_M4_PHASE (%s): unknown phase %d", dst->name, (int) phase);
    }
}

bool ggml_cuda_m4_supports_op(const ggml_tensor * op) {
    const mla_m4_tensor o = m4_desc(op);
    switch (op->op) {
        case GGML_OP_M4_WKB: {
            const mla_m4_tensor w = m4_desc(op->src[0]);
            const mla_m4_tensor q = m4_desc(op->src[1]);
            return mla_m4_supports_wkb(&w, &q, &o) == 1;
        }
        case GGML_OP_M4_KQKV: {
            const mla_m4_tensor k = m4_desc(op->src[0]);
            const mla_m4_tensor q = m4_desc(op->src[1]);
            const mla_m4_tensor m = m4_desc(op->src[2]);
            return mla_m4_supports_kqkv(&k, &q, &m, &o) == 1;
        }
        case GGML_OP_M4_PHASE: {
            const int32_t phase = ggml_get_op_params_i32(op, 0);
            if (phase == MLA_M4_PHASE_KVWRITE) {
                mla_m4_tensor s[6];
                for (int i = 0; i < 6; ++i) {
                    s[i] = m4_desc(op->src[i]);
                }
                const mla_m4_rope_params r = m4_rope(op);
                return mla_m4_supports_phase_kvwrite(&s[0], &s[1], &s[2], &s[3], &s[4], &s[5], &r, &o) == 1;
            }
            if (phase == MLA_M4_PHASE_WVB) {
                const mla_m4_tensor w = m4_desc(op->src[0]);
                const mla_m4_tensor x = m4_desc(op->src[1]);
                return mla_m4_supports_phase_wvb(&w, &x, &o) == 1;
            }
            const mla_m4_tensor p = m4_desc(op->src[0]);
            return mla_m4_supports_phase(phase, &p, &o) == 1;   // the merge; 0 for unknown selectors
        }
        default:
            return false;
    }
}

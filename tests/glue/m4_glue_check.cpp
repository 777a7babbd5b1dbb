// m4_glue_check.cpp -- host-only check of the ggml glue (ggml-glue/) against the patched ggml.
//
// The M4 builders of the patched ggml.c build nodes of the shapes aubier's engine uses (the
// reference geometry 4096 -> 256 + 64 with a Q8_0 W_kb, and the 576-wide one), and the glue's
// ggml_cuda_m4_supports_op -- libmla_m4's own contract checks -- must accept every one of them and
// reject tampered ones.  `abort:<case>` runs one builder call the patched asserts must refuse.
//
// Built by tests/test_ggml_glue.py from this file, ggml-glue/m4-mla.cpp and the builder functions
// cut out of the patched ggml.c (the whole of ggml.c needs the build-generated ggml-version.h), and
// linked against libmla_m4.so.  It launches nothing: the ggml functions outside the cut-out code
// are test doubles below, and the three the launchers would reach abort if called.
#include "common.cuh"
#include "m4-mla.cuh"
#include "mla_m4.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

// ------------------------------------------------------------------------ test doubles
static std::vector<ggml_tensor *> g_tensors;

static ggml_tensor * make(ggml_type type, int64_t n0, int64_t n1 = 1, int64_t n2 = 1, int64_t n3 = 1) {
    ggml_tensor * t = static_cast<ggml_tensor *>(calloc(1, sizeof(ggml_tensor)));
    t->type = type;
    const int64_t ne[4] = { n0, n1, n2, n3 };
    size_t esize = 4;
    int64_t blck = 1;
    switch (type) {
        case GGML_TYPE_F32: case GGML_TYPE_I32: esize = 4; break;
        case GGML_TYPE_F16: esize = 2; break;
        case GGML_TYPE_I64: esize = 8; break;
        case GGML_TYPE_Q8_0: esize = 34; blck = 32; break;     // f16 scale + 32 int8
        default: fprintf(stderr, "make: type %d\n", (int) type); exit(2);
    }
    for (int i = 0; i < 4; ++i) t->ne[i] = ne[i];
    t->nb[0] = esize;
    t->nb[1] = esize * (size_t) (n0 / blck);
    t->nb[2] = t->nb[1] * (size_t) n1;
    t->nb[3] = t->nb[2] * (size_t) n2;
    g_tensors.push_back(t);
    return t;                                    // data stays null, as during graph planning
}

extern "C" ggml_tensor * ggml_new_tensor(ggml_context *, ggml_type type, int n_dims, const int64_t * ne) {
    if (type != GGML_TYPE_F32 || n_dims != 4) {
        fprintf(stderr, "ggml_new_tensor double: type %d n_dims %d\n", (int) type, n_dims);
        exit(2);
    }
    return make(type, ne[0], ne[1], ne[2], ne[3]);
}

extern "C" void ggml_abort(const char * file, int line, const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "ggml_abort %s:%d: ", file, line);
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
    exit(86);                                    // the status an expected builder abort returns
}

void ggml_cuda_error(const char * stmt, const char *, const char *, int, const char *) {
    fprintf(stderr, "unexpected ggml_cuda_error(%s)\n", stmt);
    abort();
}
void ggml_cuda_set_device(int) {
    fprintf(stderr, "unexpected ggml_cuda_set_device\n");
    abort();
}
std::unique_ptr<ggml_cuda_pool> ggml_backend_cuda_context::new_pool_for_device(int, int) {
    fprintf(stderr, "unexpected new_pool_for_device\n");
    abort();
}

// ------------------------------------------------------------------------ checks
static int g_fail = 0;

static void expect(bool ok, const std::string & what) {
    printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) ++g_fail;
}

static bool ne_is(const ggml_tensor * t, int64_t a, int64_t b, int64_t c, int64_t d = 1) {
    return t->ne[0] == a && t->ne[1] == b && t->ne[2] == c && t->ne[3] == d;
}

// q_nope as the engine views it: [d_n, H, nt] inside q_b's [d_n + d_r, H, nt]
static ggml_tensor * q_nope_view(int64_t d_n, int64_t d_r, int64_t H, int64_t nt) {
    ggml_tensor * q = make(GGML_TYPE_F32, d_n, H, nt);
    q->nb[1] = sizeof(float) * (size_t) (d_n + d_r);
    q->nb[2] = q->nb[1] * (size_t) H;
    return q;
}

// a node whose answer must flip to false after `tamper`
static void rejects(ggml_tensor * node, const std::function<void(ggml_tensor *)> & tamper, const std::string & what) {
    const ggml_tensor saved = *node;
    ggml_tensor saved_src[GGML_MAX_SRC];
    for (int i = 0; i < GGML_MAX_SRC; ++i) {
        if (node->src[i]) saved_src[i] = *node->src[i];
    }
    tamper(node);
    expect(!ggml_cuda_m4_supports_op(node), "rejects " + what);
    *node = saved;
    for (int i = 0; i < GGML_MAX_SRC; ++i) {
        if (node->src[i]) *node->src[i] = saved_src[i];
    }
}

static void check_wkb(ggml_type wt, int64_t d_n, int64_t D_v, int64_t H, int64_t nt) {
    const std::string tag = std::string("wkb ") + (wt == GGML_TYPE_Q8_0 ? "q8_0" : "f32") + " d_n=" + std::to_string(d_n) +
                            " D_v=" + std::to_string(D_v) + " nt=" + std::to_string(nt);
    ggml_tensor * w = make(wt, d_n, D_v, H);
    ggml_tensor * q = q_nope_view(d_n, 64, H, nt);
    ggml_tensor * o = ggml_m4_wkb(nullptr, w, q);
    expect(o->op == GGML_OP_M4_WKB && o->src[0] == w && o->src[1] == q && ne_is(o, D_v, H, nt), tag + ": node [D_v, H, nt]");
    expect(ggml_cuda_m4_supports_op(o), tag + ": supported");
    rejects(o, [](ggml_tensor * t) { t->ne[0] += 1; }, tag + " with a wrong D_v");
}

static void check_kqkv(ggml_type kt, int64_t D_k, int64_t n_kv, int64_t H, int64_t nt) {
    const std::string tag = std::string("kqkv ") + (kt == GGML_TYPE_F16 ? "f16" : "f32") + " D_k=" + std::to_string(D_k) +
                            " n_kv=" + std::to_string(n_kv) + " nt=" + std::to_string(nt);
    ggml_tensor * k = make(kt, D_k, n_kv);
    ggml_tensor * q = make(GGML_TYPE_F32, D_k, H, nt);
    ggml_tensor * m = make(GGML_TYPE_F32, n_kv, nt);
    ggml_tensor * o = ggml_m4_kqkv(nullptr, k, q, m, 0.0625f);
    expect(o->op == GGML_OP_M4_KQKV && o->src[0] == k && o->src[1] == q && o->src[2] == m &&
           ne_is(o, D_k - 64, nt, H) && ggml_get_op_params_f32(o, 0) == 0.0625f, tag + ": node [D_v, nt, H], kq_scale");
    expect(ggml_cuda_m4_supports_op(o), tag + ": supported");
    rejects(o, [](ggml_tensor * t) { std::swap(t->ne[1], t->ne[2]); }, tag + " with dst [D_v, H, nt]");
    rejects(o, [](ggml_tensor * t) { t->src[0]->type = GGML_TYPE_Q8_0; }, tag + " with a Q8_0 cache");
}

static void check_kvwrite(int64_t n_embd, int64_t d_lat, int n_dims, int64_t n_kv) {
    const std::string tag = "kv-write n_embd=" + std::to_string(n_embd) + " d_lat=" + std::to_string(d_lat);
    ggml_tensor * cur = make(GGML_TYPE_F32, n_embd);
    ggml_tensor * wkv_a = make(GGML_TYPE_Q8_0, n_embd, d_lat + n_dims);
    ggml_tensor * kvn = make(GGML_TYPE_F32, d_lat);
    ggml_tensor * kc = make(GGML_TYPE_F16, d_lat + n_dims, n_kv);
    ggml_tensor * kidx = make(GGML_TYPE_I64, 1);
    ggml_tensor * pos = make(GGML_TYPE_I32, 1);
    ggml_tensor * o = ggml_m4_phase_kvwrite(nullptr, cur, wkv_a, kvn, kc, kidx, pos, 10000.0f, 0.025f, 1.0f, 1.0f,
                                            32.0f, 1.0f, 1e-6f, n_dims, 4096);
    expect(o->op == GGML_OP_M4_PHASE && ggml_get_op_params_i32(o, 0) == MLA_M4_PHASE_KVWRITE && o->src[3] == kc &&
           o->src[5] == pos && ne_is(o, d_lat + n_dims, 1, 1) && ggml_get_op_params_i32(o, 8) == n_dims &&
           ggml_get_op_params_f32(o, 2) == 0.025f, tag + ": node [d_lat + n_dims], op_params");
    expect(ggml_cuda_m4_supports_op(o), tag + ": supported");
    rejects(o, [](ggml_tensor * t) { t->src[3]->type = GGML_TYPE_F32; }, tag + " with an F32 cache");
    rejects(o, [](ggml_tensor * t) { ggml_set_op_params_i32(t, 0, 9); }, tag + " under an unknown phase selector");
}

static void check_wvb(int64_t d_in, int64_t d_out, int64_t H, int64_t nt) {
    const std::string tag = "wv_b d_in=" + std::to_string(d_in) + " nt=" + std::to_string(nt);
    ggml_tensor * w = make(GGML_TYPE_Q8_0, d_in, d_out, H);
    ggml_tensor * x = make(GGML_TYPE_F32, d_in, nt, H);
    ggml_tensor * o = ggml_m4_phase_wvb(nullptr, w, x);
    expect(o->op == GGML_OP_M4_PHASE && ggml_get_op_params_i32(o, 0) == MLA_M4_PHASE_WVB && ne_is(o, d_out, nt, H),
           tag + ": node [d_out, nt, H]");
    expect(ggml_cuda_m4_supports_op(o), tag + ": supported");
    rejects(o, [](ggml_tensor * t) { t->ne[2] -= 1; }, tag + " with a wrong head count");
}

static void check_merge(int64_t D_v, bool f32_cache, int64_t n_split, int64_t nt, int64_t H) {
    const std::string tag = "merge D_v=" + std::to_string(D_v) + (f32_cache ? " f32" : " f16") + " splits=" + std::to_string(n_split);
    const int64_t W = f32_cache ? MLA_M4_PART_FLOATS_F32(D_v) : MLA_M4_PART_FLOATS(D_v);
    ggml_tensor * part = make(GGML_TYPE_F32, W, n_split, nt, (H + 31) / 32);
    ggml_tensor * o = ggml_m4_phase_merge(nullptr, part, D_v, H);
    expect(o->op == GGML_OP_M4_PHASE && ggml_get_op_params_i32(o, 0) == MLA_M4_PHASE_MERGE && o->src[0] == part &&
           ne_is(o, D_v, nt, H), tag + ": node [D_v, nt, H], selector 2");
    expect(ggml_cuda_m4_supports_op(o), tag + ": supported");
    rejects(o, [](ggml_tensor * t) { t->src[0]->ne[0] += 16; }, tag + " with a wrong record width");
}

// builder calls the patched asserts must refuse (each exits 86 through ggml_abort)
static int run_abort_case(const std::string & name) {
    if (name == "kqkv-mask-rows") {             // mask rows < tokens
        ggml_m4_kqkv(nullptr, make(GGML_TYPE_F16, 576, 512), make(GGML_TYPE_F32, 576, 32, 4), make(GGML_TYPE_F32, 512, 2), 1.0f);
    } else if (name == "kqkv-q-width") {        // q width != cache width
        ggml_m4_kqkv(nullptr, make(GGML_TYPE_F16, 576, 512), make(GGML_TYPE_F32, 320, 32, 1), make(GGML_TYPE_F32, 512, 1), 1.0f);
    } else if (name == "wkb-d_n") {             // d_n outside {64, 128}
        ggml_m4_wkb(nullptr, make(GGML_TYPE_F32, 96, 512, 32), q_nope_view(96, 64, 32, 1));
    } else if (name == "wvb-d_in") {            // d_in outside {256, 512}
        ggml_m4_phase_wvb(nullptr, make(GGML_TYPE_Q8_0, 384, 128, 32), make(GGML_TYPE_F32, 384, 1, 32));
    } else if (name == "kvwrite-row") {         // cache row width != d_lat + n_dims
        ggml_m4_phase_kvwrite(nullptr, make(GGML_TYPE_F32, 4096), make(GGML_TYPE_Q8_0, 4096, 320), make(GGML_TYPE_F32, 256),
                              make(GGML_TYPE_F16, 576, 64), make(GGML_TYPE_I64, 1), make(GGML_TYPE_I32, 1),
                              10000.0f, 1.0f, 0.0f, 1.0f, 32.0f, 1.0f, 1e-6f, 64, 4096);
    } else if (name == "merge-width") {         // record width of neither cache type
        ggml_m4_phase_merge(nullptr, make(GGML_TYPE_F32, 1000, 4, 1, 1), 512, 32);
    } else {
        fprintf(stderr, "unknown abort case %s\n", name.c_str());
        return 2;
    }
    printf("builder accepted %s\n", name.c_str());
    return 0;                                    // not refused: the caller expects 86
}

int main(int argc, char ** argv) {
    if (argc == 2 && strncmp(argv[1], "abort:", 6) == 0) {
        return run_abort_case(argv[1] + 6);
    }
    // the reference geometry (Mistral Small 4: 4096 -> 256 + 64, Q8_0 W_kb [64, 256, 32])
    check_wkb(GGML_TYPE_Q8_0, 64, 256, 32, 1);
    check_kqkv(GGML_TYPE_F16, 320, 2501, 32, 1);
    check_kvwrite(4096, 256, 64, 2501);
    check_wvb(256, 128, 32, 1);
    check_merge(256, false, 28, 1, 32);
    // the 576-wide geometry (7168 -> 512 + 64), batches of tokens, an F32 cache
    check_wkb(GGML_TYPE_F32, 128, 512, 32, 1);
    check_wkb(GGML_TYPE_F32, 128, 512, 32, 4);
    check_kqkv(GGML_TYPE_F16, 576, 32768, 32, 1);
    check_kqkv(GGML_TYPE_F16, 576, 8192, 32, 4);
    check_kqkv(GGML_TYPE_F32, 576, 256, 32, 1);
    check_kvwrite(7168, 512, 64, 32768);
    check_wvb(512, 128, 32, 1);
    check_wvb(512, 128, 32, 3);
    check_merge(512, false, 256, 1, 32);
    check_merge(512, true, 8, 2, 32);
    for (ggml_tensor * t : g_tensors) free(t);
    printf("%s: %d failure(s)\n", g_fail ? "FAILED" : "ALL OK", g_fail);
    return g_fail ? 1 : 0;
}

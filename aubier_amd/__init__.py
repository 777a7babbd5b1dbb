"""aubier_amd -- MI355X (gfx950) native MLA attention for aubier's custom ggml ops.

The product is the C ABI of include/mla_m4.h in aubier_amd/libmla_m4.so (hand-written HIP
kernels for GGML_OP_M4_WKB, GGML_OP_M4_KQKV and GGML_OP_M4_PHASE).  This package adds the
Python mirror of the op interface (aubier_amd.ops) and the seeded synthetic inputs
(aubier_amd.inputs).  Build with ``python -m aubier_amd.build``.
"""
from .ops import (  # noqa: F401
    MlaM4Error,
    Q8_0,
    ggml_m4_phase_kvwrite,
    ggml_m4_phase_wvb,
    rope_params,
    supports_phase_kvwrite,
    supports_phase_wvb,
    default_splits,
    ggml_m4_kqkv,
    ggml_m4_kqkv_noalloc,
    ggml_m4_kqkv_partial,
    ggml_m4_phase_merge,
    ggml_m4_wkb,
    kqkv_workspace_bytes,
    load_library,
    resolve_flag,
    supports_kqkv,
    supports_phase,
    supports_wkb,
    view,
)

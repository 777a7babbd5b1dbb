// m4-mla.cuh -- the ggml HIP backend's entry points for aubier's three M4 ops, served by the
// gfx950 kernels of libmla_m4 (include/mla_m4.h).  Installed as ggml/src/ggml-cuda/m4-mla.cuh; it
// takes the place of the reference's m4-wkb.cuh, m4-kqkv.cuh and m4-phase.cuh (one launcher
// declaration each, patches/ggml-m4/m4-{wkb,kqkv,phase}.cuh) and adds the supports_op hook.
#pragma once

#include "common.cuh"

// dispatch targets of ggml_cuda_compute_forward (ggml-cuda.cu:2504-2512), same names and
// signatures as the reference's launchers
void ggml_cuda_m4_wkb(ggml_backend_cuda_context & ctx, ggml_tensor * dst);
void ggml_cuda_m4_kqkv(ggml_backend_cuda_context & ctx, ggml_tensor * dst);
void ggml_cuda_m4_phase(ggml_backend_cuda_context & ctx, ggml_tensor * dst);

// the GGML_OP_M4_* cases of ggml_backend_cuda_device_supports_op (ggml-cuda.cu:5848-5885): true
// iff the launcher accepts op's sources and shapes (the same host-side checks the launch runs)
bool ggml_cuda_m4_supports_op(const ggml_tensor * op);

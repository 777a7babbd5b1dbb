#!/bin/sh
# Install aubier's M4 glue into a llama.cpp checkout (the engine's vendor/llama.cpp):
#     ggml-glue/apply.sh <llama.cpp checkout>
# applies mla-m4-ggml.patch there and copies m4-mla.cpp / m4-mla.cuh into ggml/src/ggml-cuda/.
# Then build this checkout's library (python -m aubier_amd.build) and configure ggml with
#     -DGGML_HIP=ON -DGGML_HIP_MLA_M4_ROOT=<this checkout>
set -eu
here=$(CDPATH= cd -- "$(dirname -- "$0")" && pwd)
dst=${1:?usage: apply.sh <llama.cpp checkout>}
patch -p1 -N -d "$dst" -i "$here/mla-m4-ggml.patch"
cp "$here/m4-mla.cpp" "$here/m4-mla.cuh" "$dst/ggml/src/ggml-cuda/"
echo "installed; configure with -DGGML_HIP=ON -DGGML_HIP_MLA_M4_ROOT=$(dirname "$here")"

"""The ggml glue (ggml-glue/) against the reference's vendored ggml (vendor/llama.cpp, read only):

  * ggml-glue/mla-m4-ggml.patch applies to it without fuzz;
  * the patched builders (ggml.c), the patched ggml-cuda.cu and the glue m4-mla.cpp compile
    (syntax and types) against the patched headers;
  * tests/glue/m4_glue_check.cpp: the patched builders build the nodes of the engine's shapes and
    the glue's ggml_cuda_m4_supports_op (libmla_m4's own contract checks) accepts each of them and
    rejects tampered ones; builder calls outside the widened contracts abort.

The whole of the patched ggml.c cannot be compiled here: it includes ggml-version.h, which the
reference's CMake generates.  Its builder functions are compiled on their own instead.  Skipped
where the reference checkout (AUBIER_REFERENCE, default /root/reference) or hipcc is absent.
"""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path(os.environ.get("AUBIER_REFERENCE", "/root/reference")) / "vendor" / "llama.cpp"
GGML = REF / "ggml"
PATCH = ROOT / "ggml-glue" / "mla-m4-ggml.patch"
GLUE = [ROOT / "ggml-glue" / "m4-mla.cpp", ROOT / "ggml-glue" / "m4-mla.cuh"]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
LIB = ROOT / "aubier_amd" / "libmla_m4.so"

pytestmark = pytest.mark.skipif(not (GGML / "include" / "ggml.h").is_file() or not Path(HIPCC).exists()
                                or shutil.which("patch") is None,
                                reason="needs the reference's vendored ggml, hipcc and patch")


def run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    return r.returncode, r.stdout + r.stderr


def patched_files():
    return re.findall(r"^\+\+\+ b/(\S+)", PATCH.read_text(), flags=re.M)


@pytest.fixture(scope="module")
def tree(tmp_path_factory):
    """A scratch tree of ggml's public headers and the files the patch touches, with the glue
    installed by ggml-glue/apply.sh."""
    t = tmp_path_factory.mktemp("llama.cpp")
    shutil.copytree(GGML / "include", t / "ggml" / "include")
    for rel in patched_files():
        (t / rel).parent.mkdir(parents=True, exist_ok=True)
        if not (t / rel).exists():
            shutil.copy(REF / rel, t / rel)
    rc, out = run(["sh", str(ROOT / "ggml-glue" / "apply.sh"), str(t)])
    assert rc == 0, out
    for g in GLUE:
        assert (t / "ggml" / "src" / "ggml-cuda" / g.name).read_bytes() == g.read_bytes()
    return t


def hip_includes(t):
    # patched files first, then the reference's unpatched rest
    return ["-I", str(t / "ggml" / "include"), "-I", str(t / "ggml" / "src"), "-I", str(GGML / "src"),
            "-I", str(t / "ggml" / "src" / "ggml-cuda"), "-I", str(GGML / "src" / "ggml-cuda"),
            "-I", str(ROOT / "include")]


HIP_FLAGS = ["-x", "hip", "--offload-arch=gfx950", "-std=c++17", "-w", "-DGGML_USE_HIP"]


def test_patch_touches_the_expected_files():
    assert sorted(patched_files()) == sorted([
        "ggml/include/ggml-rpc.h", "ggml/include/ggml.h", "ggml/src/ggml-cuda/ggml-cuda.cu",
        "ggml/src/ggml-hip/CMakeLists.txt", "ggml/src/ggml.c"])


def test_patch_applies_to_reference_without_fuzz():
    rc, out = run(["patch", "--dry-run", "-p1", "-d", str(REF), "-i", str(PATCH)])
    assert rc == 0, out
    assert "FAILED" not in out and "fuzz" not in out, out


def test_patched_tree_content(tree):
    h = (tree / "ggml/include/ggml.h").read_text()
    assert "ggml_m4_phase_merge(" in h
    c = (tree / "ggml/src/ggml-cuda/ggml-cuda.cu").read_text()
    assert '#include "ggml-cuda/m4-mla.cuh"' in c and "m4-wkb.cuh" not in c
    assert "return ggml_cuda_m4_supports_op(op);" in c
    cm = (tree / "ggml/src/ggml-hip/CMakeLists.txt").read_text()
    assert "m4-mla.cpp" in cm and "GGML_HIP_MLA_M4_ROOT" in cm
    rpc = (tree / "ggml/include/ggml-rpc.h").read_text()
    assert re.search(r"RPC_PROTO_MINOR_VERSION\s+1\b", rpc)


def cut_builders(tree, dst):
    s = (tree / "ggml/src/ggml.c").read_text()
    i0 = s.index("// The MLA absorption gemv as one named op (see ggml.h).")
    i1 = s.index("// ggml_mul_mat_id", i0)
    body = s[i0:i1]
    for name in ("ggml_m4_wkb", "ggml_m4_kqkv", "ggml_m4_phase_kvwrite", "ggml_m4_phase_wvb", "ggml_m4_phase_merge"):
        assert f"struct ggml_tensor * {name}(" in body, name
    dst.write_text('#include "ggml.h"\n#include "ggml-impl.h"\n\n' + body)
    return dst


def test_patched_builders_compile(tree, tmp_path):
    src = cut_builders(tree, tmp_path / "m4_builders.c")
    rc, out = run(["gcc", "-std=gnu11", "-fsyntax-only", "-Wall", "-I", str(tree / "ggml/include"),
                   "-I", str(GGML / "src"), str(src)])
    assert rc == 0, out


def test_glue_compiles(tree):
    rc, out = run([HIPCC, "-fsyntax-only", *HIP_FLAGS, *hip_includes(tree),
                   str(tree / "ggml/src/ggml-cuda/m4-mla.cpp")])
    assert rc == 0, out


def test_patched_ggml_cuda_compiles(tree):
    rc, out = run([HIPCC, "-fsyntax-only", *HIP_FLAGS, *hip_includes(tree),
                   str(tree / "ggml/src/ggml-cuda/ggml-cuda.cu")], timeout=600)
    assert rc == 0, out


@pytest.fixture(scope="module")
def checker(tree, tmp_path_factory):
    if not LIB.exists():
        pytest.skip("libmla_m4.so not built (python -m aubier_amd.build)")
    d = tmp_path_factory.mktemp("glue_check")
    b = cut_builders(tree, d / "m4_builders.c")
    steps = [
        ["gcc", "-std=gnu11", "-O1", "-c", "-I", str(tree / "ggml/include"), "-I", str(GGML / "src"), str(b),
         "-o", str(d / "m4_builders.o")],
        [HIPCC, "-c", *HIP_FLAGS, "-O1", *hip_includes(tree), str(tree / "ggml/src/ggml-cuda/m4-mla.cpp"),
         "-o", str(d / "m4-mla.o")],
        [HIPCC, "-c", *HIP_FLAGS, "-O1", *hip_includes(tree), str(ROOT / "tests/glue/m4_glue_check.cpp"),
         "-o", str(d / "check.o")],
        [HIPCC, "--offload-arch=gfx950", str(d / "check.o"), str(d / "m4-mla.o"), str(d / "m4_builders.o"),
         str(LIB), f"-Wl,-rpath,{LIB.parent}", "-o", str(d / "m4_glue_check")],
    ]
    for cmd in steps:
        rc, out = run(cmd, timeout=600)
        assert rc == 0, (cmd, out)
    return d / "m4_glue_check"


def test_builders_and_supports_op_agree(checker):
    rc, out = run([str(checker)], timeout=120)
    print(out)
    assert rc == 0 and "ALL OK: 0 failure(s)" in out, out
    assert out.count("\nok  ") + out.startswith("ok  ") >= 40


@pytest.mark.parametrize("case", ["kqkv-mask-rows", "kqkv-q-width", "wkb-d_n", "wvb-d_in", "kvwrite-row", "merge-width"])
def test_builders_refuse_shapes_outside_the_contract(checker, case):
    rc, out = run([str(checker), f"abort:{case}"], timeout=60)
    assert rc == 86 and "GGML_ASSERT" in out, (rc, out)

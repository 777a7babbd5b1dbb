"""Register / scratch / LDS budgets of every kernel, from the compiler's own resource report
(`-Rpass-analysis=kernel-resource-usage`), the check the reference runs on each build
(patches/ggml-m4/m4-kqkv.cu:39-42; ggml-hip/CMakeLists.txt:116-118).  A spill in a streaming
loop costs more than the kernel's arithmetic, so the hot kernels are held at zero VGPR spills;
the prefill kernel's few spills sit in its epilogue (outside the tile loop) and are capped.
CPU-only: hipcc cross-compiles for gfx950 here."""
import concurrent.futures as cf
import re
import shutil
import subprocess

import pytest

from aubier_amd import build as B

HIPCC = B.HIPCC
pytestmark = pytest.mark.skipif(shutil.which(HIPCC) is None and not __import__("os").path.exists(HIPCC),
                                reason="hipcc not available")

LDS_MAX = 160 * 1024
# kernel name fragment -> (max VGPR spills, max scratch bytes per lane)
BUDGET = {
    "kqkv_decode_f16_kernel": (0, 0),
    "kqkv_decode_q8_kernel": (0, 0),
    "kqkv_prefill_f16_kernel": (24, 128),
    "kqkv_generic_kernel": (0, 0),
    "kqkv_flat_kernel": (0, 0),
    "q8_rows_to_f16_kernel": (0, 0),
    "merge_kernel": (0, 0),
    "merge_few_kernel": (0, 0),
    "wkb_f32_kernel": (0, 0),
    "wkb_gemm_kernel": (0, 0),
    "wkb_q8_kernel": (0, 0),
    "wvb_q8_kernel": (0, 0),
    "kvwrite_gemv_kernel": (0, 0),
    "kvwrite_tail_kernel": (0, 0),
}
FIELDS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch", "VGPRs Spill": "vspill",
          "SGPRs Spill": "sspill", "LDS Size [bytes/block]": "lds", "Occupancy [waves/SIMD]": "occ"}


def resources(src):
    r = subprocess.run([HIPCC, *B.HIP_FLAGS, "-I", str(B.ROOT / "include"), "--offload-device-only", "-c", str(src),
                        "-o", "/dev/null", "-Rpass-analysis=kernel-resource-usage"],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    out, cur = {}, None
    for line in r.stdout.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = {}
            continue
        m = re.search(r"remark:\s+([^:]+(?:\[[^\]]+\])?): (\S+) \[-Rpass-analysis", line)
        if m and cur is not None and m.group(1).strip() in FIELDS:
            v = m.group(2)
            out[cur][FIELDS[m.group(1).strip()]] = int(v) if v.lstrip("-").isdigit() else v
    return out


def test_kernel_resource_budgets():
    srcs = sorted(B.CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        reports = list(ex.map(resources, srcs))
    seen = set()
    for rep in reports:
        for name, r in rep.items():
            print(f"{name[:90]:90s} VGPR {r.get('vgpr')} AGPR {r.get('agpr')} spill {r.get('vspill')} "
                  f"scratch {r.get('scratch')} LDS {r.get('lds')}")
            assert r.get("lds", 0) <= LDS_MAX, name
            for frag, (vs, sc) in BUDGET.items():
                if re.search(r"\d" + frag + r"[IE]", name):
                    seen.add(frag)
                    assert r["vspill"] <= vs, (name, r)
                    assert r["scratch"] <= sc, (name, r)
    assert seen == set(BUDGET), set(BUDGET) - seen

"""The committed HBM-traffic counter summaries that bench.py reports as roofline.traffic: each file
belongs to the config bench.py looks it up under, its bytes follow from its own counters and
calibration, and the algorithmic bytes are the per-key figure (1,152 cache + 4 mask) times n_kv
plus the 73,728-byte Qcur block.  CPU-only."""
import json

import pytest

import bench

N_KV = {2: 4096, 3: 32768, 4: 262144}
KEY_BYTES = {"f16": 1152 + 4, "q8": 576 // 32 * 34 + 4}     # cache row + mask, per key


@pytest.mark.parametrize("key", sorted(bench.TRAFFIC_FILES))
def test_traffic_file_matches_its_config(key):
    config, cache = key
    path = bench.TRAFFIC_FILES[key]
    assert path.exists(), path
    tr = json.loads(path.read_text())
    assert tr["config"] == config and tr.get("cache", "f16") == cache
    import aubier_amd as A
    ctype = A.ops.TYPE_Q8_0 if cache == "q8" else A.ops.TYPE_F16
    assert tr["splits"] == A.default_splits(N_KV[config], 32, ctype)    # the library's split count at this length
    assert tr["alg_bytes"] == N_KV[config] * KEY_BYTES[cache] + 32 * 576 * 4
    cal = tr["calibration"]
    # a plain copy of B bytes each way reads about 2 B of FETCH_SIZE bytes per KiB counted and writes B
    assert cal["fetch_scale"] == pytest.approx(bench.CAL_BYTES / 1024 / cal["fetch_kib"], rel=1e-4)
    assert cal["write_scale"] == pytest.approx(bench.CAL_BYTES / 1024 / cal["write_kib"], rel=1e-4)
    assert 1.9 < cal["fetch_scale"] < 2.1 and 0.95 < cal["write_scale"] < 1.05
    fetch = tr["fetch_kib_per_dispatch"] * 1024 * cal["fetch_scale"]
    write = tr["write_kib_per_dispatch"] * 1024 * cal["write_scale"]
    assert tr["fetch_bytes"] == pytest.approx(fetch, rel=1e-4)
    assert tr["write_bytes"] == pytest.approx(write, rel=1e-4)
    assert tr["traffic_bytes"] == pytest.approx(fetch + write, rel=1e-4)
    # the cache is read once: reads within a few percent of the algorithmic bytes, plus at most one
    # fetch of the 73,728-byte Qcur block per XCD L2 (8), which weighs only at short windows
    assert 0.98 * tr["alg_bytes"] < tr["fetch_bytes"] < 1.05 * tr["alg_bytes"] + 8 * 32 * 576 * 4
    assert tr["kernel"] == bench.partial_kernel_name(True, N_KV[config], tr["splits"], q8=cache == "q8")


def test_partial_kernel_name():
    assert bench.partial_kernel_name(True, 32768, 256) == "kqkv_decode_f16_kernel<576,512>"       # 2 tiles
    assert bench.partial_kernel_name(True, 262144, 256) == "kqkv_decode_f16_kernel<576,512>"       # 16 tiles
    assert bench.partial_kernel_name(False, 4096, 16).startswith("kqkv_generic_kernel")

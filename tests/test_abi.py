"""CPU tests of the C ABI (include/mla_m4.h, aubier_amd/libmla_m4.so): the library loads, exports
every entry point the header declares, and its host-side contract checks (the supports_op
mirrors, status codes, the tri-state flag, split counts) behave as documented.  No kernel is
launched: every call here either only inspects descriptors or is rejected before any launch."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import aubier_amd as A
from aubier_amd import ops

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mla_m4.h"


@pytest.fixture(scope="module")
def lib():
    return A.load_library()


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mla_m4_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_all_exported(lib):
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    # and the Python mirror binds exactly the declared set
    assert sorted(ops.exported_symbols()) == names


def test_version_and_status_strings(lib):
    assert lib.mla_m4_version().decode().startswith("mla-m4-gfx950")
    for code, text in ops.STATUS.items():
        assert lib.mla_m4_status_str(code).decode() == text
    assert lib.mla_m4_status_str(-99).decode() == "unknown status"


@pytest.mark.parametrize("flag,gpu,want", [(-1, 1, 1), (-1, 0, 0), (0, 1, 0), (0, 0, 0), (1, 1, 1)])
def test_resolve_flag(flag, gpu, want):
    assert A.resolve_flag(flag, bool(gpu)) == bool(want)


@pytest.mark.parametrize("flag,gpu", [(1, 0), (2, 1), (-2, 0)])
def test_resolve_flag_rejects(flag, gpu):
    with pytest.raises(A.MlaM4Error) as e:
        A.resolve_flag(flag, bool(gpu))
    assert e.value.status == -6


# ------------------------------------------------------------------ descriptors (host memory)
def decode_tensors(n_kv=1024, H=32, nt=1, dk=576, dv=512, dtype=torch.float16):
    kc = torch.zeros((n_kv, dk), dtype=dtype)
    q = torch.zeros((nt, H, dk), dtype=torch.float32)
    mask = torch.zeros((nt, n_kv), dtype=torch.float32)
    out = torch.zeros((H, nt, dv), dtype=torch.float32)
    return kc, q, mask, out


def test_supports_kqkv_accepts_both_geometries_and_types():
    assert A.supports_kqkv(*decode_tensors())
    assert A.supports_kqkv(*decode_tensors(dk=320, dv=256))
    assert A.supports_kqkv(*decode_tensors(dtype=torch.float32))
    kc, q, _, out = decode_tensors(nt=4, H=8)
    assert A.supports_kqkv(kc, q, None, out)                  # no mask


def test_supports_kqkv_rejects_contract_violations():
    kc, q, mask, out = decode_tensors()
    assert not A.supports_kqkv(kc, q, mask, torch.zeros((32, 1, 511)))           # D_v not a multiple of 4
    assert not A.supports_kqkv(kc, q, mask, torch.zeros((32, 2, 512)))           # nt mismatch
    assert not A.supports_kqkv(kc, q[:, :, :320].contiguous(), mask, out)        # D_k mismatch
    assert not A.supports_kqkv(kc, q, mask[:, :1000], out)                       # mask width != n_kv
    assert not A.supports_kqkv(kc, q.half(), mask, out)                          # q must be F32
    big = torch.zeros((1024, 580), dtype=torch.float16)
    assert not A.supports_kqkv(big[:, 1:577], q, mask, out)                      # misaligned rows
    assert not A.supports_kqkv(torch.zeros((1024, 1100), dtype=torch.float16), torch.zeros((1, 32, 1100)),
                               mask, torch.zeros((32, 1, 512)))                   # D_k > 1024


def test_supports_accept_unallocated_tensors():
    """supports_op runs during graph planning, before the tensors have data."""
    views = [ops.view(t) for t in decode_tensors()]
    for v in views:
        v.data = None
    P = ctypes.byref
    lib = A.load_library()
    assert lib.mla_m4_supports_kqkv(P(views[0]), P(views[1]), P(views[2]), P(views[3])) == 1
    views[3].ne[0] = 500
    assert lib.mla_m4_supports_kqkv(P(views[0]), P(views[1]), P(views[2]), P(views[3])) == 0
    part, out = ops.view(torch.zeros((1, 1, 4, ops.part_floats(512)))), ops.view(torch.zeros((32, 1, 512)))
    part.data = out.data = None
    assert lib.mla_m4_supports_phase(ops.PHASE_MERGE, P(part), P(out)) == 1
    # the launch itself still rejects null data
    assert lib.mla_m4_phase_merge(P(part), P(out), None) == -1


def test_supports_wkb():
    w = torch.zeros((32, 512, 128))
    q = torch.zeros((1, 32, 192))
    qcur = torch.zeros((1, 32, 576))
    assert A.supports_wkb(w, q[:, :, :128], qcur[:, :, :512])      # strided views, as the engine uses
    assert not A.supports_wkb(w, q[:, :, :64], qcur[:, :, :512])   # d_n mismatch
    assert not A.supports_wkb(torch.zeros((32, 512, 96)), torch.zeros((1, 32, 96)), qcur[:, :, :512])  # d_n 96


def test_supports_phase():
    G, S, dv = 1, 256, 512
    part = torch.zeros((G, 1, S, ops.part_floats(dv)))
    out = torch.zeros((32, 1, dv))
    assert A.supports_phase(ops.PHASE_MERGE, part, out)
    assert A.supports_phase(ops.PHASE_MERGE, torch.zeros((G, 1, S, ops.part_floats(dv, False))), out)
    assert not A.supports_phase(ops.PHASE_MERGE, torch.zeros((G, 1, S, 1000)), out)
    assert not A.supports_phase(ops.PHASE_MERGE, torch.zeros((G, 1, 1025, ops.part_floats(dv))), out)
    assert not A.supports_phase(ops.PHASE_KVWRITE, part, out)     # phases 0 and 1: not in this library
    assert not A.supports_phase(ops.PHASE_WVB, part, out)
    assert not A.supports_phase(7, part, out)


def test_default_splits_and_workspace(lib):
    # one token, f16 cache: about one workgroup per CU, at most one split per 64-key tile (measured
    # fastest for the partial + merge step as well)
    assert A.default_splits(32768) == 256
    assert A.default_splits(8192) == 128 and A.default_splits(16384) == 256 and A.default_splits(24576) == 256
    assert A.default_splits(12288) == 192 and A.default_splits(4096) == 64
    assert A.default_splits(65536) == 256 and A.default_splits(262144) == 256
    assert A.default_splits(32768, 32, ops.TYPE_Q8_0) == 256                # the 8-bit cache keeps 256
    assert A.default_splits(64) == 1
    assert 1 <= A.default_splits(4096) <= 64                     # at most one split per 64-key tile
    assert A.default_splits(262144) <= ops.MAX_SPLITS
    assert lib.mla_m4_kqkv_default_splits(0, 32, 1) == -6
    kc, q, _, out = decode_tensors(n_kv=32768)
    S = A.default_splits(32768)
    assert A.kqkv_workspace_bytes(kc, q, out) == S * ops.part_floats(512) * 4
    # a short window (one token, an f16 cache of <= 256 keys or an f32 one of <= 512) runs the
    # one-launch kernel: records of (m, l, o) per (head, split of <= 32 keys), D_v + 4 floats each
    kc, q, _, out = decode_tensors(n_kv=64)
    assert A.kqkv_workspace_bytes(kc, q, out) == 32 * 2 * (512 + 4) * 4
    kc, q, _, out = decode_tensors(n_kv=256)
    assert A.kqkv_workspace_bytes(kc, q, out) == max(32 * 8 * (512 + 4) * 4, A.default_splits(256) * ops.part_floats(512) * 4)
    kc, q, _, out = decode_tensors(n_kv=512, dtype=torch.float32)
    assert A.kqkv_workspace_bytes(kc, q, out) == max(32 * 16 * (512 + 4) * 4, A.default_splits(512) * ops.part_floats(512) * 4)
    kc, q, _, out = decode_tensors(n_kv=512)                      # f16 at 512 keys: split-K
    assert A.kqkv_workspace_bytes(kc, q, out) == A.default_splits(512) * ops.part_floats(512) * 4
    # a long single-split decode needs none
    kc, q, _, out = decode_tensors(n_kv=64, dtype=torch.float16)
    q2 = torch.zeros((2, 32, 576))
    assert A.kqkv_workspace_bytes(kc, q2, torch.zeros((32, 2, 512))) == 0      # two tokens, one tile: one split


def test_entry_points_reject_before_launching(lib):
    kc, q, mask, out = decode_tensors()
    vk, vq, vm, vo = (ops.view(t) for t in (kc, q, mask, out))
    P = ctypes.byref
    assert lib.mla_m4_kqkv(None, P(vq), P(vm), ctypes.c_float(0.1), P(vo), None, 0, None) == -1
    assert lib.mla_m4_kqkv(P(vk), P(vq), P(vm), ctypes.c_float(float("nan")), P(vo), None, 0, None) == -6
    # split-K shapes need a workspace
    assert lib.mla_m4_kqkv(P(vk), P(vq), P(vm), ctypes.c_float(0.1), P(vo), None, 0, None) == -5
    part = ops.view(torch.zeros((1, 1, 8, ops.part_floats(512))))
    assert lib.mla_m4_kqkv_partial(P(vk), P(vq), P(vm), ctypes.c_float(0.1), 0, 512, P(part), None) == -6
    assert lib.mla_m4_kqkv_partial(P(vk), P(vq), P(vm), ctypes.c_float(0.1), 9, 512, P(part), None) == -3
    assert lib.mla_m4_kqkv_partial(P(vk), P(vq), P(vm), ctypes.c_float(0.1), 8, 512, None, None) == -1
    w = ops.view(torch.zeros((32, 512, 128)))
    assert lib.mla_m4_wkb(P(w), None, P(vo), None) == -1
    assert lib.mla_m4_phase_merge(None, P(vo), None) == -1


def test_q8_prefill_rejects_a_workspace_without_room_for_the_copy(lib):
    """A workspace that holds the partials but not the 8-bit cache's f16 copy is refused before
    any launch (the pointer below is never dereferenced: the size check comes first)."""
    kc = q8((1500,), 576)
    _, q, mask, out = decode_tensors(n_kv=1500, nt=20)
    need = A.kqkv_workspace_bytes(kc, q, out)
    copy = (1500 * 576 * 2 + 255) // 256 * 256
    P = ctypes.byref
    vk, vq, vm, vo = ops.view(kc), ops.view(q), ops.view(mask), ops.view(out)
    fake = ctypes.c_void_p(1 << 20)                               # 16-byte aligned, never used
    for size in (need - copy, need - 1):
        assert lib.mla_m4_kqkv(P(vk), P(vq), P(vm), ctypes.c_float(0.1), P(vo), fake, size, None) == -5


def test_product_path_has_no_cpu_fallback(monkeypatch, tmp_path):
    """Without the built library every op raises instead of computing anything on the host."""
    monkeypatch.setattr(ops, "_lib", None)
    monkeypatch.setattr(ops, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(RuntimeError, match="no CPU path"):
        A.ggml_m4_wkb(torch.zeros((32, 512, 128)), torch.zeros((1, 32, 128)))


# ------------------------------------------------------------------ quantised ops (reference geometry)
def q8(rows_shape, ne0):
    return A.Q8_0(torch.zeros(*rows_shape, ne0 // 32 * 34, dtype=torch.uint8), ne0)


def test_supports_wkb_q8():
    w = q8((32, 256), 64)                                    # the reference's W_kb, Q8_0 [64, 256, 32]
    q = torch.zeros((1, 32, 128))
    assert A.supports_wkb(w, q[:, :, :64], torch.zeros((1, 32, 256)))
    assert A.supports_wkb(q8((32, 512), 128), torch.zeros((2, 32, 192))[:, :, :128], torch.zeros((2, 32, 512)))
    assert not A.supports_wkb(q8((32, 256), 96), torch.zeros((1, 32, 96)), torch.zeros((1, 32, 256)))   # d_n 96
    v = ops.view(w)
    v.nb[0] = 36                                             # not a packed Q8_0 row
    assert A.load_library().mla_m4_supports_wkb(ctypes.byref(v), ctypes.byref(ops.view(q[:, :, :64])),
                                                ctypes.byref(ops.view(torch.zeros((1, 32, 256))))) == 0


def test_supports_phase_wvb():
    w = q8((32, 128), 256)                                   # the reference's attn_v_b, Q8_0 [256, 128, 32]
    assert A.supports_phase_wvb(w, torch.zeros((32, 1, 256)), torch.zeros((32, 1, 128)))
    assert A.supports_phase_wvb(q8((32, 128), 512), torch.zeros((32, 7, 512)), torch.zeros((32, 7, 128)))
    assert not A.supports_phase_wvb(w, torch.zeros((32, 1, 256)), torch.zeros((32, 2, 128)))      # nt mismatch
    assert not A.supports_phase_wvb(q8((32, 128), 96), torch.zeros((32, 1, 96)), torch.zeros((32, 1, 128)))
    assert not A.supports_phase_wvb(w, torch.zeros((32, 1, 256), dtype=torch.float16), torch.zeros((32, 1, 128)))


def kv_descs(n_embd=4096, d_lat=256, n_dims=64, n_kv=100):
    n_out = d_lat + n_dims
    return (torch.zeros(n_embd), q8((n_out,), n_embd), torch.zeros(d_lat), torch.zeros((n_kv, n_out), dtype=torch.float16),
            torch.zeros(1, dtype=torch.int64), torch.zeros(1, dtype=torch.int32))


RP = dict(freq_base=10000.0, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0, eps=1e-6,
          n_ctx_orig=4096)


def test_supports_phase_kvwrite():
    rp = A.rope_params(n_dims=64, **RP)
    assert A.supports_phase_kvwrite(*kv_descs(), rp, torch.zeros(320))                       # the reference's
    assert A.supports_phase_kvwrite(*kv_descs(7168, 512), rp, torch.zeros(576))                # 576-wide cache
    assert not A.supports_phase_kvwrite(*kv_descs(), rp, torch.zeros(321))                     # dst width
    assert not A.supports_phase_kvwrite(*kv_descs(n_embd=2048), rp, torch.zeros(320))          # n_embd
    d = list(kv_descs())
    d[4] = torch.zeros(1, dtype=torch.int32)                                                   # kidx must be I64
    assert not A.supports_phase_kvwrite(*d, rp, torch.zeros(320))
    bad = A.rope_params(n_dims=64, **{**RP, "freq_base": 0.0})
    assert not A.supports_phase_kvwrite(*kv_descs(), bad, torch.zeros(320))


def test_supports_phase_kvwrite_q8_cache():
    """KV-write into an 8-bit (Q8_0) cache: whole-block rows, 2-byte aligned scales."""
    rp = A.rope_params(n_dims=64, **RP)
    lib = A.load_library()
    for n_embd, d_lat in ((4096, 256), (7168, 512)):
        d = list(kv_descs(n_embd, d_lat))
        n_out = d_lat + 64
        d[3] = q8((100,), n_out)
        assert A.supports_phase_kvwrite(*d, rp, torch.zeros(n_out))
        v = [ops.view(t) for t in d]
        dst = ops.view(torch.zeros(n_out))
        ok = lambda: lib.mla_m4_supports_phase_kvwrite(*(ctypes.byref(x) for x in v), ctypes.byref(rp), ctypes.byref(dst))
        v[3].nb[1] += 2                                     # padded rows: fine
        assert ok()
        v[3].nb[1] += 1                                     # odd row pitch: scales unaligned
        assert not ok()
        v[3].nb[1] -= 3
        v[3].nb[0] = 32                                     # not ggml's block size
        assert not ok()


def test_phase_entry_points_reject_before_launching():
    lib = A.load_library()
    P = ctypes.byref
    w, x, out = ops.view(q8((32, 128), 256)), ops.view(torch.zeros((32, 1, 256))), ops.view(torch.zeros((32, 1, 128)))
    assert lib.mla_m4_phase_wvb(P(w), None, P(out), None) == -1
    descs = [ops.view(t) for t in kv_descs()]
    assert lib.mla_m4_phase_kvwrite(*(P(v) for v in descs), None, P(ops.view(torch.zeros(320))), None) == -1
    assert lib.mla_m4_phase_kvwrite(*(P(v) for v in descs), P(A.rope_params(n_dims=64, **RP)),
                                    P(ops.view(torch.zeros(300))), None) == -3


# ------------------------------------------------------------------ 8-bit (Q8_0) latent cache
def test_supports_kqkv_q8_cache():
    """A Q8_0 cache (ggml block_q8_0 rows) at both instantiated geometries; other widths, a
    non-block width and padded rows are refused.  Its partials hold f16 o, like an F16 cache's."""
    _, q, mask, out = decode_tensors(n_kv=1000)
    assert A.supports_kqkv(q8((1000,), 576), q, mask, out)
    _, q3, mask3, out3 = decode_tensors(n_kv=1000, dk=320, dv=256, nt=3)
    assert A.supports_kqkv(q8((1000,), 320), q3, mask3, out3)
    _, q5, mask5, out5 = decode_tensors(n_kv=1000, dk=512, dv=448)
    assert not A.supports_kqkv(q8((1000,), 512), q5, mask5, out5)                 # no Q8_0 kernel for 512
    kc = q8((1000,), 576)
    padded = ops.view(kc)
    padded.nb[1] = 640                                                            # rows not contiguous
    P = ctypes.byref
    lib = A.load_library()
    vq, vm, vo = ops.view(q), ops.view(mask), ops.view(out)
    assert lib.mla_m4_supports_kqkv(P(ops.view(kc)), P(vq), P(vm), P(vo)) == 1
    assert lib.mla_m4_supports_kqkv(P(padded), P(vq), P(vm), P(vo)) == 0
    odd = ops.view(kc)
    odd.ne[0] = 560                                                               # not whole 32-value blocks
    assert lib.mla_m4_supports_kqkv(P(odd), P(vq), P(vm), P(vo)) == 0
    S = A.default_splits(32768, 32, ops.TYPE_Q8_0)
    assert S == 256
    _, q, _, out = decode_tensors(n_kv=32768)
    assert A.kqkv_workspace_bytes(q8((32768,), 576), q, out) == S * ops.part_floats(512, True) * 4


@pytest.mark.parametrize("dk,dv", [(576, 512), (320, 256)])
def test_q8_prefill_workspace_holds_the_f16_copy(dk, dv):
    """From 16 tokens KQKV over an 8-bit cache runs the f16 prefill kernel on an f16 copy of the
    cache at the head of its workspace (256-byte rounded), the partials after it, at the f16
    prefill's own split count; below 16 tokens (the 8-bit decode kernel) there is no copy."""
    for n_kv in (1500, 8192):
        kc16, q, _, out = decode_tensors(n_kv=n_kv, nt=20, dk=dk, dv=dv)
        copy = (n_kv * dk * 2 + 255) // 256 * 256
        assert A.kqkv_workspace_bytes(q8((n_kv,), dk), q, out) == copy + A.kqkv_workspace_bytes(kc16, q, out)
    kc16, q, _, out = decode_tensors(n_kv=1500, nt=15, dk=dk, dv=dv)
    S = A.default_splits(1500, 32, ops.TYPE_Q8_0)   # the 8-bit decode kernel: the single-row count
    assert A.kqkv_workspace_bytes(q8((1500,), dk), q, out) == 15 * S * ops.part_floats(dv, True) * 4


def test_q8_cache_size_limit():
    """The 8-bit cache kernel addresses rows from a tile's first key to the end of the cache through a
    32-bit buffer range, so the contract keeps the whole Q8_0 cache within 4 GiB: 7,017,920 keys of
    612 bytes at D_k = 576 are accepted, one more is not (descriptors without data, as in planning)."""
    lib = A.load_library()
    P = ctypes.byref
    n_max = 0xFFFFFFFF // 612
    assert n_max == 7017920

    def views(n_kv):
        kc = ops.MlaTensor()
        kc.type = ops.TYPE_Q8_0
        for i, (ne, nb) in enumerate([(576, 34), (n_kv, 612), (1, 612 * n_kv), (1, 612 * n_kv)]):
            kc.ne[i], kc.nb[i] = ne, nb
        q = ops.view(torch.zeros((1, 32, 576)))
        out = ops.view(torch.zeros((32, 1, 512)))
        mask = ops.MlaTensor()
        mask.type = ops.TYPE_F32
        for i, (ne, nb) in enumerate([(n_kv, 4), (1, 4 * n_kv), (1, 4 * n_kv), (1, 4 * n_kv)]):
            mask.ne[i], mask.nb[i] = ne, nb
        for v in (q, out):
            v.data = None
        return kc, q, mask, out

    assert lib.mla_m4_supports_kqkv(*(P(v) for v in views(n_max))) == 1
    assert lib.mla_m4_supports_kqkv(*(P(v) for v in views(n_max + 1))) == 0

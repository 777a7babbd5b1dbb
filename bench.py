"""MLA decode attention benchmark on one MI355X (BASELINE.json metric: us per decode step plus
achieved HBM GB/s as a fraction of peak, at 32,768 keys).

    python bench.py [--steps K] [--warmup W] [--config 3] [--splits S] [--no-cpu] [--no-others]

One step = the MLA attention of one decode token, as the engine's layer graph runs it:
GGML_OP_M4_WKB (absorbed q_nope written into the Qcur buffer) -> GGML_OP_M4_KQKV (the split-K
partial kernel, then the PHASE merge kernel; for a short window, one launch that merges its own
splits), through the C ABI, on seeded synthetic inputs
(aubier_amd.inputs).  The steps are captured in hipGraphs (the way the engine runs them) and
replayed; consecutive steps read different copies of the KV cache and W_kb (enough copies that
a full rotation exceeds 512 MiB, twice the 256 MB MALL), so every step streams from HBM (COLD).
Exactly K steps are timed (whole rotations plus one graph of the remainder), after exactly W
untimed warm-up steps.

Prints ONE JSON line.  `roofline` is for the dominant kernel (the split-K partial, or the
one-launch kernel of a short window, timed as the whole op): algorithmic
bytes per launch (n_kv * (1152 cache + 4 mask) + Qcur) / its average duration, timed with HIP
events around a graph of back-to-back launches on the stream they run on.  `cpu_baseline` is the
CPU oracle (the restated unfused ggml graph) on the host threads this process may use, same
inputs, median of 5.  `extra.configs` times every other BASELINE config the same way, with the
error of one GPU step against the CPU oracle, so one run fills the results table.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs/decode-step + achieved HBM GB/s (% peak) for MLA attention at 32K keys"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
COLD_BYTES = 512 << 20         # bytes one rotation of step inputs must exceed (2 x the MALL)
GRAPH_MIN_STEPS = 64           # steps per captured graph, at least
CAL_BYTES = 256 << 20          # calibration copy size (each way) for the HBM traffic counters
TRAFFIC_FILES = {(3, "f16"): ROOT / "profiles" / "kqkv_decode_f16_cfg3_traffic.json",   # per (decode config, cache)
                 (4, "f16"): ROOT / "profiles" / "kqkv_decode_f16_cfg4_traffic.json",
                 (3, "q8"): ROOT / "profiles" / "kqkv_decode_q8_cfg3_traffic.json",
                 (4, "q8"): ROOT / "profiles" / "kqkv_decode_q8_cfg4_traffic.json",
                 (2, "f16"): ROOT / "profiles" / "kqkv_decode_f16_cfg2_traffic.json"}


def partial_kernel_name(kc_f16: bool, n_kv: int, n_split: int, q8: bool = False) -> str:
    """The kernel the library launches for the split-K partial of one decode row: an f16 cache
    takes the barrier-per-tile MFMA kernel at every split length (launch_kqkv_decode_f16); an f32
    cache the VALU kernel; a Q8_0 cache its own kernel (launch_kqkv_decode_q8)."""
    if q8:
        return "kqkv_decode_q8_kernel<576,512>"
    if not kc_f16:
        return "kqkv_generic_kernel<f32 cache>"
    return "kqkv_decode_f16_kernel<576,512>"


def cpu_threads() -> dict:
    """Host threads for the CPU baseline: every CPU this process may run on, capped by the
    OMP_NUM_THREADS share the GPU box sets for one GPU."""
    visible = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    used = min(visible, share) if share > 0 else visible
    return {"threads": used, "host_cpus_visible": visible, "omp_num_threads": share or None,
            "os_cpu_count": os.cpu_count()}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=288)
    ap.add_argument("--warmup", type=int, default=72)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--splits", type=int, default=0, help="split count (0 = library default)")
    ap.add_argument("--batch", type=int, default=0,
                    help="batch-of-N decode: N rows, each over its own 32768/N-cell region of one window")
    ap.add_argument("--no-sweep", action="store_true", help="skip the S in {64,128,192,256} sweep")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-others", action="store_true", help="time the headline config only")
    ap.add_argument("--cache", choices=("f16", "q8"), default="f16",
                    help="q8: the decode config's cache quantised to ggml Q8_0 (the 8-bit latent cache kernel); "
                         "the CPU baseline and the errors use the f16 values it stands for")
    ap.add_argument("--ops", action="store_true",
                    help="time the reference-geometry quantised ops (Q8_0 WKB, PHASE wv_b, PHASE KV-write) instead")
    ap.add_argument("--layer", action="store_true",
                    help="us per attention layer (KV-write -> WKB -> concat -> KQKV -> wv_b), both geometries")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="no timing: run the calibration copy and a few steps, for rocprofv3 --pmc")
    return ap.parse_args()


def errors(out: np.ndarray, ref: np.ndarray) -> dict:
    """max abs error, and max / RMS error relative to max|ref| (the outputs are ~0.05 / sqrt(L))."""
    d = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    scale = float(np.abs(ref).max()) or 1.0
    return {"max_abs": float(d.max()), "max_rel": float(d.max() / scale),
            "rms_rel": float(np.sqrt((d ** 2).mean()) / scale)}


class Rotated:
    """Graph capture and timing over rotating input copies (COLD): a subclass sets torch, n_rot
    (copies, one rotation > COLD_BYTES of reads), glen (steps per graph, whole rotations) and
    step(i) (one step on copy i)."""

    def capture(self, fn, n, start=0):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            # untimed eager warm-up on the capture stream, on the two copies before `start` (those
            # a replay from `start` follows anyway), so that the graph's first copy stays COLD
            for i in range(2):
                fn((start - 2 + i) % self.n_rot)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for i in range(n):
                fn((start + i) % self.n_rot)
        return g

    def time_graph(self, g, reps, per):
        """us per unit: replay g `reps` times (each replay = `per` units) between two events."""
        torch = self.torch
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (reps * per)

    def run_steps(self, k, warmup, step=None):
        """Exactly `warmup` untimed then exactly `k` timed steps (graphs of glen steps, the
        remainder as one more graph); returns (us per step, wall seconds of the timed region, the
        rotation index the timed steps start at).  The warm-up starts at rotation index 0 and the
        timed steps at the index after the warm-up's last, so the first timed step reads a copy
        last read a whole rotation (> 512 MiB of reads) earlier: every timed step is COLD."""
        torch = self.torch
        step = step or self.step
        w0 = warmup % self.n_rot
        graphs = {}

        def graph(n, start):
            if (n, start) not in graphs:
                graphs[(n, start)] = self.capture(step, n, start)
            return graphs[(n, start)]

        def replay_n(n, start):
            # a full graph covers whole rotations, so it ends at the index it started at
            for _ in range(n // self.glen):
                graph(self.glen, start).replay()
            if n % self.glen:
                graph(n % self.glen, start).replay()

        for n, start in ((warmup, 0), (k, w0)):      # capture everything before the first replay
            if n >= self.glen:
                graph(self.glen, start)
            if n % self.glen:
                graph(n % self.glen, start)
        torch.cuda.synchronize()
        replay_n(warmup, 0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        replay_n(k, w0)
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return e0.elapsed_time(e1) * 1000.0 / k, wall, w0


class Decode(Rotated):
    """Device buffers and launch closures of one decode configuration (nt rows, W keys)."""

    def __init__(self, inp, splits: int = 0):
        import torch
        import aubier_amd as A
        from aubier_amd import inputs as I
        self.A, self.I, self.torch, self.inp = A, I, torch, inp
        dev = torch.device("cuda:0")
        H, DV, DK = I.N_HEAD, I.D_V, I.D_K
        self.H, self.DV, self.DK, self.W = H, DV, DK, inp.n_kv
        self.q8 = inp.kcache_q8 is not None
        es = 2 if inp.kc_f16 else 4
        self.es = es
        row = DK // 32 * 34 if self.q8 else DK * es                                # cache bytes per key
        self.bytes_attn = inp.n_kv * (row + 4) + inp.nt * H * DK * 4               # cache + mask + Qcur
        self.bytes_wkb = H * DV * I.D_NOPE * 4 + inp.nt * H * I.D_NOPE * 4 + inp.nt * H * DV * 4
        self.bytes_out = inp.nt * H * DV * 4
        self.bytes_step = self.bytes_attn + self.bytes_out + self.bytes_wkb
        kc_bytes = inp.n_kv * row
        per_step = kc_bytes + H * DV * I.D_NOPE * 4
        self.n_rot = max(12, math.ceil(COLD_BYTES / per_step))
        # steps per captured graph: whole rotations, at least GRAPH_MIN_STEPS (a graph replay costs
        # ~6 us of its own, which an engine spreads over a whole forward pass of many layers)
        self.glen = self.n_rot * math.ceil(GRAPH_MIN_STEPS / self.n_rot)
        kc0 = torch.from_numpy(np.ascontiguousarray(inp.kcache_q8 if self.q8 else inp.kcache)).to(dev)
        wkb0 = torch.from_numpy(inp.w_kb).to(dev)
        q = np.concatenate([inp.q_nope, inp.q_pe], axis=2).astype(np.float32)
        q0 = torch.from_numpy(q).to(dev)
        self.mask = torch.from_numpy(inp.mask).to(dev)
        self.kcs = [kc0] + [kc0.clone() for _ in range(self.n_rot - 1)]
        if self.q8:
            self.kcs = [A.Q8_0(k, DK) for k in self.kcs]
        self.wkbs = [wkb0] + [wkb0.clone() for _ in range(self.n_rot - 1)]
        self.qs = [q0] + [q0.clone() for _ in range(self.n_rot - 1)]
        self.qcurs = []
        for i in range(self.n_rot):
            qc = torch.zeros((inp.nt, H, DK), dtype=torch.float32, device=dev)
            qc[:, :, DV:] = self.qs[i][:, :, I.D_NOPE:]
            self.qcurs.append(qc)
        self.S = splits or A.default_splits(self.W, H, A.ops.TYPE_Q8_0 if self.q8 else
                                            (A.ops.TYPE_F16 if inp.kc_f16 else A.ops.TYPE_F32))
        self.part = self.new_part(self.S)
        self.out = torch.empty((H, inp.nt, DV), dtype=torch.float32, device=dev)
        # the op's own workspace (what the glue takes from the ggml pool)
        need = A.kqkv_workspace_bytes(self.kcs[0], self.qcurs[0], self.out)
        self.ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        # a short window runs as one launch (kqkv_flat.hip), longer ones as partial + merge
        self.flat = inp.nt == 1 and not self.q8 and inp.n_kv <= (256 if inp.kc_f16 else 512)
        torch.cuda.synchronize()

    def new_part(self, S):
        return self.torch.empty(((self.H + 31) // 32, self.inp.nt, S, self.A.ops.part_floats(self.DV, self.inp.kc_f16)),
                                dtype=self.torch.float32, device="cuda:0")

    def wkb(self, i):
        self.A.ggml_m4_wkb(self.wkbs[i], self.qs[i][:, :, :self.I.D_NOPE], out=self.qcurs[i][:, :, :self.DV])

    def attn(self, i, part=None, S=None):
        self.A.ggml_m4_kqkv_partial(self.kcs[i], self.qcurs[i], self.mask, self.inp.kq_scale, S or self.S,
                                    part=part if part is not None else self.part, d_v=self.DV)

    def merge(self, part=None):
        self.A.ggml_m4_phase_merge(part if part is not None else self.part, out=self.out, n_head=self.H, d_v=self.DV)

    def kqkv(self, i):
        """GGML_OP_M4_KQKV as the engine's glue calls it, with its workspace: the split-K partial
        kernel, then the PHASE merge (or, for a short window, the one-launch kernel)."""
        self.A.ggml_m4_kqkv(self.kcs[i], self.qcurs[i], self.mask, self.inp.kq_scale, out=self.out, workspace=self.ws)

    def step(self, i):
        """WKB -> KQKV."""
        self.wkb(i)
        self.kqkv(i)

    def per_kernel(self, reps):
        """Per-launch us of each kernel: graphs of back-to-back launches (COLD)."""
        n = self.glen
        return {"wkb": self.time_graph(self.capture(self.wkb, n), reps, n),
                "kqkv": self.time_graph(self.capture(self.kqkv, n), reps, n),
                "partial": self.time_graph(self.capture(self.attn, n), reps, n),
                "merge": self.time_graph(self.capture(lambda i: self.merge(), n), reps, n)}

    def warm_step(self, reps):
        return self.time_graph(self.capture(lambda i: self.step(0), self.glen), reps, self.glen)

    def split_sweep(self, reps):
        """Per split count: the partial and the merge each in graphs of their own launches, and the
        whole step (WKB -> partial -> merge), in which the merge reads the records the partial has
        just written."""
        res = {}
        for S in (64, 128, 192, 256):
            p = self.new_part(S)
            ua = self.time_graph(self.capture(lambda i, p=p, S=S: self.attn(i, p, S), self.glen), reps, self.glen)
            um = self.time_graph(self.capture(lambda i, p=p: self.merge(p), self.glen), reps, self.glen)
            us = self.time_graph(self.capture(lambda i, p=p, S=S: (self.wkb(i), self.attn(i, p, S), self.merge(p)), self.glen),
                                 reps, self.glen)
            res[str(S)] = {"us_partial": round(ua, 3), "us_merge": round(um, 3), "us_step": round(us, 3),
                           "partial_GBps": round(self.bytes_attn / (ua * 1e3), 1)}
        return res

    def gpu_output(self):
        self.step(0)
        self.torch.cuda.synchronize()
        return self.out.cpu().numpy()


class Layer(Rotated):
    """One attention layer of a decode step (one token), as the engine's captured layer graph runs
    it (engine/m1_layer.cpp:411-442 builds the chain; engine/m1_session.h:155-158 prices the M4 ops per
    layer in situ), COLD: the cache and every weight rotate over copies.
      geometry "ref" -- the reference engine's: KV row 320 (256 latent + 64 rope), Q8_0 W_kb
        [64,256,32], Q8_0 wkv_a [4096,320] and wv_b [256,128,32]:
        PHASE KV-write -> WKB -> concat (the rope half into Qcur) -> KQKV -> PHASE wv_b;
      geometry "baseline" -- BASELINE.json's: KV row 576, f32 W_kb [128,512,32]: WKB -> KQKV.
    The new token's row is written at position n_kv - 1 and every key is live."""

    GEOM = {"ref": dict(d_n=64, d_r=64, d_lat=256, n_embd=4096, d_out=128),
            "baseline": dict(d_n=128, d_r=64, d_lat=512)}
    ROPE = dict(freq_base=1e6, freq_scale=0.25, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
                eps=1e-6, n_ctx_orig=8192)

    def __init__(self, geom: str, n_kv: int, seed: int = 9600):
        import torch
        import aubier_amd as A
        self.torch, self.A, self.geom, self.W = torch, A, geom, n_kv
        g = self.GEOM[geom]
        H = self.H = 32
        d_n, d_r, d_lat = self.d_n, self.d_r, self.d_lat = g["d_n"], g["d_r"], g["d_lat"]
        dk = d_lat + d_r
        self.full = geom == "ref"
        dev = torch.device("cuda:0")
        rng = np.random.default_rng(seed)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)

        def q8_blocks(rows, ne0):
            nb = ne0 // 32
            b = np.empty((rows, nb, 34), dtype=np.uint8)
            b[:, :, :2] = (np.abs(rng.standard_normal((rows, nb))) * 0.01 + 0.001).astype(np.float16) \
                .view(np.uint8).reshape(rows, nb, 2)
            b[:, :, 2:] = rng.integers(-127, 128, size=(rows, nb, 32)).astype(np.int8).view(np.uint8)
            return torch.from_numpy(b.reshape(rows, nb * 34)).to(dev)

        # bytes each step reads or writes, op by op (weights, activations, outputs, the cache)
        kc_bytes = n_kv * dk * 2
        by = {"wkb": (H * d_lat * d_n // 32 * 34 if self.full else H * d_lat * d_n * 4) + H * d_n * 4 + H * d_lat * 4,
              "kqkv": kc_bytes + n_kv * 4 + H * dk * 4 + H * d_lat * 4}
        if self.full:
            n_embd, d_out = g["n_embd"], g["d_out"]
            by["kvwrite"] = dk * n_embd // 32 * 34 + n_embd * 4 + d_lat * 4 + dk * 4 + dk * 2
            by["concat"] = 2 * H * d_r * 4
            by["wvb"] = H * d_out * d_lat // 32 * 34 + H * d_lat * 4 + H * d_out * 4
        self.bytes = by
        rot_bytes = kc_bytes + by["wkb"] + by.get("kvwrite", 0) + by.get("wvb", 0)
        self.n_rot = max(12, math.ceil(COLD_BYTES / rot_bytes))
        self.glen = self.n_rot * math.ceil(GRAPH_MIN_STEPS / self.n_rot)
        R = self.n_rot

        kc0 = (torch.randn((n_kv, dk), generator=gen, device=dev) * 0.05).to(torch.float16)
        self.kcs = [kc0] + [kc0.clone() for _ in range(R - 1)]
        q0 = torch.randn((1, H, d_n + d_r), generator=gen, device=dev) * 0.05
        self.qs = [q0] + [q0.clone() for _ in range(R - 1)]
        if self.full:
            w = q8_blocks(H * d_lat, d_n).view(H, d_lat, d_n // 32 * 34)
            self.wkbs = [A.Q8_0(x, d_n) for x in [w] + [w.clone() for _ in range(R - 1)]]
            w = q8_blocks(dk, n_embd)
            self.wkvas = [A.Q8_0(x, n_embd) for x in [w] + [w.clone() for _ in range(R - 1)]]
            w = q8_blocks(H * d_out, d_lat).view(H, d_out, d_lat // 32 * 34)
            self.wvbs = [A.Q8_0(x, d_lat) for x in [w] + [w.clone() for _ in range(R - 1)]]
            c0 = torch.randn(n_embd, generator=gen, device=dev)
            self.curs = [c0] + [c0.clone() for _ in range(R - 1)]
            self.nw = (1.0 + 0.25 * torch.randn(d_lat, generator=gen, device=dev)).contiguous()
            self.kidx = torch.tensor([n_kv - 1], dtype=torch.int64, device=dev)
            self.pos = torch.tensor([n_kv - 1], dtype=torch.int32, device=dev)
            self.rope = A.rope_params(n_dims=d_r, **self.ROPE)
            self.kcur = torch.empty(dk, dtype=torch.float32, device=dev)
            self.out = torch.empty((H, 1, d_out), dtype=torch.float32, device=dev)
        else:
            w = torch.randn((H, d_lat, d_n), generator=gen, device=dev) * 0.05
            self.wkbs = [w] + [w.clone() for _ in range(R - 1)]
        self.qcur = torch.zeros((1, H, dk), dtype=torch.float32, device=dev)
        if not self.full:                       # no concat in this chain: the rope half is set once
            self.qcur[:, :, d_lat:] = q0[:, :, d_n:]
        self.mask = torch.zeros((1, n_kv), dtype=torch.float32, device=dev)
        self.kqv = torch.empty((H, 1, d_lat), dtype=torch.float32, device=dev)
        self.kq_scale = 1.0 / math.sqrt(d_n + d_r)
        need = A.kqkv_workspace_bytes(self.kcs[0], self.qcur, self.kqv)
        self.ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        self.ops = {"wkb": self.wkb, "kqkv": self.kqkv}
        if self.full:
            self.ops = {"kvwrite": self.kvwrite, "wkb": self.wkb, "concat": self.concat, "kqkv": self.kqkv,
                        "wvb": self.wvb}
        torch.cuda.synchronize()

    def kvwrite(self, i):
        self.A.ggml_m4_phase_kvwrite(self.curs[i], self.wkvas[i], self.nw, self.kcs[i], self.kidx, self.pos, self.rope,
                                     out=self.kcur)

    def wkb(self, i):
        self.A.ggml_m4_wkb(self.wkbs[i], self.qs[i][:, :, :self.d_n], out=self.qcur[:, :, :self.d_lat])

    def concat(self, i):
        self.qcur[:, :, self.d_lat:].copy_(self.qs[i][:, :, self.d_n:])

    def kqkv(self, i):
        self.A.ggml_m4_kqkv(self.kcs[i], self.qcur, self.mask, self.kq_scale, out=self.kqv, workspace=self.ws)

    def wvb(self, i):
        self.A.ggml_m4_phase_wvb(self.wvbs[i], self.kqv, out=self.out)

    def step(self, i):
        for op in self.ops.values():
            op(i)

    def record(self, steps, warmup, reps=8):
        us, wall, w0 = self.run_steps(steps, warmup)
        per_op = {k: self.time_graph(self.capture(f, self.glen), reps, self.glen) for k, f in self.ops.items()}
        total = sum(self.bytes.values())
        return {"n_kv": self.W, "chain": " -> ".join(self.ops), "us_layer": round(us, 3), "wall_s_timed": round(wall, 6),
                "rotating_copies": self.n_rot, "steps_per_graph": self.glen, "timed_rotation_start": w0,
                "us_per_op_alone": {k: round(v, 3) for k, v in per_op.items()},
                "sum_of_ops_alone": round(sum(per_op.values()), 3),
                "alg_bytes": total, "GBps": round(total / (us * 1e3), 1),
                "frac_of_hbm_peak": round(total / (us * 1e3) / HBM_PEAK_GBPS, 4),
                "kqkv_splits": self.A.default_splits(self.W, self.H)}


def layer_bench(args) -> int:
    """--layer: us per attention layer, COLD, at both geometries and two windows (one JSON line)."""
    import torch
    res = {}
    for geom, name in (("ref", "ref_kv320_q8wkb"), ("baseline", "baseline_kv576_f32wkb")):
        res[name] = {}
        for n_kv in (4096, 32768):
            lay = Layer(geom, n_kv)
            res[name][str(n_kv)] = lay.record(args.steps, args.warmup)
            del lay
            torch.cuda.empty_cache()
    v = res["ref_kv320_q8wkb"]["32768"]["us_layer"]
    rec = {"metric": "us per MLA attention layer of one decode token (COLD)", "value": v, "unit": "us/layer",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": "q8_0/f16/f32", "data": "synthetic",
           "config": {"workload": "value: reference geometry (KV row 320, Q8_0 weights), 32,768-key window, "
                                  "KV-write -> WKB -> concat -> KQKV -> wv_b in one hipGraph of whole rotations"},
           "layers": res,
           "reference_rx9070": {"m4_ops_in_situ": "core -18.7 us/layer for WKB (engine/m1_session.h:155-158)",
                                "kvwrite_group_stock_us": 29.4, "wvb_stock_us": 16.6}}
    print(json.dumps(rec), flush=True)
    return 0


def cpu_run(inp, threads, runs):
    """The CPU oracle's full step (WKB + unfused kq / softmax / kqv): median seconds of `runs`
    after one warm-up (runs = 1: a single untimed-warm-up-free run), and the oracle output."""
    from oracle import oracle as orc
    if runs > 1:
        orc.mla_step(inp, threads=threads)
    ts = []
    ref = None
    for _ in range(runs):
        t = time.perf_counter()
        _, ref = orc.mla_step(inp, threads=threads)
        ts.append(time.perf_counter() - t)
    return statistics.median(ts), ref


def decode_timings(d, steps, warmup, reps, sweep):
    """Time one decode configuration: exactly `steps` steps after `warmup`, each kernel, WARM,
    optionally the split sweep, and the dominant kernel's roofline."""
    us_step, wall, w0 = d.run_steps(steps, warmup)
    k = d.per_kernel(reps)
    r = {"n_kv": d.W, "nt": d.inp.nt, "splits": d.S, "cache": "q8_0" if d.q8 else ("f16" if d.inp.kc_f16 else "f32"),
         "steps": steps, "warmup": warmup, "rotating_copies": d.n_rot, "steps_per_graph": d.glen,
         "timed_rotation_start": w0,
         "us_step": round(us_step, 3), "wall_s_timed": round(wall, 6),
         "us_wkb": round(k["wkb"], 3), "us_kqkv_op": round(k["kqkv"], 3),
         "kqkv_path": "one launch (flat kernel, in-kernel merge)" if d.flat else "split-K partial + PHASE merge",
         "us_kqkv_partial": round(k["partial"], 3), "us_phase_merge": round(k["merge"], 3),
         "alg_bytes_step": int(d.bytes_step),
         "cache_bytes_per_key": (d.DK // 32 * 34 if d.q8 else d.DK * d.es) + 4,     # cache row + mask
         "step_GBps": round(d.bytes_step / (us_step * 1e3), 1),
         "step_frac_of_hbm_peak": round(d.bytes_step / (us_step * 1e3) / HBM_PEAK_GBPS, 4),
         "partial_GBps": round(d.bytes_attn / (k["partial"] * 1e3), 1),
         "partial_frac_of_hbm_peak": round(d.bytes_attn / (k["partial"] * 1e3) / HBM_PEAK_GBPS, 4),
         "wkb_GBps": round(d.bytes_wkb / (k["wkb"] * 1e3), 1),
         "partial_kernel": partial_kernel_name(d.inp.kc_f16, d.W, d.S, d.q8),
         "partial_bytes_written": int(d.part.numel() * 4),
         "warm_us_step": round(d.warm_step(reps), 3)}
    if d.flat:
        r["roofline"] = {"kernel": f"kqkv_flat_kernel<{'f16' if d.inp.kc_f16 else 'f32'} cache>",
                         "alg_bytes_per_launch": int(d.bytes_attn), "us_per_launch": k["kqkv"],
                         "timing": "graph of back-to-back launches", "splits": (d.W + 31) // 32}
    else:
        r["roofline"] = {"kernel": partial_kernel_name(d.inp.kc_f16, d.W, d.S, d.q8), "alg_bytes_per_launch": int(d.bytes_attn),
                         "us_per_launch": k["partial"], "timing": "graph of back-to-back launches", "splits": d.S}
    if sweep:
        r["split_sweep"] = d.split_sweep(reps)
    return r


def decode_record(inp, args, steps, warmup, reps, sweep, cpu_runs, cpu_thr):
    """decode_timings of one config, the CPU oracle beside it and the error of one GPU step."""
    d = Decode(inp, args.splits)
    rec = decode_timings(d, steps, warmup, reps, sweep)
    rec["splits"] = rec.pop("roofline")["splits"]
    out = d.gpu_output()
    if cpu_runs:
        t, ref = cpu_run(inp, cpu_thr, cpu_runs)
        rec["cpu_ms"] = round(t * 1e3, 3)
        rec["cpu_runs"] = cpu_runs
        rec["cpu_threads"] = cpu_thr
        rec["err_vs_oracle"] = errors(out, ref)
    del d
    import torch
    torch.cuda.empty_cache()
    return rec


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the split-K decode path runs on a single "
              "MI355X); multi-GPU runs are not part of it.", file=sys.stderr)
        return 2
    import torch
    import aubier_amd as A
    from aubier_amd import inputs as I

    A.load_library()
    if args.ops:
        return ops_bench(args)
    if args.layer:
        return layer_bench(args)
    if args.batch:
        region = 32768 // args.batch
        inp = I.make_batch(args.batch, region, lens=[region] * args.batch)
        if args.cache == "q8":
            inp = I.with_q8_cache(inp)
    else:
        inp = I.make_config(args.config)
        if args.cache == "q8":
            inp = I.with_q8_cache(inp)
        if inp.nt > 1:
            rec = prefill_record(inp, args.steps, args.warmup, cpu=not args.no_cpu, cpu_thr=cpu_threads()["threads"])
            print(json.dumps(rec), flush=True)
            return 0
    if args.pmc_pass:
        return pmc_pass(inp, args)

    thr = cpu_threads()
    reps = 8
    d = Decode(inp, args.splits)
    t = decode_timings(d, args.steps, args.warmup, reps, sweep=not args.no_sweep)
    out = d.gpu_output()
    W, S, H = d.W, d.S, d.H
    us_step = t["us_step"]
    roof = t.pop("roofline")
    S = roof.pop("splits")
    extra = {k: v for k, v in t.items() if k not in ("n_kv", "nt", "splits", "cache", "steps", "warmup")}
    del d
    torch.cuda.empty_cache()

    # ---- CPU baseline: the restated unfused ggml graph on the host threads (rank 0, N=1) ----
    cpu = None
    if not args.no_cpu:
        t, ref = cpu_run(inp, thr["threads"], 5)
        t1, _ = cpu_run(inp, 1, 1)
        cpu = {"value": round(t * 1e6, 1), "unit": "us/step", "cores": thr["threads"], "kind": "port",
               "sample": f"config {args.config} full step (WKB + unfused kq/softmax/kqv) on the same inputs, "
                         f"median of 5 after 1 warm-up",
               "value_1thread": round(t1 * 1e6, 1), "host_cpus_visible": thr["host_cpus_visible"],
               "omp_num_threads": thr["omp_num_threads"]}
        extra["err_vs_oracle"] = errors(out, ref)

    # ---- every other BASELINE config, timed the same way (fills the results table) ----
    if not args.no_others and not args.batch and args.cache == "f16":
        others = {}
        for cfg in (1, 2, 4, 5):
            if cfg == args.config:
                continue
            ic = I.make_config(cfg)
            if ic.nt > 1:
                others[str(cfg)] = prefill_record(ic, 48, 8, cpu=not args.no_cpu, cpu_thr=thr["threads"], nested=True)
            else:
                others[str(cfg)] = decode_record(ic, args, steps=48, warmup=12, reps=4, sweep=False,
                                                 cpu_runs=0 if args.no_cpu else 5, cpu_thr=thr["threads"])
            del ic
        extra["configs"] = others

    # HBM bytes per launch of the partial kernel, from the committed rocprofv3 counter summary
    # (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the calibration copy's factor)
    traffic = None
    tf_path = TRAFFIC_FILES.get((args.config, args.cache))
    if tf_path is not None and tf_path.exists() and not args.batch:
        tr = json.loads(tf_path.read_text())
        if tr.get("config") == args.config and tr.get("splits") == S and tr.get("kernel") == roof["kernel"]:
            traffic = int(tr["traffic_bytes"])

    gbps = roof["alg_bytes_per_launch"] / (roof["us_per_launch"] * 1e3)
    step_desc = ("WKB + one-launch KQKV (32-key splits, merged in the kernel)" if extra["kqkv_path"].startswith("one")
                 else "WKB + split-K partial + PHASE merge")
    rec = {
        "metric": METRIC, "value": round(us_step, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1000.0, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16" if inp.kc_f16 else "f32", "data": "synthetic",
        "config": {"workload": (f"batch-of-{inp.nt} decode: {inp.nt} rows x 32 heads, each over its own "
                                f"{W // inp.nt}-cell region of one {W}-cell window, " if args.batch else
                                f"config {args.config}: MLA decode, 1 token x 32 heads, {W} keys, ") +
                               f"{'Q8_0 (ggml block_q8_0, 612 B/key)' if inp.kcache_q8 is not None else ('f16' if inp.kc_f16 else 'f32')} "
                               f"latent+rope cache [{W},576], W_kb f32 [32,512,128], "
                               f"{step_desc} (S={S}), COLD ({extra['rotating_copies']} rotating copies), hipGraph",
                   "n_kv": W, "n_head": H, "d_k": I.D_K, "d_v": I.D_V, "splits": S, "seeds": inp.seeds, "notes": inp.notes},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": roof["kernel"], "alg_bytes_per_launch": roof["alg_bytes_per_launch"],
                     "us_per_launch": round(roof["us_per_launch"], 3), "timing": roof["timing"]},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(rec), flush=True)
    return 0


def pmc_pass(inp, args) -> int:
    """The calibration kernel (a plain device copy of CAL_BYTES each way, torch's copy kernel),
    then one rotation of eager steps; rocprofv3 reports FETCH_SIZE / WRITE_SIZE per dispatch."""
    import torch
    d = Decode(inp, args.splits)
    src = torch.ones(CAL_BYTES // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for i in range(d.n_rot):
        d.step(i)
    torch.cuda.synchronize()
    print(f"pmc pass done: copy {CAL_BYTES} B x3, {d.n_rot} steps of config {args.config}, S={d.S}", flush=True)
    return 0


def prefill_record(inp, steps, warmup, cpu: bool, cpu_thr: int, nested: bool = False) -> dict:
    """Config 5 (chunked prefill, nt > 1): WKB -> KQKV through ggml_m4_kqkv, MFMA-bound, reported
    in TFLOP/s of exact causal work against the f16 dense MFMA peak.  Not the headline metric.
    Over an 8-bit cache (--cache q8) the op first writes the cache's f16 values into its workspace;
    its attention figure is then the whole op (copy + attention + merge)."""
    import torch
    import aubier_amd as A
    from aubier_amd import inputs as I
    dev = torch.device("cuda:0")
    H, DV, DK, T = I.N_HEAD, I.D_V, I.D_K, inp.nt
    q8 = inp.kcache_q8 is not None
    if q8:
        kc = A.Q8_0(torch.from_numpy(np.ascontiguousarray(inp.kcache_q8)).to(dev), DK)
    else:
        kc = torch.from_numpy(np.ascontiguousarray(inp.kcache)).to(dev)
    wkb_w = torch.from_numpy(inp.w_kb).to(dev)
    q = np.concatenate([inp.q_nope, inp.q_pe], axis=2).astype(np.float32)
    qd = torch.from_numpy(q).to(dev)
    qcur = torch.zeros((T, H, DK), dtype=torch.float32, device=dev)
    qcur[:, :, DV:] = qd[:, :, I.D_NOPE:]
    mask = torch.from_numpy(inp.mask).to(dev)
    out = torch.empty((H, T, DV), dtype=torch.float32, device=dev)
    need = A.kqkv_workspace_bytes(kc, qcur, out)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)

    def step():
        A.ggml_m4_wkb(wkb_w, qd[:, :, :I.D_NOPE], out=qcur[:, :, :DV])
        A.ggml_m4_kqkv(kc, qcur, mask, inp.kq_scale, out=out, workspace=ws)

    # a graph holds NG back-to-back calls, so that a graph launch's own overhead is spread over them
    NG = 4

    def time_fn(fn, reps):
        fn()
        torch.cuda.synchronize()
        gg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gg):
            for _ in range(NG):
                fn()
        gg.replay()
        torch.cuda.synchronize()
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record()
        for _ in range(reps):
            gg.replay()
        a1.record()
        torch.cuda.synchronize()
        return a0.elapsed_time(a1) * 1000.0 / (reps * NG)

    for _ in range(max(1, warmup)):
        step()
    torch.cuda.synchronize()
    reps = max(1, math.ceil(steps / NG))
    us = time_fn(step, reps)

    part = None
    n_split = max(1, need // (((H + 31) // 32) * T * A.ops.part_floats(DV, inp.kc_f16) * 4)) if need else 1
    if q8:
        n_split = None                       # the op's own split count, behind its f16 copy
    elif n_split > 1:
        part = torch.empty(((H + 31) // 32, T, n_split, A.ops.part_floats(DV, inp.kc_f16)), dtype=torch.float32, device=dev)
    # per kernel: 12 replays of a 4-launch graph (fewer read low right after another config's run)
    KR = 12
    us_wkb = time_fn(lambda: A.ggml_m4_wkb(wkb_w, qd[:, :, :I.D_NOPE], out=qcur[:, :, :DV]), KR)
    if part is not None:
        us_attn = time_fn(lambda: A.ggml_m4_kqkv_partial(kc, qcur, mask, inp.kq_scale, n_split, part=part), KR)
        us_merge = time_fn(lambda: A.ggml_m4_phase_merge(part, out=out), KR)
    else:
        us_attn = time_fn(lambda: A.ggml_m4_kqkv(kc, qcur, mask, inp.kq_scale, out=out, workspace=ws), KR)
        us_merge = None if q8 else 0.0
    step()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    live = (inp.mask == 0).sum(axis=1).astype(np.float64)          # keys visible to each token
    flop = float((2.0 * H * (DK + DV) * live).sum()) + 2.0 * H * DV * I.D_NOPE * T
    tf = flop / (us * 1e-6) / 1e12
    flop_attn = float((2.0 * H * (DK + DV) * live).sum())
    tf_attn = flop_attn / (us_attn * 1e-6) / 1e12
    cpu_rec, err = None, None
    if cpu:
        t, ref = cpu_run(inp, cpu_thr, 5)
        cpu_rec = {"value": round(t * 1e6, 1), "unit": "us/step", "cores": cpu_thr, "kind": "port",
                   "sample": "config 5 full step (WKB + unfused kq/softmax/kqv) on the same inputs, median of 5 after 1 warm-up"}
        err = errors(got, ref)
    if nested:
        return {"n_kv": inp.n_kv, "nt": T, "splits": n_split, "cache": "q8_0" if q8 else "f16", "steps": reps * NG, "warmup": warmup,
                "us_step": round(us, 2), "tflops_step": round(tf, 1), "frac_of_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                "us_wkb": round(us_wkb, 2), "us_kqkv_partial": round(us_attn, 2),
                "us_phase_merge": None if us_merge is None else round(us_merge, 2), "attention_tflops": round(tf_attn, 1), "attention_frac_of_mfma_peak": round(tf_attn / MFMA_F16_PEAK_TFLOPS, 4),
                "gflop_per_step": round(flop / 1e9, 2),
                "cpu_ms": round(cpu_rec["value"] / 1e3, 3) if cpu_rec else None, "cpu_threads": cpu_thr if cpu_rec else None,
                "err_vs_oracle": err}
    return {"metric": "MLA chunked prefill (config 5): us/step and TFLOP/s of exact causal work", "value": round(us, 2),
            "unit": "us/step", "n_gpus": 1, "steps": reps * NG, "warmup": warmup, "ms_per_step": round(us / 1000.0, 4),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"config 5: {T} tokens x {inp.n_kv} keys causal, 32 heads, "
                                   + ("Q8_0 cache (f16 copy in the workspace)" if q8 else "f16 cache"), "nt": T,
                       "n_kv": inp.n_kv},
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None, "gflop_per_step": round(flop / 1e9, 2),
                         "attention_kernel": {"us": round(us_attn, 2), "tflops": round(tf_attn, 1),
                                              "frac": round(tf_attn / MFMA_F16_PEAK_TFLOPS, 4), "splits": n_split}},
            "cpu_baseline": cpu_rec,
            "extra": {"us_wkb": round(us_wkb, 2), "us_kqkv_partial": round(us_attn, 2),
                      "us_phase_merge": None if us_merge is None else round(us_merge, 2),
                      "err_vs_oracle": err}}


def ops_bench(args) -> int:
    """The reference geometry's quantised ops (the shapes its builders assert: ggml.c:3405-3539),
    each COLD (weights rotated over more copies than the 256 MB MALL holds), graph-replayed, HIP
    events.  Algorithmic bytes: weights + activations + outputs (+ the f16 cache row for KV-write).
    Reference figures (RX 9070, m4-wkb.cu:11-12 and m4-phase.cu:8,31) are printed beside them."""
    import torch
    import aubier_amd as A
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(9100)

    def q8_blocks(rows, ne0, copies):
        nb = ne0 // 32
        b = np.empty((rows, nb, 34), dtype=np.uint8)
        b[:, :, :2] = (np.abs(rng.standard_normal((rows, nb))) * 0.01 + 0.001).astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
        b[:, :, 2:] = rng.integers(-127, 128, size=(rows, nb, 32)).astype(np.int8).view(np.uint8)
        t = torch.from_numpy(b.reshape(rows, nb * 34)).to(dev)
        return [t] + [t.clone() for _ in range(copies - 1)]

    def timed(fn, n):
        for i in range(2):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (reps * n)

    res = {}
    H = 32
    # WKB, Q8_0 W_kb [64, 256, 32] (0.53 MiB), q_nope with the 128-float head stride
    nrot = 600
    ws = q8_blocks(H * 256, 64, nrot)
    q = torch.from_numpy(rng.standard_normal((1, H, 128)).astype(np.float32) * 0.05).to(dev)
    out = torch.empty((1, H, 256), dtype=torch.float32, device=dev)
    us = timed(lambda i: A.ggml_m4_wkb(A.Q8_0(ws[i % nrot].view(H, 256, 68), 64), q[:, :, :64], out=out), nrot)
    by = H * 256 * 68 + H * 64 * 4 + H * 256 * 4
    res["wkb_q8_0"] = {"shape": "Q8_0 [64,256,32] x f32 [64,32,1] -> [256,32,1]", "us": round(us, 3), "bytes": by,
                       "GBps": round(by / (us * 1e3), 1), "reference_rx9070_us": 4.05}
    del ws
    # PHASE 1 wv_b, Q8_0 [256, 128, 32] (1.06 MiB)
    nrot = 300
    ws = q8_blocks(H * 128, 256, nrot)
    x = torch.from_numpy(rng.standard_normal((H, 1, 256)).astype(np.float32) * 0.05).to(dev)
    out = torch.empty((H, 1, 128), dtype=torch.float32, device=dev)
    us = timed(lambda i: A.ggml_m4_phase_wvb(A.Q8_0(ws[i % nrot].view(H, 128, 272), 256), x, out=out), nrot)
    by = H * 128 * 272 + H * 256 * 4 + H * 128 * 4
    res["phase1_wvb"] = {"shape": "Q8_0 [256,128,32] x f32 [256,1,32] -> [128,1,32]", "us": round(us, 3), "bytes": by,
                         "GBps": round(by / (us * 1e3), 1), "reference_rx9070_stock_us": 16.6}
    del ws
    # PHASE 0 KV-write, Q8_0 [4096, 320] (1.36 MiB), a 32,768-row cache
    nrot = 250
    ws = q8_blocks(320, 4096, nrot)
    cur = torch.from_numpy(rng.standard_normal(4096).astype(np.float32)).to(dev)
    nw = torch.ones(256, dtype=torch.float32, device=dev)
    kc = torch.zeros((32768, 320), dtype=torch.float16, device=dev)
    kidx = torch.tensor([12345], dtype=torch.int64, device=dev)
    pos = torch.tensor([12345], dtype=torch.int32, device=dev)
    rp = A.rope_params(freq_base=1e6, freq_scale=0.25, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
                       eps=1e-6, n_dims=64, n_ctx_orig=8192)
    out = torch.empty(320, dtype=torch.float32, device=dev)
    us = timed(lambda i: A.ggml_m4_phase_kvwrite(cur, A.Q8_0(ws[i % nrot], 4096), nw, kc, kidx, pos, rp, out=out), nrot)
    by = 320 * 128 * 34 + 4096 * 4 + 256 * 4 + 320 * 4 + 320 * 2
    res["phase0_kvwrite"] = {"shape": "Q8_0 [4096,320] gemv + norm + YaRN rope + f16 scatter (2 launches)",
                             "us": round(us, 3), "bytes": by, "GBps": round(by / (us * 1e3), 1),
                             "reference_rx9070_stock_us": 29.4}
    for v in res.values():
        v["frac_of_hbm_peak"] = round(v["GBps"] / HBM_PEAK_GBPS, 4)
    rec = {"metric": "reference-geometry quantised ops: us per launch (COLD) and achieved GB/s", "value": None,
           "unit": "us", "n_gpus": 1, "dtype": "q8_0/f32", "data": "synthetic", "ops": res,
           "note": "latency-bound launches of ~1 MB; the reference figures are per layer on an RX 9070"}
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

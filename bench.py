"""MLA decode attention benchmark on one MI355X (BASELINE.json metric: us per decode step plus
achieved HBM GB/s as a fraction of peak, at 32,768 keys).

    python bench.py [--steps K] [--warmup W] [--config 3] [--splits S] [--no-cpu]

One step = the MLA attention of one decode token: GGML_OP_M4_WKB (absorbed q_nope written into
the Qcur buffer) -> GGML_OP_M4_KQKV pass 1 (split-K partials) -> GGML_OP_M4_PHASE merge, through
the C ABI, on seeded synthetic inputs (aubier_amd.inputs).  The steps are captured in a hipGraph
(the way the engine runs them) and replayed; consecutive steps read different copies of the KV
cache and W_kb (12 copies > the 256 MB MALL), so every step streams from HBM (COLD).

Prints ONE JSON line.  `roofline` is for the dominant kernel (the split-K partial): algorithmic
bytes per launch (n_kv * (1152 cache + 4 mask) + Qcur) / its average duration, timed with HIP
events around a graph of back-to-back launches on the stream they run on.  `cpu_baseline` is the
CPU oracle (the restated unfused ggml graph) on all host cores, same inputs, median of 5.
"""
from __future__ import annotations

import argparse
import json
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
N_ROT = 12
CAL_BYTES = 256 << 20          # calibration copy size (each way) for the HBM traffic counters
TRAFFIC_FILES = {3: ROOT / "profiles" / "kqkv_decode_f16_cfg3_traffic.json",      # per decode config
                 4: ROOT / "profiles" / "kqkv_decode_long_cfg4_traffic.json"}


def partial_kernel_name(kc_f16: bool, n_kv: int, n_split: int) -> str:
    """The kernel the library launches for the split-K partial: an f16 cache takes the
    barrier-per-tile kernel for splits of at most 6 64-key tiles and the independent-wave kernel
    for longer ones (launch_kqkv_decode_f16); an f32 cache takes the VALU kernel."""
    if not kc_f16:
        return "kqkv_generic_kernel<f32 cache>"
    tiles_per_split = -(-(-(-n_kv // 64)) // n_split)
    return "kqkv_decode_f16_long_kernel<576,512>" if tiles_per_split > 6 else "kqkv_decode_f16_kernel<576,512>"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--splits", type=int, default=0, help="split count (0 = library default)")
    ap.add_argument("--batch", type=int, default=0,
                    help="batch-of-N decode: N rows, each over its own 32768/N-cell region of one window")
    ap.add_argument("--sweep", action="store_true", help="also time S in {64,128,192,256}")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--warm", action="store_true", help="also report WARM (one cache) timings")
    ap.add_argument("--ops", action="store_true",
                    help="time the reference-geometry quantised ops (Q8_0 WKB, PHASE wv_b, PHASE KV-write) instead")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="no timing: run the calibration copy and a few steps, for rocprofv3 --pmc")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the split-K decode path runs on a single "
              "MI355X); multi-GPU runs are not part of it.", file=sys.stderr)
        return 2
    import torch
    import aubier_amd as A
    from aubier_amd import inputs as I

    dev = torch.device("cuda:0")
    A.load_library()
    if args.ops:
        return ops_bench(args)
    if args.batch:
        region = 32768 // args.batch
        inp = I.make_batch(args.batch, region, lens=[region] * args.batch)
    else:
        inp = I.make_config(args.config)
        if inp.nt > 1:
            return prefill_bench(args, inp)
    H, DV, DK = I.N_HEAD, I.D_V, I.D_K
    W = inp.n_kv
    es = 2 if inp.kc_f16 else 4

    # ---- device buffers: N_ROT copies of the per-layer data (cache, W_kb, q) ----
    kc0 = torch.from_numpy(np.ascontiguousarray(inp.kcache)).to(dev)
    wkb0 = torch.from_numpy(inp.w_kb).to(dev)
    q = np.zeros((inp.nt, H, I.D_NOPE + I.D_ROPE), dtype=np.float32)
    q[:, :, :I.D_NOPE] = inp.q_nope
    q[:, :, I.D_NOPE:] = inp.q_pe
    q0 = torch.from_numpy(q).to(dev)
    mask = torch.from_numpy(inp.mask).to(dev)
    kcs = [kc0] + [kc0.clone() for _ in range(N_ROT - 1)]
    wkbs = [wkb0] + [wkb0.clone() for _ in range(N_ROT - 1)]
    qs = [q0] + [q0.clone() for _ in range(N_ROT - 1)]
    qcurs = []
    for i in range(N_ROT):
        qc = torch.zeros((inp.nt, H, DK), dtype=torch.float32, device=dev)
        qc[:, :, DV:] = qs[i][:, :, I.D_NOPE:]
        qcurs.append(qc)
    S = args.splits or A.default_splits(W, H, A.ops.TYPE_F16 if inp.kc_f16 else A.ops.TYPE_F32)
    part = torch.empty(((H + 31) // 32, inp.nt, S, A.ops.part_floats(DV)), dtype=torch.float32, device=dev)
    out = torch.empty((H, inp.nt, DV), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def wkb(i):
        A.ggml_m4_wkb(wkbs[i], qs[i][:, :, :I.D_NOPE], out=qcurs[i][:, :, :DV])

    def attn(i, part_=None, S_=None):
        A.ggml_m4_kqkv_partial(kcs[i], qcurs[i], mask, inp.kq_scale, S_ or S, part=part_ if part_ is not None else part)

    def merge(part_=None):
        A.ggml_m4_phase_merge(part_ if part_ is not None else part, out=out)

    def step(i):
        wkb(i)
        attn(i)
        merge()

    if args.pmc_pass:
        # the calibration kernel: a plain device copy of CAL_BYTES each way (torch's copy kernel),
        # then N_ROT eager steps; rocprofv3 reports FETCH_SIZE / WRITE_SIZE per dispatch of each
        src = torch.ones(CAL_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        for i in range(N_ROT):
            step(i)
        torch.cuda.synchronize()
        print(f"pmc pass done: copy {CAL_BYTES} B x3, {N_ROT} steps of config {args.config}, S={S}", flush=True)
        return 0

    def capture(fn, n):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(2):            # untimed eager warmup on the capture stream
                fn(i % N_ROT)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i % N_ROT)
        return g

    def time_graph(g, reps, per):
        """us per unit: replay g `reps` times (each replay = `per` units) between two events."""
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (reps * per)

    # ---- the timed region: K steps, graph-captured in blocks of N_ROT ----
    g_step = capture(step, N_ROT)
    reps = max(1, args.steps // N_ROT)
    K = reps * N_ROT
    for _ in range(max(1, args.warmup // N_ROT)):
        g_step.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        g_step.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us_step = e0.elapsed_time(e1) * 1000.0 / K

    # ---- per-kernel durations (graphs of back-to-back launches of one kernel, COLD) ----
    per_reps = max(4, reps)
    us_wkb = time_graph(capture(wkb, N_ROT), per_reps, N_ROT)
    us_attn = time_graph(capture(attn, N_ROT), per_reps, N_ROT)
    us_merge = time_graph(capture(lambda i: merge(), N_ROT), per_reps, N_ROT)

    bytes_attn = W * (DK * es + 4) + inp.nt * H * DK * 4              # cache + mask + Qcur
    bytes_wkb = H * DV * I.D_NOPE * 4 + inp.nt * H * I.D_NOPE * 4 + inp.nt * H * DV * 4
    bytes_step_alg = bytes_attn + inp.nt * H * DV * 4 + bytes_wkb     # + final output
    gbps_attn = bytes_attn / (us_attn * 1e3)
    gbps_step = bytes_step_alg / (us_step * 1e3)

    extra = {
        "us_wkb": round(us_wkb, 3), "us_kqkv_partial": round(us_attn, 3), "us_phase_merge": round(us_merge, 3),
        "step_GBps": round(gbps_step, 1), "step_frac_of_hbm_peak": round(gbps_step / HBM_PEAK_GBPS, 4),
        "wkb_GBps": round(bytes_wkb / (us_wkb * 1e3), 1),
        "partial_bytes": int(part.numel() * 4), "alg_bytes_step": int(bytes_step_alg),
        "wall_s_timed": round(wall, 3),
    }
    if args.sweep:
        sweep = {}
        for S_ in (64, 128, 192, 256):
            p_ = torch.empty(((H + 31) // 32, inp.nt, S_, A.ops.part_floats(DV)), dtype=torch.float32, device=dev)
            ua = time_graph(capture(lambda i, p_=p_, S_=S_: attn(i, p_, S_), N_ROT), per_reps, N_ROT)
            um = time_graph(capture(lambda i, p_=p_: merge(p_), N_ROT), per_reps, N_ROT)
            sweep[str(S_)] = {"us_partial": round(ua, 3), "us_merge": round(um, 3),
                              "partial_GBps": round(bytes_attn / (ua * 1e3), 1)}
        extra["split_sweep"] = sweep
    if args.warm:
        g_w = capture(lambda i: step(0), N_ROT)
        extra["warm_us_step"] = round(time_graph(g_w, per_reps, N_ROT), 3)

    # ---- CPU baseline: the restated unfused ggml graph on the host cores (rank 0, N=1) ----
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as orc
        nthr = min(os.cpu_count() or 1, 16)
        orc.mla_step(inp, threads=nthr)            # warm-up
        ts = []
        for _ in range(5):
            t = time.perf_counter()
            orc.mla_step(inp, threads=nthr)
            ts.append(time.perf_counter() - t)
        t1 = time.perf_counter()
        orc.mla_step(inp, threads=1)
        one = time.perf_counter() - t1
        cpu = {"value": round(statistics.median(ts) * 1e6, 1), "unit": "us/step", "cores": nthr, "kind": "port",
               "sample": f"config {args.config} full step (WKB + unfused kq/softmax/kqv), median of 5 after 1 warm-up",
               "value_1thread": round(one * 1e6, 1)}

    # HBM bytes per launch of the partial kernel, from the committed rocprofv3 counter summary
    # (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the calibration copy's factor)
    traffic = None
    tf_path = TRAFFIC_FILES.get(args.config)
    if tf_path is not None and tf_path.exists():
        tr = json.loads(tf_path.read_text())
        if tr.get("config") == args.config and tr.get("splits") == S:
            traffic = int(tr["traffic_bytes"])

    rec = {
        "metric": METRIC, "value": round(us_step, 3), "unit": "us/step", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1000.0, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16" if inp.kc_f16 else "f32", "data": "synthetic",
        "config": {"workload": (f"batch-of-{inp.nt} decode: {inp.nt} rows x 32 heads, each over its own "
                                f"{W // inp.nt}-cell region of one {W}-cell window, " if args.batch else
                                f"config {args.config}: MLA decode, 1 token x 32 heads, {W} keys, ") +
                               f"{'f16' if inp.kc_f16 else 'f32'} latent+rope cache [{W},576], W_kb f32 [32,512,128], "
                               f"split-K S={S} + PHASE merge, COLD ({N_ROT} rotating copies), hipGraph",
                   "n_kv": W, "n_head": H, "d_k": DK, "d_v": DV, "splits": S, "seeds": inp.seeds, "notes": inp.notes},
        "roofline": {"bound": "hbm", "achieved": round(gbps_attn, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps_attn / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": partial_kernel_name(inp.kc_f16, W, S), "alg_bytes_per_launch": int(bytes_attn),
                     "us_per_launch": round(us_attn, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(rec), flush=True)
    return 0


def prefill_bench(args, inp) -> int:
    """Config 5 (chunked prefill, nt > 1): WKB -> KQKV through ggml_m4_kqkv, MFMA-bound, reported
    in TFLOP/s of exact causal work against the f16 dense MFMA peak.  Not the headline metric."""
    import torch
    import aubier_amd as A
    from aubier_amd import inputs as I
    dev = torch.device("cuda:0")
    H, DV, DK, T = I.N_HEAD, I.D_V, I.D_K, inp.nt
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

    # a graph holds NG back-to-back calls, so that a graph launch's own overhead (~10 us, more than
    # the smaller kernels here) is spread over them
    NG = 4

    def time_fn(fn, reps=3):
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

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    reps = max(3, args.steps // (4 * NG))
    us = time_fn(step, reps)

    part = None
    n_split = max(1, need // (((H + 31) // 32) * T * A.ops.part_floats(DV) * 4)) if need else 1
    if n_split > 1:
        part = torch.empty(((H + 31) // 32, T, n_split, A.ops.part_floats(DV)), dtype=torch.float32, device=dev)
    us_wkb = time_fn(lambda: A.ggml_m4_wkb(wkb_w, qd[:, :, :I.D_NOPE], out=qcur[:, :, :DV]))
    if part is not None:
        us_attn = time_fn(lambda: A.ggml_m4_kqkv_partial(kc, qcur, mask, inp.kq_scale, n_split, part=part))
        us_merge = time_fn(lambda: A.ggml_m4_phase_merge(part, out=out))
    else:
        us_attn = time_fn(lambda: A.ggml_m4_kqkv(kc, qcur, mask, inp.kq_scale, out=out, workspace=ws))
        us_merge = 0.0
    live = (inp.mask == 0).sum(axis=1).astype(np.float64)          # keys visible to each token
    flop = float((2.0 * H * (DK + DV) * live).sum()) + 2.0 * H * DV * I.D_NOPE * T
    tf = flop / (us * 1e-6) / 1e12
    flop_attn = float((2.0 * H * (DK + DV) * live).sum())
    tf_attn = flop_attn / (us_attn * 1e-6) / 1e12
    rec = {"metric": "MLA chunked prefill (config 5): us/step and TFLOP/s of exact causal work", "value": round(us, 2),
           "unit": "us/step", "n_gpus": 1, "steps": reps * NG, "warmup": 3, "ms_per_step": round(us / 1000.0, 4),
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
           "config": {"workload": f"config 5: {T} tokens x {inp.n_kv} keys causal, 32 heads, f16 cache", "nt": T,
                      "n_kv": inp.n_kv},
           "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0, "unit": "TFLOP/s",
                        "frac": round(tf / 2500.0, 4), "traffic": None, "gflop_per_step": round(flop / 1e9, 2),
                        "attention_kernel": {"us": round(us_attn, 2), "tflops": round(tf_attn, 1),
                                             "frac": round(tf_attn / 2500.0, 4), "splits": n_split}},
           "cpu_baseline": None,
           "extra": {"us_wkb": round(us_wkb, 2), "us_kqkv_partial": round(us_attn, 2), "us_phase_merge": round(us_merge, 2)}}
    print(json.dumps(rec), flush=True)
    return 0


def ops_bench(args) -> int:
    """The reference geometry's quantised ops (the shapes its builders assert: ggml.c:3405-3539),
    each COLD (weights rotated over more copies than the 256 MB MALL holds), graph-replayed, HIP
    events.  Algorithmic bytes: weights + activations + outputs (+ the f16 cache row for KV-write).
    Reference figures (RX 9070, m4-wkb.cu:11-12 and m4-phase.cu:8,31) are printed beside them."""
    import torch
    import aubier_amd as A
    from aubier_amd import inputs as I
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

#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Workloads (hmoe.synth.CONFIGS):
  C4     (default) INT8 Qwen3-30B-A3B-shape block, 4096-token prefill,
         128 experts, top-8, Zipf(1.1)-skewed routing
  C3-1, C3-4, C3-16   decode shapes (1/4/16 tokens)
  M256   (not a BASELINE config) 256-token INT8 prefill of the C4 layer:
         mostly groups of at most 32 rows (with --split-k: the bounded
         split-K GEMM for those)
  C1, C2 FP32 64-expert blocks

One step = one MoE-block call (route -> permute -> INT8 SwiGLU experts:
integer-limb MFMA GEMMs at prefill, W8A32 GEMVs at decode -> combine) over a
batch already resident in HBM.  Prints ONE JSON line.

Timing: W warm-up steps; K steps timed (reported as
settle.ms_per_step_before); untimed steps until --settle-ms of GPU time have
passed; then the K timed steps whose time is the result.  A GPU that has
been idle runs its first few dozen back-to-back C4 steps about 10 % slower
than it does from then on for as long as the load lasts (its clock drops and
recovers under the continuous load); the result is the rate it keeps.

Roofline: the dominant kernel's algorithmic work per launch divided by its
average launch duration, measured with hipEvents recorded on the launch
stream at the block's stage boundaries over K further steps (the timed
steps themselves carry no events).
  prefill (C4): gate/up GEMM, ops = 2*T*k*2*H*I, bound = INT8 MFMA (5.0 POP/s)
  decode (C3):  gate/up GEMV, bytes = U*2*H*I + activations, bound = HBM 8 TB/s
The CPU baseline is the oracle's restatement of the reference CPU path
(single thread, reference loop order) timed on a bounded token sample.
The default C4 run also times the decode shapes C3-1 and C3-16 of the same
layer in child benches and reports them under "decode" (step time, the
layer's HBM fraction, the gate/up GEMV's roofline and, for C3-16, its HBM
bytes per launch); --no-decode skips them.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "hypermoe-engine_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_INT8_TOPS = 5000.0      # dense INT8 MFMA, TOP/s
PEAK_FP32_TFLOPS = 157.3
METRIC = "MoE-layer tokens/s (INT8, 128e top-8) + % of HBM / INT8-MFMA roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--settle-ms", type=float, default=60.0,
                    help="after the warm-up and a first timed pass of K steps, untimed steps "
                         "until this much GPU time has passed, then the K timed steps whose "
                         "time is the result (a GPU that has been idle runs its first few "
                         "dozen back-to-back prefill steps while its clock drops and "
                         "recovers; 0: no settling, the first pass is the result)")
    ap.add_argument("--workload", default="C4")
    ap.add_argument("--limbs-x", type=int, default=2, help="X (token row) digit planes")
    ap.add_argument("--limbs-z", type=int, default=3, help="Z (SiLU(G)*U row) digit planes")
    ap.add_argument("--cpu-sample", type=int, default=-1,
                    help="tokens timed on the CPU baseline (-1: per-workload default, 0: skip)")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--decode-graph", action="store_true",
                    help="C5: replay the decode step as one captured HIP graph instead of "
                         "launching its kernels")
    ap.add_argument("--graph", action="store_true",
                    help="replay one captured HIP graph of the block per step instead of "
                         "launching every step from the host")
    ap.add_argument("--split-k", action="store_true",
                    help="INT8 prefill: groups of at most 32 rows take the bounded split-K GEMM "
                         "(HM_EXEC_SPLIT_K) instead of the tile GEMMs' partial tiles")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc child runs that measure the dominant "
                         "kernel's HBM bytes per launch (roofline.traffic = null)")
    ap.add_argument("--no-decode", action="store_true",
                    help="C4: skip the decode legs (C3-1 and C3-16 child benches whose step "
                         "times and HBM fractions the line reports under \"decode\")")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="also run a plain device-to-device copy of this many MiB (3x) "
                         "before the timed region: the known-size kernel that calibrates "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


def log(msg, quiet=False):
    if not quiet:
        print(msg, file=sys.stderr, flush=True)


def pmc_traffic(workload: str, kernel_re: str, primary_re: str, limbs: tuple, quiet: bool):
    """HBM bytes per launch of the dominant stage: two rocprofv3 --pmc runs
    of a short child bench (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch),
    each scaled by what the same counter reads for a plain 256 MiB
    device-to-device copy recorded in the same child run.  The stage may be
    several kernels (kernel_re): their dispatches are summed and divided by
    the dispatch count of its first kernel (primary_re).  None when
    rocprofv3 is missing or a run fails."""
    import csv
    import re
    import shutil
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    copy_mib = 256
    got = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory(dir="/tmp") as d:
            cmd = [exe, "--pmc", counter, "--kernel-include-regex", f"{kernel_re}|copyBuffer",
                   "--output-format", "csv", "-d", d, "-o", "pmc", "--", sys.executable,
                   str(REPO / "bench.py"), "--workload", workload, "--steps", "2", "--warmup",
                   "1", "--settle-ms", "0", "--cpu-sample", "0", "--quiet", "--no-traffic",
                   "--no-decode", "--limbs-x", str(limbs[0]), "--limbs-z", str(limbs[1]),
                   "--copy-mb", str(copy_mib)]
            env = dict(os.environ, TMPDIR="/tmp")
            log(f"[bench] traffic: rocprofv3 --pmc {counter}", quiet)
            try:
                subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL,
                               stderr=subprocess.DEVNULL, timeout=240)
            except subprocess.TimeoutExpired:
                return None
            files = list(Path(d).rglob("*counter_collection.csv"))
            if not files:
                return None
            kern, copies, launches = [], [], 0
            with open(files[0]) as f:
                for r in csv.DictReader(f):
                    v = float(r["Counter_Value"])
                    if re.search(kernel_re, r["Kernel_Name"]):
                        kern.append(v)
                        launches += bool(re.search(primary_re, r["Kernel_Name"]))
                    elif "copyBuffer" in r["Kernel_Name"]:
                        copies.append(v)
            if not kern or not copies or not launches:
                return None
            calib = max(copies)  # the 256 MiB calibration copies are the largest
            got[counter] = (sum(kern) / launches, calib)
    fetch, fcal = got["FETCH_SIZE"]
    write, wcal = got["WRITE_SIZE"]
    copy_kib = copy_mib * 1024.0
    ff, wf = copy_kib / fcal, copy_kib / wcal
    return {"bytes": int((fetch * ff + write * wf) * 1024), "fetch_kib_raw": round(fetch, 1),
            "write_kib_raw": round(write, 1), "fetch_scale": round(ff, 4),
            "write_scale": round(wf, 4),
            "calibration": f"{copy_mib} MiB device copy: FETCH_SIZE {fcal:.0f} KiB, "
                           f"WRITE_SIZE {wcal:.0f} KiB"}


def pmc_mfma(workload: str, kernels: dict, limbs: tuple, quiet: bool):
    """Matrix-core utilisation of the prefill GEMMs from hardware counters:
    one rocprofv3 --pmc run of a short child bench with
    SQ_VALU_MFMA_BUSY_CYCLES (summed over the SIMDs), SQ_BUSY_CU_CYCLES
    (summed over the CUs) and SQ_INSTS_MFMA.  Per kernel (name -> regex):
    mfma_busy_frac = MFMA busy cycles / (4 SIMDs x CU busy cycles), averaged
    over its dispatches.  None when rocprofv3 is missing or the run fails."""
    import csv
    import re
    import shutil
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    counters = ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_MFMA"]
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = [exe, "--pmc", *counters, "--kernel-include-regex", "|".join(kernels.values()),
               "--output-format", "csv", "-d", d, "-o", "pmc", "--", sys.executable,
               str(REPO / "bench.py"), "--workload", workload, "--steps", "2", "--warmup", "1",
               "--settle-ms", "0", "--cpu-sample", "0", "--quiet", "--no-traffic", "--no-decode",
               "--limbs-x", str(limbs[0]),
               "--limbs-z", str(limbs[1])]
        log("[bench] counters: rocprofv3 --pmc " + " ".join(counters), quiet)
        try:
            subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"),
                           stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=240)
        except subprocess.TimeoutExpired:
            return None
        files = list(Path(d).rglob("*counter_collection.csv"))
        if not files:
            return None
        vals = {name: {c: [] for c in counters} for name in kernels}
        with open(files[0]) as f:
            for r in csv.DictReader(f):
                for name, rx in kernels.items():
                    if re.search(rx, r["Kernel_Name"]) and r["Counter_Name"] in counters:
                        vals[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
    out = {"counters": "SQ_VALU_MFMA_BUSY_CYCLES / (4 x SQ_BUSY_CU_CYCLES), per dispatch"}
    for name, v in vals.items():
        if not v["SQ_BUSY_CU_CYCLES"]:
            return None
        busy = sum(v["SQ_VALU_MFMA_BUSY_CYCLES"]) / len(v["SQ_VALU_MFMA_BUSY_CYCLES"])
        cu = sum(v["SQ_BUSY_CU_CYCLES"]) / len(v["SQ_BUSY_CU_CYCLES"])
        out[name] = {"mfma_busy_frac": round(busy / (4.0 * cu), 4),
                     "mfma_busy_cycles": busy, "busy_cu_cycles": cu,
                     "mfma_insts": sum(v["SQ_INSTS_MFMA"]) / max(1, len(v["SQ_INSTS_MFMA"]))}
    return out


def decode_legs(quiet: bool):
    """The decode shapes of the same layer (C3-1, C3-16: one and sixteen
    tokens, 128 experts, top-8, INT8), each timed by a child bench in this
    run: step time, tokens/s, the whole layer's algorithmic bytes over the
    step against HBM peak, and the gate/up stage's own roofline line (C3-16
    with its HBM bytes per launch from the rocprofv3 --pmc child runs).
    None for a leg whose child fails."""
    import subprocess
    legs = {}
    for wl, steps, traffic in (("C3-1", 400, False), ("C3-16", 200, True)):
        cmd = [sys.executable, str(REPO / "bench.py"), "--workload", wl, "--steps", str(steps),
               "--warmup", str(steps // 10), "--cpu-sample", "0", "--quiet", "--no-decode"]
        if not traffic:
            cmd.append("--no-traffic")
        log(f"[bench] decode leg {wl}", quiet)
        try:
            res = subprocess.run(cmd, cwd=str(REPO), stdout=subprocess.PIPE,
                                 stderr=subprocess.DEVNULL, text=True, timeout=420)
            d = json.loads(res.stdout.strip().splitlines()[-1])
        except Exception as ex:  # noqa: BLE001 -- the leg is reported as missing
            log(f"[bench] decode leg {wl} failed: {ex}", quiet)
            legs[wl] = None
            continue
        r = d["roofline"]
        legs[wl] = {"tokens": d["config"]["tokens"], "ms_per_step": d["ms_per_step"],
                    "tokens_per_s": d["value"], "unique_experts": d["config"]["unique_experts"],
                    "layer_hbm_frac": d["layer_roofline"]["hbm_frac"],
                    "layer_algorithmic_bytes": d["layer_roofline"]["algorithmic_bytes"],
                    "gate_up": {k: r.get(k) for k in ("kernel", "achieved", "peak", "unit",
                                                           "frac", "traffic", "launch_ms")},
                    "stages_ms": d["stages_ms"]}
    return legs


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every box in this build has one MI355X and the "
              "block runs on one GPU's share (across GPUs the experts would shard by "
              "expert, with an all-to-all of the grouped rows and outputs over RCCL). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from hmoe import capi, synth
    from hmoe.block import DeviceExpertLayer, MoEBlock

    cfg = synth.CONFIGS[args.workload]
    if cfg.layers > 1:
        return run_stack(args, cfg)
    T, H, E, I, k = cfg.tokens, cfg.hidden, cfg.experts, cfg.inter, cfg.top_k
    q = args.quiet
    log(f"[bench] workload {cfg.name}: T={T} H={H} E={E} I={I} k={k} int8={cfg.int8} "
        f"skew={cfg.skew} limbs=({args.limbs_x}, {args.limbs_z})", q)
    t0 = time.time()
    payload, scale, zp = synth.expert_layer(cfg.seed, 0, E, H, I, cfg.int8,
                                            threads=min(16, os.cpu_count() or 1))
    # Decode-size steps rotate through a pool of distinct token batches so
    # that consecutive steps select different experts: the weights a step
    # streams are not the ones the previous step left in the 256 MB
    # Infinity Cache.  A prefill batch already touches every expert.
    pool = 1 if T >= 256 else 16
    raw = synth.raw_hidden(cfg.seed, T * pool, H)
    w = synth.router_weights(cfg.seed, 0, H, E)
    torch.cuda.set_device(0)
    lib = capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    # hidden = RMSNorm(N(0,1)) on the device (bit-exact with the reference)
    d_raw = torch.from_numpy(raw).cuda()
    gamma = torch.ones(H, dtype=torch.float32, device="cuda")
    d_h = torch.empty_like(d_raw)
    capi.call("hm_rmsnorm", d_raw.data_ptr(), gamma.data_ptr(), d_h.data_ptr(), T * pool, H, 1e-6,
              stream)
    batches = [d_h[i * T:(i + 1) * T] for i in range(pool)]
    if cfg.skew:
        bias = synth.zipf_bias(cfg.seed, E)
        d_h[:, -1] = 1.0
        w[-1, :] = bias
    d_w = torch.from_numpy(w).cuda()
    layer = DeviceExpertLayer(payload, scale, zp, H, I)
    block = MoEBlock(layer, k, limbs_x=args.limbs_x, limbs_z=args.limbs_z)
    if args.split_k:
        block.flags |= capi.HM_EXEC_SPLIT_K
    torch.cuda.synchronize()
    log(f"[bench] setup {time.time() - t0:.1f}s", q)

    # events: per step HM_BLOCK_EVENTS stage marks + overall start/stop
    def new_event():
        h = C.c_void_p()
        capi.call("hm_event_create", C.byref(h))
        return h.value

    stage_ev = [[new_event() for _ in range(capi.HM_BLOCK_EVENTS)] for _ in range(args.steps)]
    ev_start, ev_stop = new_event(), new_event()

    if args.copy_mb > 0:
        src = torch.empty(args.copy_mb << 20, dtype=torch.uint8, device="cuda")
        src.fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            capi.call("hm_memcpy_d2d", dst.data_ptr(), src.data_ptr(), src.numel(), stream)
        torch.cuda.synchronize()
        del src, dst

    for i in range(max(args.warmup, pool)):
        block.launch(batches[i % pool], d_w)
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done", q)

    # Optionally one step captured as a HIP graph (the block's kernels only;
    # no memset or copy nodes) and replayed; the replayed result must equal
    # the eager one.
    # (one graph per pool batch).
    graph = None
    if args.graph:
        try:
            graph = []
            for b in batches:
                ref_out = block.launch(b, d_w)["out"].clone()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    block.launch(b, d_w)
                for _ in range(2):
                    g.replay()
                    torch.cuda.synchronize()
                    if not torch.equal(block._io_bufs["out"], ref_out):
                        raise RuntimeError("graph replay differs from the eager launch")
                graph.append(g)
        except Exception as ex:  # noqa: BLE001 -- report and time eagerly
            log(f"[bench] graph capture unavailable ({ex}); timing eager launches", q)
            graph = None
        torch.cuda.synchronize()

    ms = C.c_float()

    def timed(n, first=0):
        # n steps between two events, nothing else on the stream
        torch.cuda.synchronize()
        capi.call("hm_event_record", ev_start, stream)
        for i in range(first, first + n):
            if graph is not None:
                graph[i % pool].replay()
            else:
                block.launch(batches[i % pool], d_w)
        capi.call("hm_event_record", ev_stop, stream)
        torch.cuda.synchronize()
        capi.call("hm_event_elapsed_ms", C.byref(ms), ev_start, ev_stop)
        return ms.value

    # The first K steps after the warm-up, timed and reported; then the
    # clock settles under the continuous load (untimed steps until
    # --settle-ms of GPU time have passed) and the timed region proper: K
    # steps whose time is the result.
    first_ms = timed(args.steps)
    settle_steps, settle_ms = 0, 0.0
    while settle_ms < args.settle_ms:
        n = max(1, min(200, int((args.settle_ms - settle_ms) / max(first_ms / args.steps, 1e-3)) + 1))
        settle_ms += timed(n, settle_steps)
        settle_steps += n
    total_ms = timed(args.steps) if settle_steps else first_ms
    ms_per_step = total_ms / args.steps
    # a second pass with the stage events recorded inside every step: the
    # per-stage times and the dominant kernel's launch duration
    for i in range(args.steps):
        block.launch(batches[i % pool], d_w, events=stage_ev[i])
    torch.cuda.synchronize()
    names = ["route", "permute", "quantize", "gate_up", "down", "combine"]
    stage = {n: 0.0 for n in names}
    for i in range(args.steps):
        for j, n in enumerate(names):
            capi.call("hm_event_elapsed_ms", C.byref(ms), stage_ev[i][j], stage_ev[i][j + 1])
            stage[n] += ms.value / args.steps
    log(f"[bench] timed {args.steps} steps: {ms_per_step:.4f} ms/step", q)

    # one checked call: routing stats + parity of a token sample
    # distinct experts per step, averaged over the pool (before the checked
    # call: each call reuses the block's output buffer)
    unique = float(np.mean([int((block.execute_batch(b, d_w).counts > 0).sum())
                            for b in batches]))
    res = block.execute_batch(batches[0], d_w)
    counts = res.counts
    h_host = batches[0].cpu().numpy()
    out = res.output.cpu().numpy()
    tokens_per_s = T / (ms_per_step / 1e3)

    gemv = cfg.int8 and T <= capi.HM_GEMV_MAX_TOKENS and T * k <= capi.HM_GEMV_MAX_PAIRS
    if gemv:
        # W8A32 GEMV: gate+up weights of the selected experts, gathered FP32
        # activation rows in, FP32 Z rows out
        gu_ops = 2 * T * k * 2 * H * I
        dn_ops = 2 * T * k * H * I
        gu_bytes = unique * 2 * H * I + T * k * H * 4 + T * k * I * 4
    elif cfg.int8:
        gu_ops = 2 * T * k * 2 * H * I
        dn_ops = 2 * T * k * H * I
        # X digit planes in, SiLU(G)*U floats out (their Z digits are the
        # next launch's work)
        gu_bytes = unique * 2 * H * I + T * H * args.limbs_x + T * k * I * args.limbs_z
    else:
        gu_ops = 2 * T * k * 2 * H * I
        dn_ops = 2 * T * k * H * I
        gu_bytes = unique * 2 * H * I * 4 + T * H * 4 + T * k * I * 4
    prefill = T >= 256
    gu_s = stage["gate_up"] / 1e3
    if prefill:
        achieved = gu_ops / gu_s / 1e12
        peak = PEAK_INT8_TOPS if cfg.int8 else PEAK_FP32_TFLOPS
        roof = {"bound": "mfma",
                "kernel": ("gate/up stage: ring_gemm_kernel<Lx, false> (G, U) + "
                           "limb_swiglu_quantize_vec_kernel<Lz, I/256> (SiLU(G)*U, Z digits)"
                           if cfg.int8 else "expert_f32_mfma_kernel<true>"),
                "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": None,
                "work_per_launch": gu_ops, "launch_ms": round(stage["gate_up"], 5),
                "hw_mfma_frac_with_limbs": round(achieved * (args.limbs_x if cfg.int8 else 1) / peak, 4)}
    else:
        achieved = gu_bytes / gu_s / 1e9
        roof = {"bound": "hbm",
                "kernel": ("gate/up GEMV: select_gateup_kernel<EPL, LJ> (one token: the select "
                           "and the 8-column slices in one launch), gateup_slice_kernel<NG, LJ> "
                           "(two tokens) or gemv_kernel<true, 1> (more)" if gemv else
                           "gate/up stage: ring_gemm_kernel<Lx, false> + "
                           "limb_swiglu_quantize_vec_kernel<Lz, I/256>" if cfg.int8
                           else "gate/up GEMV: gemv_f32_kernel<true, CW, MJ>" if T <= 16
                           else "expert_f32_mfma_kernel<true>"),
                "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                "work_per_launch": gu_bytes, "launch_ms": round(stage["gate_up"], 5)}
    if not args.no_traffic:
        if gemv:
            kre = prim = "select_gateup_kernel|gateup_slice_kernel|gemv_kernel<true"
        elif cfg.int8:
            kre, prim = ("ring_gemm_kernel<[0-9], false>|limb_swiglu_quantize",
                         "ring_gemm_kernel<[0-9], false>")
        else:
            kre = prim = "gemv_f32_kernel<true|expert_f32_mfma_kernel<true>"
        tr = pmc_traffic(cfg.name, kre, prim, (args.limbs_x, args.limbs_z), q)
        if tr is not None:
            roof["traffic"] = tr.pop("bytes")
            roof["traffic_detail"] = tr
        if prefill and cfg.int8:
            hw = pmc_mfma(cfg.name, {"gate_up": "ring_gemm_kernel<[0-9], false>",
                                     "down": "ring_gemm_kernel<[0-9], true>|limb_gemm_kernel"},
                          (args.limbs_x, args.limbs_z), q)
            if hw is not None:
                roof["hw_mfma"] = hw
    layer_bytes = synth.algorithmic_bytes(cfg, unique)
    layer_ops = synth.algorithmic_ops(cfg)
    layer = {"hbm_frac": round(layer_bytes / (ms_per_step / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
             "mfma_frac": round(layer_ops / (ms_per_step / 1e3) / 1e12 /
                                (PEAK_INT8_TOPS if cfg.int8 else PEAK_FP32_TFLOPS), 4),
             "algorithmic_bytes": layer_bytes, "algorithmic_ops": layer_ops}

    cpu = None
    sample = args.cpu_sample
    if sample < 0:
        sample = min(T, 160 if cfg.int8 else 32)
    parity = None
    if sample > 0:
        sys.path.insert(0, str(REPO / "oracle"))
        import hm_oracle as O
        hs = np.ascontiguousarray(h_host[:sample])
        # repeat the bounded sample until about 10 s of CPU work is timed
        t1 = time.time()
        runs = 0
        while True:
            rout, rids, _ = O.moe_block(payload, scale, zp, hs, w, k, I)
            runs += 1
            if time.time() - t1 >= 10.0:
                break
        dt = time.time() - t1
        cpu = {"value": round(sample * runs / dt, 3), "unit": "tokens/s", "cores": 1,
               "kind": "port",
               "sample": f"first {sample} of the {T} tokens of {cfg.name} (same weights and "
                         f"router) x {runs} runs, oracle restatement of the reference CPU path "
                         f"(MoERuntime CPU branch, single thread, -O3 -ffp-contract=off), "
                         f"{dt:.1f}s on a host with {os.cpu_count()} cores"}
        ids_ok = bool(np.array_equal(res.ids[:sample], rids))
        d = np.abs(out[:sample].astype(np.float64) - rout)
        parity = {"tokens_checked": sample, "ids_bitexact": ids_ok,
                  "normwise_vs_reference": float(d.max() / max(np.abs(rout).max(), 1e-30)),
                  "compare_1e-4": bool(np.all(d <= 1e-4 + 1e-4 * np.abs(rout)))}
        log(f"[bench] cpu baseline {cpu['value']} tokens/s; parity {parity}", q)

    decode = None
    if cfg.name == "C4" and not args.no_decode:
        decode = decode_legs(q)

    line = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "settle": {"steps": settle_steps, "gpu_ms": round(settle_ms, 2),
                   "ms_per_step_before": round(first_ms / args.steps, 5)},
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8" if cfg.int8 else "fp32", "data": "synthetic",
        "config": {"workload": cfg.name, "tokens": T, "hidden": H, "experts": E,
                   "intermediate": I, "top_k": k, "weights": "int8" if cfg.int8 else "fp32",
                   "skewed_routing": cfg.skew,
                   "limbs": [args.limbs_x, args.limbs_z] if cfg.int8 else None,
                   "unique_experts": unique, "max_expert_rows": int(counts.max()),
                   "input_batches": pool},
        "launch": "hip_graph_replay" if graph is not None else "eager",
        "roofline": roof, "layer_roofline": layer,
        "stages_ms": {n: round(v, 5) for n, v in stage.items()},
        "cpu_baseline": cpu, "parity": parity,
    }
    if decode is not None:
        line["decode"] = decode
    print(json.dumps(line), flush=True)


def run_stack(args, cfg):
    """C5: the 48-layer stack (RMSNorm + MoE block + residual per layer, all
    experts resident): a `tokens`-token prefill, then DECODE_STEPS single-token
    decode steps, each step's output feeding the next (the decode step is
    captured once as a HIP graph and replayed).  One bench step = the whole
    job; `value` = (prefill tokens + decode steps) / job time."""
    import numpy as np
    import torch
    from hmoe import synth
    from hmoe.stack import build_stack
    decode_steps = 128
    q = args.quiet
    T, H, E, I, k = cfg.tokens, cfg.hidden, cfg.experts, cfg.inter, cfg.top_k
    log(f"[bench] workload {cfg.name}: {cfg.layers} layers, prefill T={T}, {decode_steps} decode "
        f"steps, H={H} E={E} I={I} k={k} limbs=({args.limbs_x}, {args.limbs_z})", q)
    torch.cuda.set_device(0)
    t0 = time.time()
    stack = build_stack(cfg, limbs_x=args.limbs_x, limbs_z=args.limbs_z,
                        log=lambda l: log(f"[bench] layer {l + 1}/{cfg.layers} resident "
                                          f"({time.time() - t0:.0f}s)", q or (l + 1) % 8))
    resident = sum(l.packed.numel() for l in stack.layers)
    h_prefill = torch.from_numpy(synth.raw_hidden(cfg.seed, T, H)).cuda()
    h_tok = torch.from_numpy(synth.raw_hidden(cfg.seed + 1, 1, H)).cuda()
    torch.cuda.synchronize()
    log(f"[bench] setup {time.time() - t0:.1f}s, {resident / 2**30:.1f} GiB of experts resident", q)

    # the decode step as a graph: static input -> stack -> copy back into the input
    static_in = h_tok.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        stack.launch(static_in)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = stack.launch(static_in)
            static_in.copy_(out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # the prefill needs its own buffers (the stack re-plans per token count)
    prefill_stack = build_prefill_view(stack)

    def decode_step():
        if args.decode_graph:
            g.replay()
        else:
            static_in.copy_(stack.launch(static_in))

    def job():
        prefill_stack.launch(h_prefill)
        static_in.copy_(h_tok)
        for _ in range(decode_steps):
            decode_step()

    for _ in range(args.warmup):
        job()
    torch.cuda.synchronize()
    stack.check_status()
    prefill_stack.check_status()
    log(f"[bench] warmup {args.warmup} done", q)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    torch.cuda.synchronize()
    ev[0].record()
    for _ in range(args.steps):
        prefill_stack.launch(h_prefill)
    ev[1].record()
    for _ in range(args.steps):
        static_in.copy_(h_tok)
        for _ in range(decode_steps):
            decode_step()
    ev[2].record()
    torch.cuda.synchronize()
    prefill_ms = ev[0].elapsed_time(ev[1]) / args.steps
    decode_ms = ev[1].elapsed_time(ev[2]) / args.steps
    job_ms = prefill_ms + decode_ms
    stack.check_status()
    prefill_stack.check_status()
    # per-layer times from one eager pass of each shape with events between layers
    lev = [torch.cuda.Event(enable_timing=True) for _ in range(cfg.layers + 1)]
    prefill_stack.launch(h_prefill, events=lev)
    torch.cuda.synchronize()
    per_prefill = [lev[i].elapsed_time(lev[i + 1]) for i in range(cfg.layers)]
    stack.launch(h_tok.clone(), events=lev)
    torch.cuda.synchronize()
    per_decode = [lev[i].elapsed_time(lev[i + 1]) for i in range(cfg.layers)]
    log(f"[bench] prefill {prefill_ms:.3f} ms, {decode_steps} decode steps {decode_ms:.3f} ms", q)
    tokens = T + decode_steps
    line = {
        "metric": METRIC, "value": round(tokens / (job_ms / 1e3), 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(job_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": cfg.name, "layers": cfg.layers, "prefill_tokens": T,
                   "decode_steps": decode_steps, "hidden": H, "experts": E, "intermediate": I,
                   "top_k": k, "weights": "int8", "limbs": [args.limbs_x, args.limbs_z],
                   "experts_resident_bytes": int(resident)},
        "launch": ("prefill eager, decode step as one HIP graph (all layers) replayed"
                   if args.decode_graph else "prefill and decode steps eager"),
        "prefill_ms": round(prefill_ms, 4),
        "prefill_tokens_per_s": round(T / (prefill_ms / 1e3), 1),
        "decode_ms_per_token": round(decode_ms / decode_steps, 5),
        "decode_tokens_per_s": round(decode_steps / (decode_ms / 1e3), 1),
        "per_layer_ms": {"prefill_mean": round(float(np.mean(per_prefill)), 5),
                         "prefill_max": round(float(np.max(per_prefill)), 5),
                         "decode_mean": round(float(np.mean(per_decode)), 5),
                         "decode_max": round(float(np.max(per_decode)), 5)},
        "roofline": None, "cpu_baseline": None,
        "note": "per-layer rooflines and the CPU baseline are reported by the single-layer "
                "workloads (C3-1 decode, C4 prefill)",
    }
    print(json.dumps(line), flush=True)


def build_prefill_view(stack):
    """A second executor over the same resident layers (its own buffers, so
    the captured decode step's buffers stay untouched)."""
    from hmoe.stack import MoEStack
    return MoEStack(stack.layers, stack.router_w, stack.top_k, eps=stack.eps,
                    limbs_x=stack.limbs_x, limbs_z=stack.limbs_z, flags=stack.flags)


if __name__ == "__main__":
    main()

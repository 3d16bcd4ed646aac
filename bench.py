"""Benchmark of the quantized-weight hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu]
    python bench.py --copy-calibration
    python bench.py --write-traffic DIR   (DIR: rocprofv3 --pmc csv output, see below)

Headline (the JSON line's "value"): Q8_0 decode GEMV y[14336] = W[14336 x 4096]
x[4096], batch 1 -- packed-weight GB/s -- with exact bf16 weights (the
default product). The same line carries the other
workloads under "workloads": Q4_0 GEMV (14336 x 4096), the Q4_0 small-batch
product at m = 4 (same matrix), Q4_0 -> bf16 dequant (4096 x 4096), Q6_K GEMV
and Q6_K -> bf16 dequant (4096 x 14336), Q4_0 dequant-GEMM (M = 512, N = K = 4096), the Q4_0 MoE
grouped GEMM (128 experts, 64 tokens, top-8) and its gate_up stage fused with
SwiGLU, and the Q8_0 GEMV in the named relaxed mode (gemv_relaxed_q8_0).

Measurement
  - Inputs are synthetic and seeded, converted to the planar layout and
    resident in HBM before timing. Every workload cycles through enough
    copies of its weights to exceed the 256 MB Infinity Cache twice over, so
    successive launches read HBM, not the last-level cache.
  - A "step" is one launch of the workload's kernel(s). W warm-up steps, then
    K steps launched back to back and timed by one HIP event pair on the
    launch stream, between two device synchronizations. The host issues the
    K launches while an untimed pre-roll kernel (a bounded device spin, sized
    from the host's measured issue time) keeps the GPU busy, so the timed
    window holds the K steps and not the host's launch latency; a run whose
    start event completed before the last launch was issued is repeated with
    a longer pre-roll. "ms_per_step" is the window / K, "value" is K steps of
    algorithmic work over it (whole-job throughput, inputs resident in HBM),
    and "roofline.achieved" is the algorithmic bytes (or FLOPs) of one launch
    over the mean step. One untimed pre-rolled run of K steps precedes the
    timed one. "issue_us_per_step" is the host's time to issue one step
    (measured over K untimed launches), which the pre-roll hides.
  - "roofline.traffic" is the HBM bytes one launch of the workload's kernel
    moves, from rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE runs of this
    script, each scaled by the factor that makes a plain 256 MiB device copy
    (--copy-calibration) read and write 256 MiB; the scaled figures are kept
    in profiles/traffic.json (null when that file is absent). --write-traffic
    DIR rebuilds that file from DIR/{bench,copy}_{FETCH,WRITE}_SIZE/
    p_counter_collection.csv (rocprofv3 --pmc X --output-format csv -o p
    over this script, and over this script with --copy-calibration).
  - "cpu_baseline" (the headline's, and one in each of the Q8_0 and Q6_K GEMV,
    Q4_0 and Q6_K dequant, Q4_0 GEMM and Q4_0 MoE workloads):
    oracle/cpu_baseline.c over the same
    canonical tensors -- the reference's CPU semantics, vectorized (AVX-512 /
    AVX2 clones picked at load) and spread over min(16, usable) host threads --
    repeated for --cpu-seconds split across the legs; each records nproc,
    the usable CPUs, OMP_NUM_THREADS and the CPU model.
  - "step_us_replays": p10 / p50 / p90 of the step time over ten further
    timed runs of K steps, each behind its own pre-roll (not part of "value").
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA
LLC_BYTES = 256 << 20        # Infinity Cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default=None, help="run one workload (for profiling)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--write-traffic", metavar="DIR", default=None,
                    help="rebuild profiles/traffic.json from rocprofv3 --pmc csv output in DIR")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run five 256 MiB device-to-device copies (known-size reference for HBM counters)")
    return ap.parse_args()


def copies_for(bytes_per_step):
    return max(2, int(np.ceil(2 * LLC_BYTES / bytes_per_step)))


class Timer:
    """W eager warm-up launches, then K launches timed back to back.

    Before each timed run the device is synchronized and an untimed pre-roll
    (torch.cuda._sleep, a bounded spin) is queued; the start event, the K
    launches and the end event follow while it runs, so the event window
    holds the K steps and none of the host's issue time. The pre-roll lasts
    twice the host's measured issue time for K launches plus 0.2 ms; if the
    start event has already completed when the last launch is issued, the
    run is repeated with a pre-roll twice as long, and the workload's later
    runs keep that length. One untimed run of the
    same kind comes first (clocks settle after the spin), then the timed
    one. Returns (host issue seconds for K launches, event seconds) of the
    timed run; "spread" holds the per-step time of ten further runs."""

    def __init__(self, torch, replays=10):
        self.torch = torch
        self.replays = replays
        self.spread = []
        self.preroll = 0.0
        self.late = False  # the last run's window still held host issue time
        self.timed_late = False  # the same, for the timed run
        self._cps = None

    def _cycles_per_s(self):
        """Rate of the pre-roll's spin counter (measured once)."""
        if self._cps is None:
            torch = self.torch
            torch.cuda._sleep(1000)
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            torch.cuda._sleep(2_000_000)
            b.record()
            torch.cuda.synchronize()
            self._cps = 2_000_000 / max(a.elapsed_time(b) * 1e-3, 1e-6)
        return self._cps

    def _timed(self, launch, steps, preroll_s):
        torch = self.torch
        stream = torch.cuda.current_stream()
        for _ in range(4):
            torch.cuda.synchronize()
            torch.cuda._sleep(int(preroll_s * self._cycles_per_s()))
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(stream)
            t0 = time.perf_counter()
            for i in range(steps):
                launch(i)
            end.record(stream)
            late = start.query()  # the GPU reached the window before the last launch was issued
            issue = time.perf_counter() - t0
            torch.cuda.synchronize()
            if not late:
                break
            preroll_s *= 2
        self.preroll = preroll_s  # later runs start from the length that sufficed
        self.late = late
        return issue, start.elapsed_time(end) * 1e-3

    def run(self, launch, steps, warmup):
        torch = self.torch
        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()  # the host's issue time for K launches, untimed on the device
        for i in range(steps):
            launch(i)
        issue = time.perf_counter() - t0
        torch.cuda.synchronize()
        self.preroll = min(0.05, 2.0 * issue + 2e-4)
        self._timed(launch, steps, self.preroll)  # untimed: the same sequence once, clocks settling
        _, ev = self._timed(launch, steps, self.preroll)
        self.timed_late = self.late
        self.spread = [self._timed(launch, steps, self.preroll)[1] / steps for _ in range(self.replays)]
        return issue, ev


def traffic_table():
    """workload name -> scaled HBM bytes per launch, from profiles/traffic.json."""
    p = ROOT / "profiles" / "traffic.json"
    try:
        kernels = json.loads(p.read_text()).get("kernels", {})
    except (OSError, ValueError):
        return {}
    return {name: e.get("traffic_bytes") for name, e in kernels.items()}


# workload -> (kernel-name fragments whose dispatches make one step, algorithmic
# bytes of one step or None)
TRAFFIC_KERNELS = {
    "gemv_q8_0": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<8>,"], 14336 * 4096 // 32 * 34 + 4096 * 2 + 14336 * 2),
    "gemv_q6_k": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<14>,"], 4096 * 14336 // 256 * 210 + 14336 * 2 + 4096 * 2),
    "gemv_q4_0": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<2>,"], 14336 * 4096 // 32 * 18 + 4096 * 2 + 14336 * 2),
    "gemv_q4_k": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<12>,"], 14336 * 4096 // 256 * 144 + 4096 * 2 + 14336 * 2),
    "gemv_q5_k": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<13>,"], 14336 * 4096 // 256 * 176 + 4096 * 2 + 14336 * 2),
    "gemv_iq4_nl": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<20>,"], 14336 * 4096 // 32 * 18 + 4096 * 2 + 14336 * 2),
    "gemv_iq4_xs": (["gemv_exact_kernel<spiral::(anonymousnamespace)::Exact<23>,"], 14336 * 4096 // 256 * 136 + 4096 * 2 + 14336 * 2),
    "gemv_relaxed_q8_0": (["gemv_kernel<spiral::(anonymousnamespace)::Fmt<8>,"],
                          14336 * 4096 // 32 * 34 + 4096 * 2 + 14336 * 2),
    "mul_mat_q4_0_m4": (["skinny_kernel<2,"], 14336 * 4096 // 32 * 18 + 4 * 4096 * 2 + 4 * 14336 * 2),
    "dequant_q4_0": (["dequant_kernel<2>"], 4096 * 4096 // 32 * 18 + 4096 * 4096 * 2),
    "dequant_q6_k": (["dequant_kernel<14>"], 4096 * 14336 // 256 * 210 + 4096 * 14336 * 2),
    "gemm_q4_0": (["pack_x_kernel", "gemm_kernel<2,"], 4096 * 4096 // 32 * 18 + 2 * (512 * 4096 * 2)),
    "moe_q4_0": (["moe_stream_kernel<2,false,false,1,8>"], None),
    "moe_gate_up_swiglu_q4_0": (["moe_stream_kernel<2,false,true,1,8>"], None),
    # prefill (64 pairs an expert: the streaming form): gate_up in passes of 32 tokens, down in passes of 64
    "moe_prefill_q4_0": (["moe_stream_kernel<2,false,false,2,12>", "moe_stream_kernel<2,false,false,4,12>"], None),
}


def write_traffic(d):
    """Scaled HBM bytes per step from rocprofv3 FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch). Each counter is scaled so that the 256 MiB calibration copy
    reads it as 256 MiB."""
    import csv
    from collections import defaultdict
    d = Path(d)

    def per_kernel(sub):
        acc = defaultdict(list)
        with open(d / sub / "p_counter_collection.csv") as f:
            for r in csv.DictReader(f):
                acc[r["Kernel_Name"].replace(" ", "")].append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in acc.items()}

    def pick(table, frag):
        hits = [v for k, v in table.items() if frag in k]
        if len(hits) != 1:
            raise SystemExit(f"{len(hits)} kernels match {frag!r}")
        return hits[0]

    bf, bw = per_kernel("bench_FETCH_SIZE"), per_kernel("bench_WRITE_SIZE")
    cf, cw = per_kernel("copy_FETCH_SIZE"), per_kernel("copy_WRITE_SIZE")
    kib = 256 * 1024
    fs, ws = kib / pick(cf, "copyBuffer"), kib / pick(cw, "copyBuffer")
    out = {"note": "HBM bytes per step: rocprofv3 FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled "
                   "so that a 256 MiB device-to-device copy reads as 262144 KiB; MoE steps are two "
                   "MUL_MAT_ID launches (one grouped-GEMM kernel each at decode sizes)",
           "copy_calibration": {"bytes": 256 << 20, "fetch_kb_raw": round(kib / fs, 1),
                                "write_kb_raw": round(kib / ws, 1), "fetch_scale": round(fs, 4),
                                "write_scale": round(ws, 4)},
           "kernels": {}}
    for name, (frags, alg) in TRAFFIC_KERNELS.items():
        launches = 2 if name == "moe_q4_0" else 1
        f = sum(pick(bf, fr) for fr in frags) * launches
        w = sum(pick(bw, fr) for fr in frags) * launches
        tb = (f * fs + w * ws) * 1024
        e = {"kernels": frags, "launches_per_step": launches, "fetch_kb_raw": round(f, 1),
             "write_kb_raw": round(w, 1), "traffic_bytes": int(round(tb))}
        if alg:
            e["algorithmic_bytes"] = alg
            e["traffic_over_algorithmic"] = round(tb / alg, 3)
        out["kernels"][name] = e
    dst = ROOT / "profiles" / "traffic.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out, indent=1))


def copy_calibration(torch):
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 5}))


def cpu_legs(args, results, inputs):
    """CPU baselines of the same workloads (bounded samples of each), on the
    host's cores: oracle/cpu_baseline.c, the reference's CPU semantics
    (dequantize to bf16, fp32 products) vectorized and spread over OpenMP
    threads. Each leg lands in its workload's entry as "cpu_baseline"."""
    from oracle import oracle as O
    host = O.host_cpu()
    threads = min(16, host["affinity"] or 1)  # the GPU box's CPU share is 16 cores
    legs = [n for n in ("gemv_q8_0", "gemv_q6_k", "dequant_q4_0", "dequant_q6_k", "gemm_q4_0", "moe_q4_0")
            if n in inputs and n in results]
    budget = args.cpu_seconds / max(1, len(legs))

    def timed(fn):
        fn()  # warm-up
        passes, t0 = 0, time.perf_counter()
        while True:
            fn()
            passes += 1
            if time.perf_counter() - t0 >= budget:
                return passes, time.perf_counter() - t0

    for name in legs:
        base = {"cores": threads, "kind": "port", **host}
        if name == "gemv_q8_0":
            raw, x = inputs[name]
            p, dt = timed(lambda: O.cb_gemv_q8_0(raw, 14336, 4096, x, threads))
            base.update(value=raw.size * p / dt / 1e9, unit="GB/s",
                        sample=f"{p} passes of the Q8_0 14336x4096 GEMV (canonical GGUF bytes, packed-weight GB/s), "
                               f"{dt:.1f} s")
        elif name == "gemv_q6_k":
            raw, x = inputs[name]
            p, dt = timed(lambda: O.cb_gemv_q6_k(raw, 4096, 14336, x, threads))
            base.update(value=raw.size * p / dt / 1e9, unit="GB/s",
                        sample=f"{p} passes of the Q6_K 4096x14336 GEMV (canonical GGUF bytes, packed-weight GB/s), "
                               f"{dt:.1f} s")
        elif name == "dequant_q4_0":
            (raw,) = inputs[name]
            out = np.empty((4096, 4096), dtype=np.uint16)
            p, dt = timed(lambda: O.cb_dequant_q4_0(raw, 4096, 4096, threads, out))
            base.update(value=(raw.size + out.nbytes) * p / dt / 1e9, unit="GB/s",
                        packed_GBps=raw.size * p / dt / 1e9,
                        sample=f"{p} passes of the Q4_0 4096x4096 -> bf16 dequant (bytes in + out), {dt:.1f} s")
        elif name == "dequant_q6_k":
            (raw,) = inputs[name]
            out = np.empty((4096, 14336), dtype=np.uint16)
            p, dt = timed(lambda: O.cb_dequant_q6_k(raw, 4096, 14336, threads, out))
            base.update(value=(raw.size + out.nbytes) * p / dt / 1e9, unit="GB/s",
                        packed_GBps=raw.size * p / dt / 1e9,
                        sample=f"{p} passes of the Q6_K 4096x14336 -> bf16 dequant (bytes in + out), {dt:.1f} s")
        elif name == "gemm_q4_0":
            raw, x = inputs[name]
            p, dt = timed(lambda: O.cb_gemm_q4_0(raw, 4096, 4096, x, threads))
            base.update(value=2.0 * 512 * 4096 * 4096 * p / dt / 1e9, unit="GFLOP/s",
                        sample=f"{p} passes of the Q4_0 GEMM Y[512x4096] = X W^T, {dt:.1f} s")
        else:
            gu_raw, dn_raw, ids, x1, x2 = inputs[name]
            gu_per, dn_per = gu_raw.size // 128, dn_raw.size // 128

            def step():
                O.cb_moe_q4_0(gu_raw, gu_per, 128, 1536, 2048, x1, ids, threads)
                O.cb_moe_q4_0(dn_raw, dn_per, 128, 2048, 768, x2, ids, threads)

            p, dt = timed(step)
            touched = np.unique(ids).size
            base.update(value=touched * (gu_per + dn_per) * p / dt / 1e9, unit="GB/s",
                        sample=f"{p} steps of the Q4_0 MoE (gate_up + down MUL_MAT_ID over 128 experts, 64 tokens, "
                               f"top-8; touched experts' packed bytes), {dt:.1f} s")
        r = results[name]
        gpu = r["value"] * (1e3 if r["unit"] == "TFLOP/s" else 1.0)
        base["gpu_over_cpu"] = gpu / base["value"]
        r["cpu_baseline"] = base


def main():
    args = parse()
    if args.write_traffic:
        write_traffic(args.write_traffic)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    from spiral_amd import (ops, synth, TYPE_IQ4_NL, TYPE_IQ4_XS, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K,
                            TYPE_Q8_0, lib)
    from spiral_amd import row_bytes

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    if args.copy_calibration:
        copy_calibration(torch)
        return
    lib()  # fail loudly if the library is missing
    dev = torch.device("cuda:0")
    timer = Timer(torch)
    steps, warmup = args.steps, args.warmup
    results = {}

    def upload_planar(qtype, n, k, seed, copies):
        raw = synth.make_weights(qtype, n, k, seed)
        src = torch.from_numpy(raw).to(dev)
        first = ops.to_planar(qtype, src, n, k)
        ws = [first] + [first.clone() for _ in range(copies - 1)]
        del src
        return raw, ws

    def x_dev(m, k, seed):
        x = synth.make_x(m, k, seed)
        return x, torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)

    def record(name, issue, ev, per_launch, unit, peak, bound, extra=None):
        scale = 1e9 if unit == "GB/s" else 1e12
        step = ev / steps
        achieved = per_launch / step / scale
        r = {"value": per_launch * steps / ev / scale, "unit": unit, "ms_per_step": step * 1e3,
             "issue_us_per_step": issue / steps * 1e6, "step_us": step * 1e6,
             "preroll_ms": timer.preroll * 1e3, "late": bool(timer.timed_late),
             "roofline": {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                          "frac": achieved / peak}}
        if timer.spread:
            q = np.percentile(np.array(timer.spread) * 1e6, [10, 50, 90])
            r["step_us_replays"] = {"p10": float(q[0]), "p50": float(q[1]), "p90": float(q[2]),
                                    "replays": len(timer.spread), "launches_each": steps}
        if extra:
            r.update(extra)
        results[name] = r

    want = (lambda n: args.only in (None, n))
    cpu_inputs = {}  # workload -> canonical inputs for its CPU baseline leg

    # --- Q8_0 GEMV (headline) -------------------------------------------------
    if want("gemv_q8_0"):
        n, k = 14336, 4096
        wbytes = n * row_bytes(TYPE_Q8_0, k)
        raw, ws = upload_planar(TYPE_Q8_0, n, k, 1, copies_for(wbytes))
        x, xd = x_dev(1, k, 2)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        issue, ev = timer.run(lambda i: ops.mul_mat(TYPE_Q8_0, ws[i % len(ws)], n, k, xd, out=y), steps, warmup)
        record("gemv_q8_0", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q8_0 decode GEMV y[14336] = W[14336x4096] x[4096], batch 1, bf16 out",
                "bytes_per_launch": wbytes, "copies": len(ws)})
        cpu_inputs["gemv_q8_0"] = (raw, x)
        # the named relaxed mode on the same weights (block scale after the
        # block sum, weights not rounded to bf16): not the headline
        del ws

    if want("gemv_relaxed_q8_0"):
        n, k = 14336, 4096
        wbytes = n * row_bytes(TYPE_Q8_0, k)
        _, ws = upload_planar(TYPE_Q8_0, n, k, 1, copies_for(wbytes))
        _, xd = x_dev(1, k, 2)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        issue, ev = timer.run(lambda i: ops.gemv_relaxed(TYPE_Q8_0, ws[i % len(ws)], n, k, xd, out=y), steps,
                              warmup)
        record("gemv_relaxed_q8_0", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q8_0 decode GEMV 14336x4096, batch 1, bf16 out, in the named relaxed mode "
                            "(spiral_gemv_relaxed: block scale after the block sum; not the exact default)",
                "bytes_per_launch": wbytes, "copies": len(ws)})
        del ws

    # --- Q6_K GEMV ------------------------------------------------------------
    if want("gemv_q6_k"):
        n, k = 4096, 14336
        wbytes = n * row_bytes(TYPE_Q6_K, k)
        raw6, ws = upload_planar(TYPE_Q6_K, n, k, 3, copies_for(wbytes))
        x6, xd = x_dev(1, k, 4)
        cpu_inputs["gemv_q6_k"] = (raw6, x6)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        issue, ev = timer.run(lambda i: ops.mul_mat(TYPE_Q6_K, ws[i % len(ws)], n, k, xd, out=y), steps, warmup)
        record("gemv_q6_k", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q6_K decode GEMV y[4096] = W[4096x14336] x[14336], batch 1, bf16 out",
                "bytes_per_launch": wbytes, "copies": len(ws)})
        del ws

    # --- Q4_0 GEMV (the FFN up/gate shape of the Q8_0 workload) --------------------
    if want("gemv_q4_0"):
        n, k = 14336, 4096
        wbytes = n * row_bytes(TYPE_Q4_0, k)
        _, ws = upload_planar(TYPE_Q4_0, n, k, 5, copies_for(wbytes))
        _, xd = x_dev(1, k, 6)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        issue, ev = timer.run(lambda i: ops.mul_mat(TYPE_Q4_0, ws[i % len(ws)], n, k, xd, out=y), steps, warmup)
        record("gemv_q4_0", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q4_0 decode GEMV y[14336] = W[14336x4096] x[4096], batch 1, bf16 out",
                "bytes_per_launch": wbytes, "copies": len(ws)})
        del ws

    # --- K-quant and IQ4 GEMV (6-bit scales and mins; the non-linear codebook) ---
    for qname, qt in (("q4_k", TYPE_Q4_K), ("q5_k", TYPE_Q5_K), ("iq4_nl", TYPE_IQ4_NL), ("iq4_xs", TYPE_IQ4_XS)):
        wl = f"gemv_{qname}"
        if not want(wl):
            continue
        n, k = 14336, 4096
        wbytes = n * row_bytes(qt, k)
        _, ws = upload_planar(qt, n, k, 21, copies_for(wbytes))
        _, xd = x_dev(1, k, 22)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        issue, ev = timer.run(lambda i: ops.mul_mat(qt, ws[i % len(ws)], n, k, xd, out=y), steps, warmup)
        record(wl, issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": f"{qname.upper()} decode GEMV y[14336] = W[14336x4096] x[4096], batch 1, bf16 out",
                "bytes_per_launch": wbytes, "copies": len(ws)})
        del ws

    # --- Q4_0 small-batch product, m = 4 (speculative-decode batch) ---------------
    if want("mul_mat_q4_0_m4"):
        m, n, k = 4, 14336, 4096
        wbytes = n * row_bytes(TYPE_Q4_0, k)
        step_bytes = wbytes + m * k * 2 + m * n * 2
        _, ws = upload_planar(TYPE_Q4_0, n, k, 11, copies_for(wbytes))
        _, xd = x_dev(m, k, 12)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        issue, ev = timer.run(lambda i: ops.mul_mat(TYPE_Q4_0, ws[i % len(ws)], n, k, xd, out=y), steps, warmup)
        record("mul_mat_q4_0_m4", issue, ev, step_bytes, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q4_0 small-batch product Y[4x14336] = X[4x4096] W[14336x4096]^T, bf16 MFMA, "
                            "fp32 acc, bf16 out",
                "bytes_per_launch": step_bytes, "copies": len(ws)})
        del ws

    # --- Q4_0 -> bf16 dequant ---------------------------------------------------
    if want("dequant_q4_0"):
        n = k = 4096
        inb = n * row_bytes(TYPE_Q4_0, k)
        outb = n * k * 2
        copies = copies_for(inb + outb)
        raw0, ws = upload_planar(TYPE_Q4_0, n, k, 0, copies)
        cpu_inputs["dequant_q4_0"] = (raw0,)
        outs = [torch.empty((n, k), dtype=torch.bfloat16, device=dev) for _ in range(copies)]
        issue, ev = timer.run(lambda i: ops.dequant(TYPE_Q4_0, ws[i % copies], n, k, out=outs[i % copies]),
                               steps, warmup)
        record("dequant_q4_0", issue, ev, inb + outb, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q4_0 -> bf16 dequant, 4096x4096 (524,288 blocks)",
                "bytes_per_launch": inb + outb, "packed_bytes": inb, "copies": copies})
        results["dequant_q4_0"]["packed_GBps"] = inb / (ev / steps) / 1e9
        del ws, outs

    # --- Q6_K -> bf16 dequant ---------------------------------------------------
    if want("dequant_q6_k"):
        n, k = 4096, 14336
        inb = n * row_bytes(TYPE_Q6_K, k)
        outb = n * k * 2
        copies = copies_for(inb + outb)
        raw6, ws = upload_planar(TYPE_Q6_K, n, k, 3, copies)
        cpu_inputs["dequant_q6_k"] = (raw6,)
        outs = [torch.empty((n, k), dtype=torch.bfloat16, device=dev) for _ in range(copies)]
        issue, ev = timer.run(lambda i: ops.dequant(TYPE_Q6_K, ws[i % copies], n, k, out=outs[i % copies]),
                               steps, warmup)
        record("dequant_q6_k", issue, ev, inb + outb, "GB/s", HBM_PEAK_GBS, "hbm",
               {"workload": "Q6_K -> bf16 dequant, 4096x14336 (229,376 super-blocks)",
                "bytes_per_launch": inb + outb, "packed_bytes": inb, "copies": copies})
        results["dequant_q6_k"]["packed_GBps"] = inb / (ev / steps) / 1e9
        del ws, outs

    # --- Q4_0 dequant-GEMM, M = 512 ---------------------------------------------
    if want("gemm_q4_0"):
        m, n, k = 512, 4096, 4096
        wbytes = n * row_bytes(TYPE_Q4_0, k)
        copies = copies_for(wbytes + m * k * 2 + m * n * 2)
        raw7, ws = upload_planar(TYPE_Q4_0, n, k, 7, copies)
        xh = [x_dev(m, k, 8 + c) for c in range(copies)]
        xs = [t for _, t in xh]
        cpu_inputs["gemm_q4_0"] = (raw7, xh[0][0])
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        gws = ops.mul_mat_workspace(TYPE_Q4_0, n, k, m, dev)
        flops = 2.0 * m * n * k
        issue, ev = timer.run(lambda i: ops.mul_mat(TYPE_Q4_0, ws[i % copies], n, k, xs[i % copies], out=y,
                                                   workspace=gws), steps, warmup)
        record("gemm_q4_0", issue, ev, flops, "TFLOP/s", MFMA_BF16_PEAK_TFS, "mfma",
               {"workload": "Q4_0 prefill dequant-GEMM Y[512x4096] = X[512x4096] W[4096x4096]^T, bf16 MFMA, fp32 acc "
                            "(one step = X packing + GEMM kernel)",
                "flops_per_launch": flops, "copies": copies})
        del ws, xs

    # --- Q4_0 MoE grouped GEMM ----------------------------------------------------
    if want("moe_q4_0") or want("moe_gate_up_swiglu_q4_0") or want("moe_prefill_q4_0"):
        n_expert, hidden, inter2, inter = 128, 2048, 1536, 768
        n_tokens, top_k = 64, 8
        rng = np.random.default_rng(9)
        ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
        touched = np.unique(ids).size
        gu_per = inter2 * row_bytes(TYPE_Q4_0, hidden)
        dn_per = hidden * row_bytes(TYPE_Q4_0, inter)
        copies = max(2, int(np.ceil(2 * LLC_BYTES / (n_expert * (gu_per + dn_per)))))

        def stacked(n, k, per, seed):
            # every expert generated on its own (seed * 1000 + e), as the Q4_0
            # workload defines a weight; the copies repeat the stack
            first = torch.empty(n_expert * per, dtype=torch.uint8, device=dev)
            canon = np.empty(n_expert * per, dtype=np.uint8)  # canonical bytes, for the CPU leg
            for e in range(n_expert):
                raw = synth.make_weights(TYPE_Q4_0, n, k, seed * 1000 + e)
                canon[e * per:(e + 1) * per] = raw
                first[e * per:(e + 1) * per] = ops.to_planar(TYPE_Q4_0, torch.from_numpy(raw).to(dev), n, k)
            return canon, [first] + [first.clone() for _ in range(copies - 1)]

        gu_raw, gus = stacked(inter2, hidden, gu_per, 10)
        dn_raw, dns = stacked(hidden, inter, dn_per, 11)
        ids_d = torch.from_numpy(ids).to(dev)
        x1h, x1 = x_dev(n_tokens, hidden, 12)
        x1 = x1.view(n_tokens, 1, hidden)
        x2h, x2 = x_dev(n_tokens * top_k, inter, 13)
        x2 = x2.view(n_tokens, top_k, inter)
        cpu_inputs["moe_q4_0"] = (gu_raw, dn_raw, ids, x1h, x2h)
        y1 = torch.empty((n_tokens, top_k, inter2), dtype=torch.bfloat16, device=dev)
        y2 = torch.empty((n_tokens, top_k, hidden), dtype=torch.bfloat16, device=dev)
        ws1 = ops.mul_mat_id_workspace(n_expert, n_tokens, top_k, dev)
        ws2 = ops.mul_mat_id_workspace(n_expert, n_tokens, top_k, dev)

        def launch(i):
            c = i % copies
            ops.mul_mat_id(TYPE_Q4_0, gus[c], gu_per, n_expert, inter2, hidden, x1, ids_d, workspace=ws1, out=y1)
            ops.mul_mat_id(TYPE_Q4_0, dns[c], dn_per, n_expert, hidden, inter, x2, ids_d, workspace=ws2, out=y2)

        if want("moe_q4_0"):
            issue, ev = timer.run(launch, steps, warmup)
            wbytes = touched * (gu_per + dn_per)
            flops = 2.0 * n_tokens * top_k * (inter2 * hidden + hidden * inter)
            record("moe_q4_0", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
                   {"workload": "Q4_0 MoE: 128 experts (gate_up 1536x2048, down 2048x768), 64 tokens, top-8; "
                                "one step = gate_up + down MUL_MAT_ID",
                    "bytes_per_launch": wbytes, "touched_experts": int(touched),
                    "tflops": flops / (ev / steps) / 1e12, "copies": copies})

        # gate_up fused with SwiGLU: [64][8][768] bf16, the down stage's input
        if want("moe_gate_up_swiglu_q4_0"):
            h = torch.empty((n_tokens, top_k, inter), dtype=torch.bfloat16, device=dev)

            def launch_glu(i):
                ops.mul_mat_id_glu(TYPE_Q4_0, gus[i % copies], gu_per, n_expert, inter2, hidden, x1, ids_d,
                                   ops.GLU_SWIGLU, workspace=ws1, out=h)

            issue, ev = timer.run(launch_glu, steps, warmup)
            wbytes = touched * gu_per
            record("moe_gate_up_swiglu_q4_0", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
                   {"workload": "Q4_0 MoE gate_up (128 experts of 1536x2048, 64 tokens, top-8) fused with SwiGLU "
                                "into the [64][8][768] bf16 down-stage input; one step = one fused MUL_MAT_ID + GLU",
                    "bytes_per_launch": wbytes, "touched_experts": int(touched), "copies": copies})

        # prefill-sized batch: 1024 tokens, top-8 (64 pairs an expert on average)
        if want("moe_prefill_q4_0"):
            pt = 1024
            prng = np.random.default_rng(14)
            pids = np.stack([prng.choice(n_expert, top_k, replace=False) for _ in range(pt)]).astype(np.int32)
            pids_d = torch.from_numpy(pids).to(dev)
            _, px1 = x_dev(pt, hidden, 15)
            px1 = px1.view(pt, 1, hidden)
            _, px2 = x_dev(pt * top_k, inter, 16)
            px2 = px2.view(pt, top_k, inter)
            py1 = torch.empty((pt, top_k, inter2), dtype=torch.bfloat16, device=dev)
            py2 = torch.empty((pt, top_k, hidden), dtype=torch.bfloat16, device=dev)
            pws = ops.mul_mat_id_workspace(n_expert, pt, top_k, dev)  # the routing lists

            def launch_prefill(i):
                c = i % copies
                ops.mul_mat_id(TYPE_Q4_0, gus[c], gu_per, n_expert, inter2, hidden, px1, pids_d, workspace=pws,
                               out=py1)
                ops.mul_mat_id(TYPE_Q4_0, dns[c], dn_per, n_expert, hidden, inter, px2, pids_d, workspace=pws,
                               out=py2)

            issue, ev = timer.run(launch_prefill, steps, warmup)
            ptouched = np.unique(pids).size
            wbytes = ptouched * (gu_per + dn_per)
            flops = 2.0 * pt * top_k * (inter2 * hidden + hidden * inter)
            record("moe_prefill_q4_0", issue, ev, wbytes, "GB/s", HBM_PEAK_GBS, "hbm",
                   {"workload": "Q4_0 MoE prefill: 128 experts (gate_up 1536x2048, down 2048x768), 1024 tokens, "
                                "top-8 (64 pairs an expert on average); one step = gate_up + down MUL_MAT_ID",
                    "bytes_per_launch": wbytes, "touched_experts": int(ptouched),
                    "tflops": flops / (ev / steps) / 1e12, "copies": copies})
        del gus, dns

    if not results:
        raise SystemExit(f"unknown workload {args.only}")

    traffic = traffic_table()
    for name, r in results.items():
        r["roofline"]["traffic"] = traffic.get(name)
    head_name = "gemv_q8_0" if "gemv_q8_0" in results else next(iter(results))
    head = results[head_name]
    roof = dict(head["roofline"])

    cpu = None
    if not args.no_cpu:
        cpu_legs(args, results, cpu_inputs)
        if head_name in results and "cpu_baseline" in results[head_name]:
            cpu = results[head_name]["cpu_baseline"]

    line = {
        "metric": "quant GEMV packed-weight GB/s (% of HBM peak); dequant-GEMM TFLOP/s (% MFMA)",
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": head.get("workload", head_name), "kernel": head_name},
        "roofline": roof,
        "cpu_baseline": cpu,
        "workloads": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()

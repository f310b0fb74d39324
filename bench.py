#!/usr/bin/env python3
"""Decode-token-path benchmark on one MI355X.

Default workload (the headline metric): top-p sampling of B=1024 rows over a
V=65536 bf16 vocabulary (Zipf-like logits, T=0.6, p=0.95, top-k off).  A "step"
is one lsg_sample launch over one batch.  Inputs are resident in HBM before the
timed region; the timed region replays a HIP graph of K launches that rotate
over NBUF distinct logits buffers (> 512 MB in total, so the 256 MB Infinity
Cache cannot serve them), bracketed by torch.cuda.synchronize() and timed with
HIP events on the launch stream; the graph is replayed five times, each replay
timed on its own, and the median replay gives ms_per_step ("timing" holds the
spread).  cpu_baseline times the same step restated in torch on the host CPU,
at all host threads and at one.

Prints one JSON line (metric / value / roofline / cpu_baseline ...).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                  [--no-cpu-baseline]
Workloads: sample_huginn (default), sample_ouro, gate_cdb, cdb_mixed_depth, coda_ouro.

HBM traffic per launch (the roofline's "traffic" field) comes from two
rocprofv3 counter runs of the probe mode, then the summary mode:

  rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o run -- python3 bench.py --traffic-probe
  rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o run -- python3 bench.py --traffic-probe
  python3 bench.py --traffic-summary OUT/fetch OUT/write

The probe launches the workload's kernel on rotating buffers plus a plain
device-to-device copy of known size; the summary scales each counter by the
copy's ratio (bytes moved / counter reading) and writes
profiles/traffic_<workload>.json.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/sec and achieved HBM GB/s (% of peak) at batch 1024, vocab 65536"


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="sample_huginn",
                    choices=["sample_huginn", "sample_ouro", "gate_cdb", "cdb_mixed_depth", "coda_ouro"])
    ap.add_argument("--nbuf", type=int, default=0, help="logits buffers rotated (0: auto, > 512 MB)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=0, help="rows in the CPU baseline sample (0: auto)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="launch the kernel and a calibration copy for rocprofv3 --pmc, print nothing else")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 --pmc runs of --traffic-probe")
    return ap.parse_args()


COPY_BYTES = 256 << 20  # calibration copy: 256 MiB read + 256 MiB written
PROBE_LAUNCHES = 10


def _pmc_per_dispatch(outdir: str, counter: str):
    """Average counter value (KiB, as rocprofv3 reports FETCH_SIZE/WRITE_SIZE)
    per dispatch of the sampler/gate kernels and of the calibration copy."""
    import csv
    import glob

    files = glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {outdir}")
    kern, copy = [], []
    with open(files[0]) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            name, v = r["Kernel_Name"], float(r["Counter_Value"])
            if "lsg::" in name:
                kern.append((name, v))
            elif "copyBuffer" in name or "elementwise" in name and "copy" in name:
                copy.append(v)
    if not kern or not copy:
        raise SystemExit(f"{outdir}: kernel or calibration copy dispatches missing")
    names = sorted({n for n, _ in kern})
    return names, sum(v for _, v in kern) / len(kern), max(copy)


def _traffic_summary(a):
    kn, fk, fc = _pmc_per_dispatch(a.traffic_summary[0], "FETCH_SIZE")
    _, wk, wc = _pmc_per_dispatch(a.traffic_summary[1], "WRITE_SIZE")
    ff, fw = COPY_BYTES / (fc * 1024.0), COPY_BYTES / (wc * 1024.0)
    fetch_b, write_b = fk * 1024.0 * ff, wk * 1024.0 * fw
    out = {"workload": a.workload, "kernels": kn,
           "fetch_kib_per_dispatch": fk, "write_kib_per_dispatch": wk,
           "copy_fetch_kib": fc, "copy_write_kib": wc, "copy_bytes": COPY_BYTES,
           "fetch_scale": ff, "write_scale": fw,
           "traffic_bytes_per_launch": fetch_b + write_b}
    path = os.path.join(ROOT, "profiles", f"traffic_{a.workload}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


def _traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), if a summary has been recorded."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


REPLAYS = 5


def _time_graph(torch, launch, nlaunch: int, warmup: int):
    """Warm up eagerly, capture nlaunch launches in one graph, then time REPLAYS
    replays one by one (HIP events on the current stream, where the replay is
    launched, synchronised on both sides).  Returns the seconds of every timed replay."""
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for i in range(nlaunch):
            launch(i)
    torch.cuda.synchronize()
    graph.replay()  # untimed replay: graph upload
    torch.cuda.synchronize()
    times = []
    for _ in range(REPLAYS):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()  # graph.replay() launches on the current stream
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / 1e3)
    return times


def _median(v):
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def _timing(times, K):
    return {"replays": len(times), "steps_per_replay": K,
            "ms_per_step_median": _median(times) / K * 1e3,
            "ms_per_step_min": min(times) / K * 1e3, "ms_per_step_max": max(times) / K * 1e3}


def _host_threads():
    """Host threads for the all-cores CPU baseline: the affinity mask, capped by
    OMP_NUM_THREADS when the environment sets it (a shared host's CPU share)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def _timed_threads(torch, fn, min_seconds: float):
    """Calls fn() until min_seconds have passed; returns calls per second."""
    fn()  # warm-up (allocations, thread pool)
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            return n / dt


def _torch_cpu_sampling(torch, x, T, K, P, U):
    """The reference's token step restated in torch on the CPU: argmax for an
    all-greedy batch (sample.py:110-111), else softmax(x / T) (sample.py:66-68),
    top-k then top-p filtering on the descending sort (sample.py:72-81: kept set
    = the largest k, then the smallest prefix holding p of the renormalised
    mass, ties at the threshold kept) and the inverse CDF in vocabulary order
    with one uniform per row."""
    if T is None:
        return torch.argmax(x, dim=-1).to(torch.int32)
    xf = x.float()
    probs = torch.softmax(xf / T[:, None], dim=-1)
    V = x.shape[1]
    if K is not None:
        kk = torch.where((K >= 1) & (K < V), K, torch.full_like(K, V)).long()
        kth = torch.topk(probs, int(kk.max()), dim=-1).values.gather(1, (kk - 1)[:, None])
        probs = torch.where(probs >= kth, probs, torch.zeros_like(probs))  # ties at the k-th kept
    thr = torch.zeros_like(probs[:, :1])
    if P is not None:
        srt, _ = torch.sort(probs, dim=-1, descending=True)
        cs = torch.cumsum(srt, dim=-1)
        idx = torch.searchsorted(cs, P[:, None] * cs[:, -1:]).clamp_max(V - 1)
        thr = srt.gather(1, idx)  # the smallest kept value; its ties are kept too
    kept = torch.where((probs >= thr) & (probs > 0), probs, torch.zeros_like(probs))
    cdf = torch.cumsum(kept, dim=-1)
    ids = torch.searchsorted(cdf, (U * cdf[:, -1])[:, None], right=True).clamp_max(V - 1)
    return ids[:, 0].to(torch.int32)


def _cpu_baseline_sampling(torch, wl, rows: int, seconds: float):
    """torch-CPU restatement of the sampling step on a bounded sample of the
    workload's rows, at all host threads and at one."""
    x = wl["logits"][:rows].cpu()
    sel = lambda t: None if t is None else t[:rows].cpu()
    args = (x, sel(wl["temperatures"]), sel(wl.get("top_k")), sel(wl["top_p"]), sel(wl["uniforms"]))
    prev = torch.get_num_threads()
    out = {}
    try:
        for n in (_host_threads(), 1):
            torch.set_num_threads(n)
            out[n] = rows * _timed_threads(torch, lambda: _torch_cpu_sampling(torch, *args), seconds)
    finally:
        torch.set_num_threads(prev)
    return out


def _torch_cpu_gate(torch, h, w, b, F, step, tau):
    """The reference's gate step restated in torch on the CPU: F.linear in the
    model dtype (ouro.py:149, linear.py:32-33), F' = F + (1 - F) sigmoid(z)
    (exit_gates.py:13-15), the threshold and depth test (ouro.py:151-154) and
    the stable exit/keep filter (cdb_scheduler.py:215-228)."""
    z = torch.nn.functional.linear(h, w[None, :], b).squeeze(-1)
    Fn = F + (1.0 - F) * z.float().sigmoid()
    mask = (Fn >= tau) & (step + 1 >= 1)
    return Fn, torch.nonzero(mask)[:, 0].to(torch.int32), torch.nonzero(~mask)[:, 0].to(torch.int32)


def _cpu_baseline_gate(torch, wl, seconds: float):
    h = [t.cpu() for t in wl["hidden"]]
    w, b = wl["weight"].cpu(), wl["bias"].cpu()
    F0 = torch.zeros(h[0].shape[0])
    prev = torch.get_num_threads()
    out = {}

    def four_steps():
        F = F0
        for st, hs in enumerate(h):
            F, _, _ = _torch_cpu_gate(torch, hs, w, b, F, st, wl["tau"])

    try:
        for n in (_host_threads(), 1):
            torch.set_num_threads(n)
            out[n] = len(h) * _timed_threads(torch, four_steps, seconds)
    finally:
        torch.set_num_threads(prev)
    return out


def _probe(torch, launch, dev):
    for i in range(PROBE_LAUNCHES):
        launch(i)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def main():
    a = _parse()
    if a.traffic_summary:
        _traffic_summary(a)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}); the sampler shards rows across GPUs "
              "with no exchange, so run one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__

    pkg = __graft_entry__.package()
    wlmod = pkg.workloads
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    K, W = a.steps, a.warmup
    if a.traffic_probe:  # eager launches for the counter runs; no timing, no output
        K, W = PROBE_LAUNCHES, 0

    if a.workload in ("sample_huginn", "sample_ouro", "cdb_mixed_depth"):
        if a.workload == "sample_huginn":
            make = lambda seed: wlmod.sample_huginn(dev, seed=seed)
            desc = "sample_huginn: B=1024 V=65536 bf16 Zipf-like logits, T=0.6 top_p=0.95 top_k off"
        elif a.workload == "sample_ouro":
            make = lambda seed: wlmod.sample_ouro(dev, seed=seed)
            desc = "sample_ouro: B=256 V=49152 bf16 logits=hW^T, mixed T/top_k/top_p"
        else:
            make = lambda seed: wlmod.cdb_mixed_depth(dev, seed=seed)
            desc = "cdb_mixed_depth sampling: B=2048 V=65536 fp32 Student-t, mixed greedy/top_k/top_p"
        wl = make(3 if a.workload == "sample_huginn" else 1)
        x0 = wl["logits"]
        B, V = x0.shape
        buf_bytes = x0.numel() * x0.element_size()
        nbuf = a.nbuf or max(3, -(-(600 << 20) // buf_bytes))
        bufs = [x0] + [make(100 + i)["logits"] for i in range(nbuf - 1)]
        T, Kt, P, U = wl["temperatures"], wl.get("top_k"), wl["top_p"], wl["uniforms"]
        outs = [torch.empty(B, dtype=torch.int32, device=dev) for _ in range(nbuf)]

        def launch(i):
            pkg.sample_rows(bufs[i % nbuf], T, Kt, P, U, out=outs[i % nbuf])

        if a.traffic_probe:
            _probe(torch, launch, dev)
            return
        times = _time_graph(torch, launch, K, W)
        secs = _median(times)
        n_params = 2 + (Kt is not None)  # temperature, top_p (+ top_k) per row
        alg = wlmod.algorithmic_bytes_sampling(B, V, x0.element_size(), n_params)
        rows_per_s = B * K / secs
        per_launch = secs / K
        cpu = None
        if not a.no_cpu_baseline:
            rows = a.cpu_rows or 128
            r = _cpu_baseline_sampling(torch, wl, rows, seconds=5.0)
            (na, va), (_, v1) = list(r.items())[0], list(r.items())[-1]
            cpu = {"value": va, "unit": "rows/s", "cores": na, "kind": "port",
                   "value_1_core": v1, "cores_1_core": 1,
                   "sample": f"first {rows} rows of the same {B}x{V} workload, repeated for 5 s per thread "
                             "count: torch on the CPU (softmax, descending sort, cumsum top-k/top-p, "
                             "inverse CDF by searchsorted)"}
        result = {
            "metric": METRIC,
            "value": rows_per_s,
            "unit": "rows/s",
            "n_gpus": 1,
            "steps": K,
            "warmup": W,
            "ms_per_step": per_launch * 1e3,
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "f32",
            "data": "synthetic",
            "config": {"workload": desc, "batch": B, "vocab": V, "logits_dtype": str(x0.dtype).split(".")[-1],
                       "rotated_buffers": nbuf, "rotated_bytes": nbuf * buf_bytes},
            "timing": _timing(times, K),
            "roofline": {
                "bound": "hbm",
                "achieved": alg / per_launch / 1e9,
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": alg / per_launch / 1e9 / HBM_PEAK_GBS,
                "traffic": _traffic_from_profiles(a.workload),
            },
            "cpu_baseline": cpu,
        }
    elif a.workload == "coda_ouro":  # the fused coda tail: LM-head projection + token step
        B, H, V = 256, 2048, 49152
        g = torch.Generator(device=dev).manual_seed(1)
        h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
        nW = 3  # 3 x 201 MB of weights rotate, beyond the 256 MB Infinity Cache
        Ws = [(torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16) for _ in range(nW)]
        T = 0.3 + 0.9 * torch.rand(B, generator=g, device=dev)
        Kt = torch.tensor([1, 20, 50, V], dtype=torch.int32, device=dev)[
            torch.randint(0, 4, (B,), generator=g, device=dev)].contiguous()
        P = 0.8 + 0.2 * torch.rand(B, generator=g, device=dev)
        U = torch.rand(B, generator=g, device=dev)
        args = pkg.BatchSamplingArgs(T, Kt, P, U)
        ws = torch.empty(pkg.coda.workspace_bytes(B, V), dtype=torch.uint8, device=dev)
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        lg = torch.empty(B, V, dtype=torch.bfloat16, device=dev)

        def launch(i):
            pkg.coda.coda_sample(h, Ws[i % nW], args, workspace=ws, out=ids)

        def launch_gemm(i):
            pkg.coda.lm_head(h, Ws[i % nW], out=lg)

        f32 = torch.empty(B, V, device=dev)

        def launch_flinear(i):  # the reference's projection (hipBLASLt through F.linear)
            torch.nn.functional.linear(h, Ws[i % nW])

        def launch_ref_flow(i):  # the reference's data flow: bf16 logits -> fp32 buffer -> sampler
            f32.copy_(torch.nn.functional.linear(h, Ws[i % nW]))
            pkg.sample_rows(f32, T, Kt, P, U, out=ids)

        if a.traffic_probe:
            _probe(torch, launch_gemm, dev)
            return
        times = _time_graph(torch, launch, K, W)
        secs = _median(times)
        per = secs / K
        gtimes = _time_graph(torch, launch_gemm, K, W)
        gper = _median(gtimes) / K
        fper = _median(_time_graph(torch, launch_flinear, K, W)) / K
        rper = _median(_time_graph(torch, launch_ref_flow, K, W)) / K
        ntiles = -(-V // 192)
        gemm_bytes = V * H * 2 + B * H * 2 + B * V * 2 + B * ntiles * 8  # W, h, bf16 logits, tile maxima
        flops = 2.0 * B * H * V
        cpu = None
        if not a.no_cpu_baseline:
            rows = a.cpu_rows or 16
            hc, Wc = h[:rows].cpu(), Ws[0].cpu()
            sel = lambda t: t[:rows].cpu()
            Tc, Kc, Pc, Uc = sel(T), sel(Kt), sel(P), sel(U)
            prev = torch.get_num_threads()
            r = {}
            try:
                for n in (_host_threads(), 1):
                    torch.set_num_threads(n)
                    step = lambda: _torch_cpu_sampling(
                        torch, torch.nn.functional.linear(hc, Wc).float(), Tc, Kc, Pc, Uc)
                    r[n] = rows * _timed_threads(torch, step, 5.0 if n > 1 else 10.0)
            finally:
                torch.set_num_threads(prev)
            (na, va), (_, v1) = list(r.items())[0], list(r.items())[-1]
            cpu = {"value": va, "unit": "rows/s", "cores": na, "kind": "port", "value_1_core": v1,
                   "cores_1_core": 1,
                   "sample": f"first {rows} rows: torch on the CPU, F.linear in bf16 against the full "
                             f"[{V}, {H}] weight, then the sampling restatement; repeated for 5 s (10 s at 1 thread)"}
        result = {
            "metric": "coda rows/sec (LM-head projection + token step), B=256 H=2048 V=49152 bf16",
            "value": B / per, "unit": "rows/s", "n_gpus": 1, "steps": K, "warmup": W,
            "ms_per_step": per * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "coda_ouro: h [256, 2048] bf16 N(0,1), W [49152, 2048] bf16 N(0, 0.02^2), "
                                   "mixed T/top_k/top_p", "batch": B, "hidden": H, "vocab": V,
                       "rotated_weights": nW},
            "timing": _timing(times, K),
            "projection": {"ms_per_launch": gper * 1e3, "timing": _timing(gtimes, K),
                           "mfma_tflops": flops / gper / 1e12, "mfma_peak_tflops": 2500.0,
                           "mfma_frac": flops / gper / 1e12 / 2500.0},
            "reference_flow": {"f_linear_ms": fper * 1e3, "f_linear_fp32_copy_sample_ms": rper * 1e3,
                               "note": "the same graph harness: F.linear (hipBLASLt) alone, and F.linear -> "
                                       "copy into an fp32 [B, V] buffer -> lsg_sample on fp32"},
            "roofline": {"bound": "hbm", "achieved": gemm_bytes / gper / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gemm_bytes / gper / 1e9 / HBM_PEAK_GBS,
                         "traffic": _traffic_from_profiles(a.workload)},
            "cpu_baseline": cpu,
        }
    else:  # gate_cdb: the 4-step exit gate with compaction (latency-bound)
        wl = wlmod.gate_cdb(dev)
        gate = pkg.OuroExitGate(wl["weight"], wl["bias"], exit_threshold=wl["tau"], loop_steps=4)
        B, H = wl["hidden"][0].shape
        nset = 320  # 320 hidden-state sets of 2 MiB: 640 MiB rotate, beyond the 256 MB Infinity Cache
        hs = [torch.randn(B, H, device=dev).to(torch.bfloat16) for _ in range(nset)]
        F = torch.zeros(B, device=dev)

        def launch(i):
            gate.exit_signal_compact(hs[i % nset], F, i % 4)

        if a.traffic_probe:
            _probe(torch, launch, dev)
            return
        times = _time_graph(torch, launch, K, W)
        secs = _median(times)
        per = secs / K
        alg = wlmod.algorithmic_bytes_gate(B, H)
        cpu = None
        if not a.no_cpu_baseline:
            r = _cpu_baseline_gate(torch, wl, seconds=3.0)
            (na, va), (_, v1) = list(r.items())[0], list(r.items())[-1]
            cpu = {"value": va, "unit": "steps/s", "cores": na, "kind": "port", "value_1_core": v1,
                   "cores_1_core": 1,
                   "sample": "the same 4 gate steps (B=512, H=2048 bf16), repeated for 3 s per thread count: "
                             "torch on the CPU (F.linear, sigmoid update, threshold, nonzero compaction)"}
        result = {
            "metric": "exit-gate steps/sec (B=512, H=2048 bf16, with compaction)",
            "value": K / secs, "unit": "steps/s", "n_gpus": 1, "steps": K, "warmup": W,
            "ms_per_step": per * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": "gate_cdb: B=512 H=2048 bf16, tau=0.2, 4 loop steps", "batch": B, "hidden": H,
                       "rotated_sets": nset},
            "timing": _timing(times, K),
            "roofline": {"bound": "hbm", "achieved": alg / per / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": alg / per / 1e9 / HBM_PEAK_GBS, "traffic": _traffic_from_profiles(a.workload)},
            "cpu_baseline": cpu,
        }
    print(json.dumps(result))


if __name__ == "__main__":
    main()

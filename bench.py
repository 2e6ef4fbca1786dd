#!/usr/bin/env python3
"""Benchmark of the quantized MoE gather_qmm path on one MI355X.

Headline (``value``): the decode gate_up gather_qmm with fused SwiGLU --
1 token, hidden 2048, 256 experts, top-10, fused gate_up W [256, 1024, 2048]
4-bit group 64 -- in HBM GB/s of algorithmic bytes (each routed expert's packed
codes + scales + biases once, plus x in and h out).  One step is one call.

Method: every step reads a different weight set and a different set of 10
experts (weight sets rotated over >= 1.2 GB so the 256 MB Infinity Cache cannot
serve them), each window of K launches is captured in one HIP graph between
two single-wave launches that write the GPU's 100 MHz clock, and the windows'
graphs are replayed back to back: a window's time is the difference of its two
clock stamps, which leaves each graph's own launch outside it (events around
the same replays, which include it, are reported beside).  The other workloads
are measured the same way and reported under ``configs``; the CPU baseline is
the oracle's C restatement timed on this host.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--configs 0,1,2,3,4,5,6,7]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE gather_qmm HBM GB/s (decode), TFLOP/s (prefill), % roofline, 1 MI355X"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, vendor spec
BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA, vendor spec
INT8_PEAK_TOPS = 5000.0     # dense int8 MFMA, vendor spec


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="0,1,2,3,4,5,6,7",
                    help="0-4 the five workloads, 5 workload 0 with 8-bit codes, 6 the decode-width sweep, "
                         "7 the whole MoE block")
    ap.add_argument("--rotate-gb", type=float, default=1.2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default=None,
                    help="run one workload's timed loop only, or 'copy' for the calibration copy kernel")
    ap.add_argument("--eager", action="store_true", help="launch the timed steps eagerly (no graph)")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured-peak probes")
    ap.add_argument("--gemm-units", action="store_true",
                    help="per-unit timing of workload 3's grouped GEMM (measurement build) and exit")
    ap.add_argument("--decode-phases", action="store_true",
                    help="per-phase timestamps of the decode gate_up kernel (workload 1) from libqmoe_stamps.so")
    ap.add_argument("--traffic", action="store_true",
                    help="measure the decode kernel's HBM traffic live with rocprofv3 counter passes")
    ap.add_argument("--power", type=float, default=0.0, metavar="SECONDS",
                    help="after timing each workload, replay its windows for SECONDS while sampling the "
                         "board's socket power and gfx clocks (amd-smi)")
    return ap.parse_args()


def to_dev(a, dtype, dev):
    import torch

    a = np.ascontiguousarray(a)
    if dtype == "bf16":
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    if dtype == "words":
        return torch.from_numpy(a.view(np.int32)).to(dev)
    return torch.from_numpy(a).to(dev)


def random_like_words(shape, dev, gen):
    import torch

    return torch.randint(-2 ** 31, 2 ** 31 - 1, shape, dtype=torch.int32, device=dev, generator=gen)


def random_scales(shape, dev, gen):
    import torch

    s = torch.rand(shape, device=dev, generator=gen) * 0.015 + 0.005
    return s.to(torch.bfloat16)


def random_biases(shape, dev, gen):
    import torch

    return (torch.randn(shape, device=dev, generator=gen) * 0.05).to(torch.bfloat16)


def weight_sets(wl, n_sets, dev, seed):
    """Set 0 is the seeded workload; the others are fresh random sets on the device."""
    import torch

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    sets = [(to_dev(wl["w"], "words", dev), to_dev(wl["s"], "bf16", dev), to_dev(wl["b"], "bf16", dev))]
    for _ in range(1, n_sets):
        sets.append((random_like_words(wl["w"].shape, dev, gen), random_scales(wl["s"].shape, dev, gen),
                     random_biases(wl["b"].shape, dev, gen)))
    return sets


def time_eager(cycle, steps, warmup, dev):
    """The first `steps` launches of the cycle, eagerly (used under counter
    collection, where each dispatch is profiled on its own)."""
    import torch

    for i in range(warmup):
        cycle[i % len(cycle)]()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    st = torch.cuda.current_stream()
    e0.record(st)
    for fn in cycle[:steps]:
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / steps
    return sec, {"min": sec, "median": sec, "max": sec, "rounds": 1, "windows": 1, "graphs": None}


CALIBRATION_MIB = 256


def calibration_copy(dev, mib=CALIBRATION_MIB, reps=5):
    """A plain device copy of known size: the scale for HBM byte counters."""
    import torch

    n = mib * 2 ** 20 // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes_read": n * 4, "bytes_written": n * 4, "reps": reps}))


# ------------------------------------------------------------- HBM traffic
#
# rocprofv3 FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the decode kernel,
# scaled by what the same counters read for a plain device copy of known size.
# `--traffic` measures them live (rocprofv3 children started before this
# process touches the GPU); otherwise the committed summary supplies them.

TRAFFIC_KERNEL = "qmv64_flat_kernel<1, 64, 4>"  # the one-token decode gate_up + SwiGLU kernel (bench workload 1)
TRAFFIC_PROFILE = ROOT / "profiles" / "qmv64_decode_gate_up.traffic.txt"


def _pmc_run(counter, only, outdir):
    import csv
    import subprocess

    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", str(outdir), "-o", "run", "--",
           sys.executable, str(ROOT / "bench.py"), "--only", only, "--eager", "--steps", "20", "--warmup", "2",
           "--no-cpu-baseline"]
    env = dict(os.environ, TMPDIR="/tmp")
    subprocess.run(cmd, cwd="/tmp", env=env, check=True, timeout=90, stdout=subprocess.DEVNULL,
                   stderr=subprocess.DEVNULL)
    per = {}
    for path in Path(outdir).rglob("*counter_collection.csv"):
        for row in csv.DictReader(open(path)):
            per.setdefault(row["Kernel_Name"], {}).setdefault(row["Dispatch_Id"], 0.0)
            per[row["Kernel_Name"]][row["Dispatch_Id"]] += float(row["Counter_Value"])
    return {k: sum(v.values()) / len(v) for k, v in per.items()}


def _pick(per, needle):
    hits = [v for k, v in per.items() if needle in k]
    if not hits:
        raise RuntimeError(f"no dispatch of {needle} in the counter output")
    return hits[0]


def measure_traffic_live():
    """Four counter passes: FETCH_SIZE and WRITE_SIZE of the decode kernel and
    of the calibration copy.  Bytes per launch, or None when rocprofv3 fails."""
    import shutil
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None
    tmp = Path(tempfile.mkdtemp(prefix="qmoe_pmc_", dir="/tmp"))
    try:
        f_k = _pick(_pmc_run("FETCH_SIZE", "1", tmp / "f1"), TRAFFIC_KERNEL)
        w_k = _pick(_pmc_run("WRITE_SIZE", "1", tmp / "w1"), TRAFFIC_KERNEL)
        f_c = _pick(_pmc_run("FETCH_SIZE", "copy", tmp / "fc"), "copyBuffer")
        w_c = _pick(_pmc_run("WRITE_SIZE", "copy", tmp / "wc"), "copyBuffer")
    except Exception as exc:  # noqa: BLE001 - traffic is optional
        print(f"[bench] traffic measurement failed: {exc}", file=sys.stderr, flush=True)
        return None
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return _traffic(f_k, w_k, f_c, w_c, "live rocprofv3 --pmc")


def _traffic(fetch_kib, write_kib, copy_fetch_kib, copy_write_kib, source):
    copy_bytes = CALIBRATION_MIB * 2 ** 20
    f_scale = copy_bytes / (copy_fetch_kib * 1024)
    w_scale = copy_bytes / (copy_write_kib * 1024)
    return {"bytes": fetch_kib * 1024 * f_scale + write_kib * 1024 * w_scale, "fetch_kib": fetch_kib,
            "write_kib": write_kib, "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
            "source": source}


def traffic_from_profile():
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("json: "):
                d = json.loads(line[6:])
                return _traffic(d["fetch_kib"], d["write_kib"], d["copy_fetch_kib"], d["copy_write_kib"],
                                TRAFFIC_PROFILE.name)
    except (OSError, ValueError, KeyError):
        pass
    return None


def cycle_len(steps: int, per_call_bytes: float, rotate_bytes: float) -> int:
    """Launches in one rotation cycle: at least `steps` and enough that the
    cycle touches `rotate_bytes` of distinct weights, rounded up to whole
    windows of exactly `steps` launches."""
    need = max(steps, int(np.ceil(rotate_bytes / max(per_call_bytes, 1.0))))
    return steps * int(np.ceil(need / steps))


def time_graph(cycle, steps, warmup, dev, min_rounds=7):
    """Time a rotation cycle of launches in windows of exactly `steps`.

    The cycle (a multiple of `steps` long) is cut into windows of `steps`
    consecutive launches, each captured as one graph.  After `warmup` eager
    launches and ~0.3 s of untimed replays of the whole cycle, max(min_rounds,
    windows) windows are replayed back to back in cycle order, each bracketed by
    events on the replay stream (no host sync in between: the GPU never waits
    for the host to submit a graph).  Consecutive windows continue the cycle, so
    a weight byte comes back only after the whole cycle's other bytes have
    streamed past.  Returns (median seconds per step, {"min", "median", "max",
    "rounds", "windows", "graphs"})."""
    import statistics

    import torch

    L = len(cycle)
    assert L % steps == 0, (L, steps)
    for i in range(warmup):
        cycle[i % L]()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graphs = []
    with torch.cuda.stream(s):
        for w in range(L // steps):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for fn in cycle[w * steps:(w + 1) * steps]:
                    fn()
            graphs.append(g)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    n_warm = min(50, max(1, int(0.3 / max(time.perf_counter() - t0, 1e-4))))
    st = torch.cuda.current_stream()
    for _ in range(n_warm):
        for g in graphs:
            g.replay()
    rounds = max(min_rounds, len(graphs))
    evs = []
    for r in range(rounds):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        graphs[r % len(graphs)].replay()
        e1.record(st)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    per = [e0.elapsed_time(e1) / 1e3 / steps for e0, e1 in evs]
    med = statistics.median(per)
    return med, {"min": min(per), "median": med, "max": max(per), "rounds": rounds, "windows": len(graphs),
                 "graphs": graphs}


def time_stamped(cycle, steps, warmup, dev, min_rounds=7):
    """Time a rotation cycle of launches in windows of exactly `steps`, from
    the GPU's own clock.

    max(min_rounds, windows) windows -- consecutive windows continue the
    cycle, as in time_graph -- are each captured as one graph that opens and
    closes with a single-wave stamp launch (qmoe_peak_stamp: the 100 MHz
    s_memrealtime counter, written with a vector store), and the graphs are
    replayed back to back.  A window's time is the difference of its two
    stamps: its `steps` launches plus the one stamp launch that closes it.  The
    GPU-side cost of launching each graph falls before its opening stamp,
    outside every window (time_graph brackets each graph launch with events,
    and that cost is then spread over the window's calls).  HIP does not time
    events recorded by graph nodes (hipEventElapsedTime fails on them), hence
    the stamp kernel.  After `warmup` eager launches and ~0.3 s of untimed
    replays, the graphs are replayed once more and the stamps read.  Returns
    (median seconds per step, {"min", "median", "max", "rounds", "windows",
    "graphs"})."""
    import statistics

    import torch

    L = len(cycle)
    assert L % steps == 0, (L, steps)
    windows = L // steps
    rounds = max(min_rounds, windows)
    for i in range(warmup):
        cycle[i % L]()
    torch.cuda.synchronize()
    P = peaks_lib()
    stamps = torch.zeros(2 * rounds, dtype=torch.int64, device=dev)

    def stamp(slot, st):
        if P.qmoe_peak_stamp(stamps.data_ptr(), slot, st) != 0:
            raise RuntimeError("qmoe_peak_stamp failed")

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graphs = []
    with torch.cuda.stream(s):
        for r in range(rounds):
            w = r % windows
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                stamp(2 * r, s.cuda_stream)
                for fn in cycle[w * steps:(w + 1) * steps]:
                    fn()
                stamp(2 * r + 1, s.cuda_stream)
            graphs.append(g)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    n_warm = min(50, max(1, int(0.3 / max(time.perf_counter() - t0, 1e-4))))
    for _ in range(n_warm):
        for g in graphs:
            g.replay()
    # the timed pass: also events around each graph launch (their span adds
    # the graph launch to the window: both figures from the same replays)
    st = torch.cuda.current_stream()
    evs = []
    for g in graphs:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    t = stamps.cpu().numpy()
    per = [float(t[2 * r + 1] - t[2 * r]) * 1e-8 / steps for r in range(rounds)]
    if min(per) <= 0:
        raise RuntimeError(f"non-increasing GPU clock stamps: {t.tolist()}")
    med = statistics.median(per)
    ev = statistics.median([a.elapsed_time(b) / 1e3 / steps for a, b in evs])
    return med, {"min": min(per), "median": med, "max": max(per), "rounds": rounds, "windows": windows,
                 "graphs": graphs, "events_per_step": ev}


def timer(args):
    return time_eager if args.eager else time_stamped


def sample_power(run_once, seconds):
    """Socket power (W) and per-XCD gfx clocks (MHz) from `amd-smi metric -p -c`
    sampled every ~0.25 s while `run_once` (one pass over a workload's windows)
    repeats for `seconds`.  The first second of samples is dropped (the board
    ramps to its limit).  Returns min / median / max of each, or the reason
    there are none."""
    import csv
    import io
    import shutil
    import statistics
    import subprocess
    import threading

    import torch

    smi = shutil.which("amd-smi")
    if smi is None:
        return {"error": "amd-smi not found"}
    samples, stop = [], threading.Event()

    def sampler():
        t0 = time.perf_counter()
        while not stop.is_set():
            try:
                out = subprocess.run([smi, "metric", "-p", "-c", "--csv"], capture_output=True, text=True,
                                     timeout=10).stdout
                rows = [ln for ln in out.splitlines() if ln.strip() and "," in ln]
                row = next(csv.DictReader(io.StringIO("\n".join(rows))))
                clk = [float(row[f"gfx_{i}_clk"]) for i in range(8) if row.get(f"gfx_{i}_clk", "N/A") != "N/A"]
                samples.append((time.perf_counter() - t0, float(row["socket_power"]), statistics.mean(clk)))
            except Exception:  # noqa: BLE001 - a missing field drops that sample
                pass
            stop.wait(0.25)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        run_once()
        torch.cuda.synchronize()
    stop.set()
    th.join()
    kept = [s for s in samples if s[0] >= 1.0]
    if not kept:
        return {"error": "no samples", "raw": len(samples)}

    def summ(v):
        return {"min": round(min(v), 1), "median": round(statistics.median(v), 1), "max": round(max(v), 1)}

    return {"socket_power_W": summ([s[1] for s in kept]), "gfx_clock_MHz": summ([s[2] for s in kept]),
            "samples": len(kept), "seconds": seconds}


# ------------------------------------------------------------ measured peaks


def peaks_lib():
    """libqmoe_peaks.so (include/qmoe_peaks.h) through ctypes."""
    import ctypes

    from titan_amd import build as tbuild

    L = ctypes.CDLL(str(tbuild.PEAKS_LIB))
    c_int, c_vp = ctypes.c_int, ctypes.c_void_p
    sigs = {"qmoe_peak_stream_read": [c_vp, ctypes.c_size_t, c_vp, c_vp],
            "qmoe_peak_mfma_bf16": [c_int, c_vp, c_vp],
            "qmoe_peak_mfma_i8": [c_int, c_vp, c_vp],
            "qmoe_peak_launch": [c_int, c_int, c_vp],
            "qmoe_peak_stamp": [c_vp, c_int, c_vp],
            "qmoe_peak_chain": [c_vp, c_int, c_int, c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp],
            "qmoe_peak_burst": [c_vp, c_int, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp, c_vp]}
    for name, argtypes in sigs.items():
        fn = getattr(L, name)
        fn.restype = c_int
        fn.argtypes = argtypes
    return L


def measure_peaks(dev, read_gib=4, power_seconds=0.0):
    """What this part sustains, with the probe kernels of libqmoe_peaks.so: a
    streaming read of `read_gib` GiB (beyond the 256 MB Infinity Cache) and
    dense bf16 / int8 MFMA loops over random register operands.  Medians of
    five timed runs after one warm-up.  With power_seconds > 0 each probe is
    then repeated for that long while the board's power and clocks are
    sampled (sample_power)."""
    import statistics

    import torch

    L = peaks_lib()
    nbytes = read_gib * 2 ** 30
    buf = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).random_()
    sink = torch.zeros(max(L.qmoe_peak_stream_blocks(), L.qmoe_peak_mfma_waves()), dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream()

    def timed(launch, reps=5):
        launch()
        torch.cuda.synchronize()
        out = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(st)
            launch()
            e1.record(st)
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1) / 1e3)
        return statistics.median(out)

    def check(rc):
        if rc != 0:
            raise RuntimeError(f"peak probe failed (code {rc})")

    t_read = timed(lambda: check(L.qmoe_peak_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), st.cuda_stream)))
    iters = 20000
    waves = L.qmoe_peak_mfma_waves()
    t_bf16 = timed(lambda: check(L.qmoe_peak_mfma_bf16(iters, sink.data_ptr(), st.cuda_stream)))
    t_i8 = timed(lambda: check(L.qmoe_peak_mfma_i8(iters, sink.data_ptr(), st.cuda_stream)))
    power = None
    if power_seconds > 0:
        power = {
            "stream_read": sample_power(
                lambda: check(L.qmoe_peak_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), st.cuda_stream)),
                power_seconds),
            "mfma_bf16": sample_power(lambda: check(L.qmoe_peak_mfma_bf16(iters, sink.data_ptr(), st.cuda_stream)),
                                      power_seconds),
            "mfma_i8": sample_power(lambda: check(L.qmoe_peak_mfma_i8(iters, sink.data_ptr(), st.cuda_stream)),
                                    power_seconds),
        }
    del buf
    torch.cuda.empty_cache()
    res = {"hbm_read_GBps": round(nbytes / t_read / 1e9, 1),
            "bf16_mfma_TFLOPs": round(waves * iters * 4 * 32768 / t_bf16 / 1e12, 1),
            "int8_mfma_TOPs": round(waves * iters * 4 * 65536 / t_i8 / 1e12, 1),
            "method": f"stream read of {read_gib} GiB (16-byte non-temporal loads, 2048 blocks); "
                      f"{waves} waves x {iters} x 4 independent v_mfma_f32_32x32x16_bf16 / "
                      "v_mfma_i32_32x32x32_i8 on random register operands; median of 5"}
    if power is not None:
        res["power"] = power
    return res


# --------------------------------------------------------------- workloads
#
# Every setup returns (workload, cycle, meta): `cycle` is the rotation of
# launches timed in windows of exactly --steps (time_graph), long enough that
# its weight bytes exceed --rotate-gb, with weight sets sized so that a cycle
# touches every weight byte at most about once.


MAX_ROTATION_BYTES = 16e9  # cap on the weight sets one workload keeps resident


def n_sets_needed(wl, cycle_bytes, rotate_gb):
    per = wl["w"].nbytes + wl["s"].nbytes + wl["b"].nbytes
    want = min(max(rotate_gb * 1e9, cycle_bytes), MAX_ROTATION_BYTES)
    return max(1, int(np.ceil(want / per)))


def setup_cfg1(args, dev):
    """Decode gate_up + SwiGLU: 10 experts of one token.  Each launch reads 10
    experts no other launch of the cycle reads (sets x 256 experts, dealt out
    by per-set permutations)."""
    import torch
    from titan_amd import ops, synth

    wl = synth.make(1)
    per_call = synth.algorithmic_bytes(1)
    L = cycle_len(args.steps, per_call, args.rotate_gb * 1e9)
    sets = weight_sets(wl, max(n_sets_needed(wl, L * per_call, args.rotate_gb), int(np.ceil(L * 10 / 256))), dev,
                       101)
    rng = np.random.default_rng(1001)
    x = to_dev(wl["x"], "bf16", dev)
    E = wl.meta["E"]
    perms = [rng.permutation(E) for _ in sets]
    cursor = [0] * len(sets)
    idxs = []
    for i in range(L):
        si = i % len(sets)
        if cursor[si] + 10 > E:
            perms[si] = rng.permutation(E)
            cursor[si] = 0
        idxs.append(torch.from_numpy(perms[si][cursor[si]:cursor[si] + 10].astype(np.int32)[None]).to(dev))
        cursor[si] += 10
    idxs[0] = to_dev(wl["idx"], "i32", dev)
    outs = [torch.empty(1, 10, 512, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    # load-time repack into the gate/up-paired tile layout (outside the timed region)
    tsets = [ops.repack_tiles(w, s, b, swiglu_pairs=True) for (w, s, b) in sets]
    torch.cuda.synchronize()

    def mk_tiles(i):
        tw = tsets[i % len(tsets)]
        idx = idxs[i]

        def f():
            ops._lib.call("qmoe_moe_gate_up_swiglu_tiles", x.data_ptr(), idx.data_ptr(), 1, 10, 2048,
                          tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 512, outs[i % 2].data_ptr(),
                          torch.cuda.current_stream().cuda_stream)
        return f

    def mk_mlx(i):
        w, s, b = sets[i % len(sets)]
        idx = idxs[i]

        def f():
            ops._lib.call("qmoe_moe_gate_up_swiglu", x.data_ptr(), idx.data_ptr(), 1, 10, 2048, w.data_ptr(),
                          s.data_ptr(), b.data_ptr(), 256, 512, 64, 4, outs[i % 2].data_ptr(),
                          torch.cuda.current_stream().cuda_stream)
        return f

    # the per-call floor of this launch shape (libqmoe_peaks.so): the same
    # 1280 single-wave blocks doing nothing, and walking the dependent chain
    # (arguments -> expert id -> the first 1 KiB weight row) over the same
    # ids and weight sets
    P = peaks_lib()
    sink = torch.zeros(1280, dtype=torch.int32, device=dev)

    def check(rc):
        if rc != 0:
            raise RuntimeError(f"floor probe failed (code {rc})")

    def mk_chain(i, wpb=1):
        w = sets[i % len(sets)][0]
        idx = idxs[i]

        def f():
            check(P.qmoe_peak_chain(idx.data_ptr(), 10, E, w.data_ptr(), 1024, 1024, 8, wpb, sink.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream))
        return f

    def mk_launch(wpb):
        def f():
            check(P.qmoe_peak_launch(1280, wpb, torch.cuda.current_stream().cuda_stream))
        return f

    # the whole memory work after the ids: every wave reads all eight of its
    # code rows and their scale and bias bytes (four-wave workgroups)
    def mk_burst(i):
        w, s_, b_ = sets[i % len(sets)]
        idx = idxs[i]

        def f():
            check(P.qmoe_peak_burst(idx.data_ptr(), 10, E, w.data_ptr(), s_.data_ptr(), b_.data_ptr(), 1024, 1024, 64,
                                    8, 4, sink.data_ptr(), torch.cuda.current_stream().cuda_stream))
        return f

    return wl, [mk_mlx(i) for i in range(L)], {
        # the same 1280 waves also in workgroups of two and four waves
        "floor": {"launch": [mk_launch(1)] * L, "chain": [mk_chain(i) for i in range(L)],
                  "wider": {w: ([mk_launch(w)] * L, [mk_chain(i, w) for i in range(L)]) for w in (2, 4)},
                  "burst": [mk_burst(i) for i in range(L)], "burst_bytes": 10 * 1024 * (1024 + 2 * 64),
                  "chain_bytes": 1280 * 1024 + 10 * 4},
        "bytes": per_call, "flops": synth.algorithmic_flops(1), "bound": "hbm",
        "kernel": "qmv64_flat_kernel<1, 64, 4>", "sets": len(sets),
        "cycle_bytes": L * per_call,
        "alt": ("tile_layout_us_per_call", [mk_tiles(i) for i in range(L)]),
        "workload": "decode gate_up gather_qmm + SwiGLU: 1 token, H=2048, E=256, top_k=10, "
                    "W [256,1024,2048] int4 g64 bf16 scale/bias -> h [10,512]"}


def setup_cfg0(args, dev):
    """Dense quantized_matmul: every launch of the cycle reads its own weight set."""
    import torch
    from titan_amd import ops, synth

    wl = synth.make(0)
    per_call = synth.algorithmic_bytes(0)
    L = cycle_len(args.steps, per_call, args.rotate_gb * 1e9)
    sets = weight_sets(wl, min(L, n_sets_needed(wl, L * per_call, args.rotate_gb)), dev, 100)
    x = to_dev(wl["x"], "bf16", dev)
    out = torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)
    tsets = [ops.repack_tiles(w[None], s[None], b[None]) for (w, s, b) in sets]
    torch.cuda.synchronize()

    def mk_tiles(i):
        tw = tsets[i % len(tsets)]

        def f():
            ops._lib.call("qmoe_gather_qmv_tiles", x.data_ptr(), None, None, 1, 2048, tw.wp.data_ptr(),
                          tw.sb.data_ptr(), 1, 4096, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        return f

    def mk_mlx(i):
        w, s, b = sets[i % len(sets)]

        def f():
            ops._lib.call("qmoe_quantized_matmul", x.data_ptr(), 1, 2048, w.data_ptr(), s.data_ptr(),
                          b.data_ptr(), 4096, 64, 4, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        return f

    return wl, [mk_mlx(i) for i in range(L)], {
        "bytes": per_call, "flops": synth.algorithmic_flops(0), "bound": "hbm",
        "kernel": "qmv64_kernel<1, 0, 0, 2, 64, false, false>", "sets": len(sets),
        "cycle_bytes": min(L, len(sets)) * per_call,
        "alt": ("tile_layout_us_per_call", [mk_tiles(i) for i in range(L)]),
        "workload": "dense quantized_matmul x [1,2048] . W [4096,2048] int4 g64"}


def setup_cfg2(args, dev):
    """Decode down + weighted sum, 8 tokens: a fresh routing per launch (the
    workload's distinct-expert statistics), weight sets cycled."""
    import torch
    from titan_amd import ops, synth

    wl = synth.make(2)
    est_call = wl.meta["distinct"] * 2048 * (256 + 32)
    L = cycle_len(args.steps, est_call, args.rotate_gb * 1e9)
    sets = weight_sets(wl, n_sets_needed(wl, L * est_call, args.rotate_gb), dev, 102)
    h = to_dev(wl["h"], "bf16", dev)
    idx = to_dev(wl["idx"], "i32", dev)
    sc = to_dev(wl["scores"], "f32", dev)
    rng = np.random.default_rng(1002)
    idx_np = [wl["idx"]] + [np.stack([rng.choice(256, 10, replace=False) for _ in range(8)]).astype(np.int32)
                            for _ in range(1, L)]
    idxs = [idx] + [torch.from_numpy(a).to(dev) for a in idx_np[1:]]
    distinct = [int(np.unique(a).size) for a in idx_np]
    y = torch.empty(8, 2048, dtype=torch.bfloat16, device=dev)
    tsets = [ops.repack_tiles(w, s, b) for (w, s, b) in sets]
    torch.cuda.synchronize()

    def mk(i):
        w, s, b = sets[i % len(sets)]
        ii = idxs[i]

        def f():
            ops._lib.call("qmoe_moe_down_wsum", h.data_ptr(), ii.data_ptr(), sc.data_ptr(), 8, 10, 512,
                          w.data_ptr(), s.data_ptr(), b.data_ptr(), 256, 2048, 64, 4, y.data_ptr(),
                          torch.cuda.current_stream().cuda_stream)
        return f

    def mk_tiles(i):
        tw = tsets[i % len(tsets)]
        ii = idxs[i]

        def f():
            ops._lib.call("qmoe_moe_down_wsum_tiles", h.data_ptr(), ii.data_ptr(), sc.data_ptr(), 8, 10, 512,
                          tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 2048, y.data_ptr(),
                          torch.cuda.current_stream().cuda_stream)
        return f

    # the floor of this launch shape (libqmoe_peaks.so): 10,240 waves in
    # ten-wave workgroups, each reading its pair's expert id, then its 16 rows
    # of codes (4 KiB) and their scales and biases, with no arithmetic
    P = peaks_lib()
    sink = torch.zeros(10240, dtype=torch.int32, device=dev)

    def mk_burst(i):
        w, s_, b_ = sets[i % len(sets)]
        ii = idxs[i]

        def f():
            rc = P.qmoe_peak_burst(ii.data_ptr(), 80, 256, w.data_ptr(), s_.data_ptr(), b_.data_ptr(), 2048, 256, 16,
                                   16, 10, sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"floor probe failed (code {rc})")
        return f

    mean_distinct = float(np.mean(distinct))
    row_bytes = 512 // 2 + 8 * 4
    bytes_ = int(mean_distinct * 2048 * row_bytes + 8 * 10 * 512 * 2 + 8 * 2048 * 2 + 8 * 10 * 4)
    return wl, [mk(i) for i in range(L)], {
        "bytes": bytes_, "flops": synth.algorithmic_flops(2, wl), "bound": "hbm",
        "kernel": "down_pair_kernel<16>", "sets": len(sets), "mean_distinct_experts": mean_distinct,
        "cycle_bytes": L * bytes_, "alt": ("tile_layout_us_per_call", [mk_tiles(i) for i in range(L)]),
        "floor": {"burst": [mk_burst(i) for i in range(L)], "burst_bytes": 80 * 2048 * (256 + 2 * 16)},
        "workload": "decode down + top-10 weighted sum: 8 tokens, I=512, D=2048, E=256, "
                    "W [256,2048,512] int4 g64 -> y [8,2048]"}


def _prefill_common(args, dev, cfg):
    import torch
    from titan_amd import ops, synth

    wl = synth.make(cfg)
    T, k = wl["idx"].shape
    x = to_dev(wl["x"], "bf16", dev)
    sets = weight_sets(wl, 2, dev, 100 + cfg)
    r = ops.route(to_dev(wl["idx"], "i32", dev), 256)
    lhs = torch.div(r.order, k, rounding_mode="floor").to(torch.int32)
    out = torch.empty(T * k, 1024, dtype=torch.bfloat16, device=dev)
    return wl, x, sets, r, lhs, out


def prefill_steps(args):
    """Steps per timed window of the prefill workloads (each call ~0.2 ms)."""
    return max(1, args.steps // 10)


def setup_cfg3(args, dev):
    import torch
    from titan_amd import ops, synth

    wl, x, sets, r, lhs, out = _prefill_common(args, dev, 3)
    t = r.tiles
    L = 2 * prefill_steps(args)  # two weight sets of 302 MB alternate: each call reads cold weights
    # load-time repack into the tile layout (outside the timed region)
    tsets = [ops.repack_tiles(w, s, b) for (w, s, b) in sets]
    torch.cuda.synchronize()

    def mk_tiles(i):
        tw = tsets[i % len(tsets)]

        def f():
            ops._lib.call("qmoe_gather_qmm_sorted_tiles", x.data_ptr(), lhs.data_ptr(), t.rows, 2048,
                          tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 1024, t.offsets.data_ptr(),
                          t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                          out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        return f

    def mk_mlx(i):
        w, s, b = sets[i % len(sets)]

        def f():
            ops._lib.call("qmoe_gather_qmm_sorted", x.data_ptr(), lhs.data_ptr(), t.rows, 2048, w.data_ptr(),
                          s.data_ptr(), b.data_ptr(), 256, 1024, 64, 4, t.offsets.data_ptr(),
                          t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                          out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        return f

    return wl, [mk_tiles(i) for i in range(L)], {
        "flops": synth.algorithmic_flops(3, wl), "bound": "mfma", "peak_tflops": BF16_PEAK_TFLOPS,
        "peak_key": "bf16_mfma_TFLOPs", "kernel": "gemm_bf16_kernel<true, false>", "sets": len(sets),
        "steps": prefill_steps(args),
        "alt": ("mlx_layout_us_per_call", [mk_mlx(i) for i in range(L)]),
        "workload": "prefill grouped GEMM: 4096 tokens x top-10 Zipf(1.1) routed rows sorted by expert, "
                    "gate_up W [256,1024,2048] int4 g64 (tile layout, repacked at load), x gathered "
                    "in-kernel -> [40960,1024]"}


def setup_cfg4(args, dev):
    import torch
    from titan_amd import ops, synth

    wl, x, sets, r, lhs, out = _prefill_common(args, dev, 4)
    t = r.tiles
    T = wl.meta["T"]
    xi = torch.empty(T, 2048, dtype=torch.int8, device=dev)
    sx = torch.empty(T, dtype=torch.float32, device=dev)
    L = 2 * prefill_steps(args)
    # load-time repack into the tile layout (outside the timed region)
    tsets = [ops.repack_tiles(w, s, b) for (w, s, b) in sets]
    torch.cuda.synchronize()

    def mk(i):
        tw = tsets[i % len(tsets)]

        def f():
            st = torch.cuda.current_stream().cuda_stream
            ops._lib.call("qmoe_quantize_act_int8", x.data_ptr(), T, 2048, xi.data_ptr(), sx.data_ptr(), st)
            ops._lib.call("qmoe_gather_qmm_int8_sorted_tiles", xi.data_ptr(), sx.data_ptr(), lhs.data_ptr(),
                          t.rows, 2048, tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 1024, t.offsets.data_ptr(),
                          t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                          out.data_ptr(), st)
        return f

    def mk_mlx(i):
        w, s, b = sets[i % len(sets)]

        def f():
            st = torch.cuda.current_stream().cuda_stream
            ops._lib.call("qmoe_quantize_act_int8", x.data_ptr(), T, 2048, xi.data_ptr(), sx.data_ptr(), st)
            ops._lib.call("qmoe_gather_qmm_int8_sorted", xi.data_ptr(), sx.data_ptr(), lhs.data_ptr(), t.rows,
                          2048, w.data_ptr(), s.data_ptr(), b.data_ptr(), 256, 1024, 64, 4,
                          t.offsets.data_ptr(), t.tile_row.data_ptr(), t.tile_exp.data_ptr(),
                          t.ntiles.data_ptr(), t.maxt, out.data_ptr(), st)
        return f

    # the down projection of the same 40960 routed rows (h [40960, 512] in
    # sorted order, W [256, 2048, 512]): int8 (quantiser + GEMM) against the
    # bf16 GEMM, as the reference reports both projections
    # (engine/patches/moe-int8/REPORT.md:230-239)
    rows = T * wl["idx"].shape[1]
    gen = torch.Generator(device=dev)
    gen.manual_seed(404)
    dsets = [ops.repack_tiles(random_like_words((256, 2048, 64), dev, gen), random_scales((256, 2048, 8), dev, gen),
                              random_biases((256, 2048, 8), dev, gen)) for _ in range(2)]
    h = (torch.randn(rows, 512, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    hi = torch.empty(rows, 512, dtype=torch.int8, device=dev)
    hs = torch.empty(rows, dtype=torch.float32, device=dev)
    yd = torch.empty(rows, 2048, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def mk_down(i, int8):
        tw = dsets[i % len(dsets)]

        def f():
            st = torch.cuda.current_stream().cuda_stream
            if int8:
                ops._lib.call("qmoe_quantize_act_int8", h.data_ptr(), rows, 512, hi.data_ptr(), hs.data_ptr(), st)
                ops._lib.call("qmoe_gather_qmm_int8_sorted_tiles", hi.data_ptr(), hs.data_ptr(), None, rows, 512,
                              tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 2048, t.offsets.data_ptr(),
                              t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                              yd.data_ptr(), st)
            else:
                ops._lib.call("qmoe_gather_qmm_sorted_tiles", h.data_ptr(), None, rows, 512, tw.wp.data_ptr(),
                              tw.sb.data_ptr(), 256, 2048, t.offsets.data_ptr(), t.tile_row.data_ptr(),
                              t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt, yd.data_ptr(), st)
        return f

    down_flops = 2 * rows * 2048 * 512
    return wl, [mk(i) for i in range(L)], {
        "extras": [("down_int8", [mk_down(i, True) for i in range(L)], down_flops),
                   ("down_bf16", [mk_down(i, False) for i in range(L)], down_flops)],
        "flops": synth.algorithmic_flops(4, wl), "bound": "mfma", "peak_tflops": INT8_PEAK_TOPS,
        "peak_key": "int8_mfma_TOPs", "kernel": "quant_act_kernel + gemm_int8_kernel<true>", "sets": len(sets),
        "steps": prefill_steps(args),
        "alt": ("mlx_layout_us_per_call", [mk_mlx(i) for i in range(L)]),
        "workload": "int8-activation x int4-weight gate_up prefill: 4096 tokens x top-10 Zipf(1.1), "
                    "per-token symmetric int8 x, W [256,1024,2048] int4 g64 (tile layout, repacked at load) "
                    "-> [40960,1024]"}


def setup_cfg5(args, dev):
    """Workload 0 with 8-bit codes (the small-M kernel's other bit width)."""
    import torch
    from titan_amd import ops, synth

    wl = synth.make(5)
    per_call = synth.algorithmic_bytes(5)
    L = cycle_len(args.steps, per_call, args.rotate_gb * 1e9)
    sets = weight_sets(wl, min(L, n_sets_needed(wl, L * per_call, args.rotate_gb)), dev, 105)
    x = to_dev(wl["x"], "bf16", dev)
    out = torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def mk(i):
        w, s, b = sets[i % len(sets)]

        def f():
            ops._lib.call("qmoe_quantized_matmul", x.data_ptr(), 1, 2048, w.data_ptr(), s.data_ptr(),
                          b.data_ptr(), 4096, 64, 8, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        return f

    return wl, [mk(i) for i in range(L)], {
        "bytes": per_call, "flops": synth.algorithmic_flops(5), "bound": "hbm",
        "kernel": "qmv64_kernel8<1, 2, 64, false, false>", "sets": len(sets), "cycle_bytes": min(L, len(sets)) * per_call,
        "workload": "dense quantized_matmul x [1,2048] . W [4096,2048] int8 codes g64"}


WIDTHS = (1, 2, 4, 6, 8, 16)


def run_widths(args, dev):
    """Decode widths: T tokens x top-10 of 256 experts through the gate_up +
    SwiGLU step two ways -- the decode GEMV (qmoe_moe_gate_up_swiglu) and the
    sorted path (qmoe_route + the SwiGLU-epilogue grouped GEMM) -- on the
    workload-1 weights.  GB/s counts each distinct expert's bytes once."""
    import torch
    from titan_amd import ops, synth

    wl = synth.make(1)
    sets = weight_sets(wl, n_sets_needed(wl, 0, args.rotate_gb), dev, 106)
    tsets = [ops.repack_tiles(w, s, b, swiglu_pairs=True) for (w, s, b) in sets]
    rng = np.random.default_rng(1006)
    per_expert = 2 * 512 * (2048 // 2 + 32 * 4)
    res = {}
    steps = max(8, args.steps // 2)
    for T in WIDTHS:
        x = to_dev(synth.bf16_bits(rng.normal(size=(T, 2048)).astype(np.float32)), "bf16", dev)
        n_idx = len(sets)
        idx_np = [np.stack([rng.choice(256, 10, replace=False) for _ in range(T)]).astype(np.int32)
                  for _ in range(n_idx)]
        idx = [torch.from_numpy(a).to(dev) for a in idx_np]
        distinct = float(np.mean([np.unique(a).size for a in idx_np]))
        h = torch.empty(T * 10, 512, dtype=torch.bfloat16, device=dev)
        routes = [ops.route(i, 256) for i in idx]
        lhs = [torch.div(r.order, 10, rounding_mode="floor").to(torch.int32) for r in routes]
        ws = torch.empty(max(int(ops._lib.load().qmoe_route_workspace_size(T * 10, 256)), 256) // 4,
                         dtype=torch.int32, device=dev)
        torch.cuda.synchronize()

        def mk_dec(i, T=T, x=x, idx=idx, h=h):
            w, s, b = sets[i % len(sets)]
            ix = idx[i % len(sets)]

            def f():
                ops._lib.call("qmoe_moe_gate_up_swiglu", x.data_ptr(), ix.data_ptr(), T, 10, 2048, w.data_ptr(),
                              s.data_ptr(), b.data_ptr(), 256, 512, 64, 4, h.data_ptr(),
                              torch.cuda.current_stream().cuda_stream)
            return f

        def mk_sorted(i, T=T, x=x, h=h, ws=ws):
            j = i % len(sets)
            tw, r, lh = tsets[j], routes[j], lhs[j]
            t = r.tiles
            flat = idx[j].reshape(-1)

            def f():
                st = torch.cuda.current_stream().cuda_stream
                ops._lib.call("qmoe_route", flat.data_ptr(), T * 10, 256, t.tile_rows, r.order.data_ptr(),
                              r.inv_order.data_ptr(), r.sorted_ids.data_ptr(), t.offsets.data_ptr(),
                              t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                              ws.data_ptr(), ws.numel() * 4, st)
                ops._lib.call("qmoe_gather_qmm_swiglu_sorted_tiles", x.data_ptr(), lh.data_ptr(), T * 10, 2048,
                              tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 1024, t.offsets.data_ptr(),
                              t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                              h.data_ptr(), st)
            return f

        L = steps * int(np.ceil(len(sets) / steps))
        sec_d, _ = timer(args)([mk_dec(i) for i in range(L)], steps, args.warmup, dev)
        sec_s, _ = timer(args)([mk_sorted(i) for i in range(L)], steps, args.warmup, dev)
        nbytes = distinct * per_expert + T * 2048 * 2 + T * 10 * 512 * 2
        res[T] = {"pairs": T * 10, "distinct_experts": distinct, "decode_us": round(sec_d * 1e6, 3),
                  "decode_GBps": round(nbytes / sec_d / 1e9, 1), "sorted_us": round(sec_s * 1e6, 3),
                  "sorted_GBps": round(nbytes / sec_s / 1e9, 1),
                  "faster": "decode" if sec_d <= sec_s else "sorted"}
        print(f"[bench] width T={T}: {res[T]}", file=sys.stderr, flush=True)
        del routes, lhs, idx
    return {"workload": "decode widths: T tokens x top-10 of E=256, gate_up + SwiGLU, W [256,1024,2048] int4 g64; "
                        "decode GEMV vs route + SwiGLU grouped GEMM",
            "kernel": "qmv64_flat_kernel<1, 64, 4> (T = 1), qmv64_kernel<1, 0, 1, 4, 64, true, false> (T > 1) | route_* + gemm_bf16_kernel<true, true>",
            "widths": res}


def run_block(args, dev):
    """The whole routed MoE block (titan_amd.moe_block.SparseMoeBlock) as one
    call: router logits, top-k, then the decode kernels (T = 1) or routing
    sort + SwiGLU GEMM + down GEMM + weighted sum (T = 4096), E = 256,
    H = 2048, I = 512, top-10, random weights rotated over several blocks."""
    import torch
    from titan_amd import moe_block, synth

    gen = torch.Generator(device=dev)
    gen.manual_seed(107)

    def block(resident="tiles"):
        gu = (random_like_words((256, 1024, 256), dev, gen), random_scales((256, 1024, 32), dev, gen),
              random_biases((256, 1024, 32), dev, gen))
        dn = (random_like_words((256, 2048, 64), dev, gen), random_scales((256, 2048, 8), dev, gen),
              random_biases((256, 2048, 8), dev, gen))
        router = (torch.randn(256, 2048, device=dev, generator=gen) * 0.05).to(torch.bfloat16)
        return moe_block.SparseMoeBlock(router, gu, dn, 10, resident=resident)

    rng = np.random.default_rng(1007)
    res = {}
    per_gu, per_dn = 1024 * (1024 + 32 * 4), 2048 * (256 + 8 * 4)
    for T, nblocks in ((1, 4), (4096, 2)):
        blocks = [block() for _ in range(nblocks)]
        x = to_dev(synth.bf16_bits(rng.normal(size=(T, 2048)).astype(np.float32)), "bf16", dev)
        torch.cuda.synchronize()
        steps = args.steps if T == 1 else prefill_steps(args)
        L = steps * int(np.ceil(nblocks / steps))
        fns = [(lambda b=blocks[i % nblocks]: b(x)) for i in range(L)]
        sec, tinfo = timer(args)(fns, steps, args.warmup if T == 1 else 2, dev)
        r = {"us_per_call": round(sec * 1e6, 3), "us_per_call_min": round(tinfo["min"] * 1e6, 3)}
        if T == 1:
            nbytes = 256 * 2048 * 2 + 10 * (per_gu + per_dn) + 2048 * 2 * 2
            r.update(metric="HBM GB/s", value=round(nbytes / sec / 1e9, 1), bytes_per_call=nbytes,
                     pct_hbm_peak=round(100 * nbytes / sec / 1e9 / HBM_PEAK_GBS, 2),
                     path="router logits + gate_up/SwiGLU GEMV selecting its experts (top-k in-kernel) "
                          "+ down/weighted-sum GEMV")
        else:
            fl = 2 * T * 10 * 2048 * 1024 + 2 * T * 10 * 512 * 2048 + 2 * T * 2048 * 256
            r.update(metric="TFLOP/s", value=round(fl / sec / 1e12, 1), flops_per_call=fl,
                     pct_bf16_peak=round(100 * fl / sec / 1e12 / BF16_PEAK_TFLOPS, 2),
                     path="router + top-k + route + SwiGLU GEMM + down GEMM + weighted sum")
        r["resident"] = "tiles (one copy)"
        res[T] = r
        print(f"[bench] block T={T}: {r}", file=sys.stderr, flush=True)
        del blocks, fns, tinfo
        torch.cuda.empty_cache()
        if T == 1:
            # the same decode with the MLX tensors kept too (resident="both")
            blocks = [block("both") for _ in range(nblocks)]
            fns = [(lambda b=blocks[i % nblocks]: b(x)) for i in range(L)]
            sec_b, _ = timer(args)(fns, steps, args.warmup, dev)
            res[T]["us_per_call_resident_both"] = round(sec_b * 1e6, 3)
            del blocks, fns
            torch.cuda.empty_cache()
    return {"workload": "whole MoE block, E=256, H=2048, I=512, top-10, int4 g64 (tile layout for prefill)",
            "tokens": res}


SETUPS = {0: setup_cfg0, 1: setup_cfg1, 2: setup_cfg2, 3: setup_cfg3, 4: setup_cfg4, 5: setup_cfg5}


def decode_phases(args, dev, samples=16):
    """Workload 1 through the measurement build libqmoe_stamps.so, whose one-token
    decode GEMV writes s_memrealtime stamps (10 ns ticks) per block: entry, kernel
    arguments ready, expert id ready, first weight row consumed, all rows
    consumed and reduced, output store acknowledged.  The cycle is replayed
    as time_graph does; after each of `samples` window replays the stamps of
    that window's last launch are read.  Returns percentiles per phase (us)."""
    import ctypes

    import torch
    from titan_amd import _lib, build as tbuild, synth

    base = _lib.load()
    L = ctypes.CDLL(str(tbuild.STAMPS_LIB))
    fn = L.qmoe_moe_gate_up_swiglu
    fn.restype, fn.argtypes = ctypes.c_int, base.qmoe_moe_gate_up_swiglu.argtypes
    rd = L.qmoe_qmv_stamps_read
    rd.restype, rd.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64]
    wl, cycle, meta = setup_cfg1(args, dev)
    # the same launches (weights, ids, outputs) through the stamped library
    x = to_dev(wl["x"], "bf16", dev)
    sets = weight_sets(wl, meta["sets"], dev, 101)
    rng = np.random.default_rng(1001)
    idxs = [torch.from_numpy(rng.permutation(256)[:10].astype(np.int32)[None]).to(dev) for _ in cycle]
    out = torch.empty(1, 10, 512, dtype=torch.bfloat16, device=dev)

    def mk(i):
        w, s_, b = sets[i % len(sets)]
        ix = idxs[i]

        def f():
            rc = fn(x.data_ptr(), ix.data_ptr(), 1, 10, 2048, w.data_ptr(), s_.data_ptr(), b.data_ptr(), 256, 512,
                    64, 4, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"stamped qmoe_moe_gate_up_swiglu failed ({rc})")
        return f

    stamped = [mk(i) for i in range(len(cycle))]
    sec, tinfo = time_graph(stamped, args.steps, args.warmup, dev)
    sec_prod, _ = time_graph(cycle, args.steps, args.warmup, dev)
    nb = 1024  # blocks of one launch: 10 experts x 512 gate/up row pairs / 5 (the flat one-token kernel)
    names = ["entry", "args", "id", "first_row", "reduced", "stored"]
    buf = np.zeros(nb * len(names), np.uint64)
    rows = []
    graphs = tinfo["graphs"]
    for k in range(samples):
        graphs[k % len(graphs)].replay()
        torch.cuda.synchronize()
        if rd(buf.ctypes.data, buf.size) != 0:
            raise RuntimeError("qmoe_qmv_stamps_read failed")
        rows.append(buf.reshape(nb, len(names)).astype(np.int64).copy())
    tick_us = 0.01  # s_memrealtime runs at 100 MHz
    pct = (0, 10, 50, 90, 100)

    def q(v):
        return [round(float(a), 3) for a in np.percentile(np.concatenate(v), pct)]

    t0 = [r[:, 0] - r[:, 0].min() for r in rows]
    res = {
        "percentiles": list(pct),
        "launch_offset_us": q([v * tick_us for v in t0]),
        "args_wait_us": q([(r[:, 1] - r[:, 0]) * tick_us for r in rows]),
        "id_wait_us": q([(r[:, 2] - r[:, 1]) * tick_us for r in rows]),
        "first_weight_row_us": q([(r[:, 3] - r[:, 2]) * tick_us for r in rows]),
        "other_rows_and_reduce_us": q([(r[:, 4] - r[:, 3]) * tick_us for r in rows]),
        "store_ack_us": q([(r[:, 5] - r[:, 4]) * tick_us for r in rows]),
        "block_end_offset_us": q([(r[:, 5] - r[:, 0].min()) * tick_us for r in rows]),
        "dispatch_span_us": q([np.array([(r[:, 5].max() - r[:, 0].min()) * tick_us]) for r in rows]),
        "stamped_us_per_call": round(sec * 1e6, 3),
        "product_us_per_call": round(sec_prod * 1e6, 3),
        "samples": samples,
        "workload": meta["workload"],
        "note": "stamps in 10 ns ticks, lane 0 of each of the flat kernel's 1024 waves (four per workgroup)",
    }
    return res


def gemm_units(args, dev, samples=8):
    """Workload 3's grouped GEMM through the measurement build
    libqmoe_stamps.so, whose persistent blocks record s_memrealtime (10 ns
    ticks) before and after each (tile, column block) unit.  Per subtile
    count: units and median unit time, split by the block's half of the grid
    (the first P/2 blocks are dispatched first, one per CU, so each CU holds
    one of each); the blocks' end times and busy times; the kernel span."""
    import ctypes

    import torch
    from titan_amd import _lib, build as tbuild, ops

    base = _lib.load()
    L = ctypes.CDLL(str(tbuild.STAMPS_LIB))
    fn = L.qmoe_gather_qmm_sorted_tiles
    fn.restype, fn.argtypes = ctypes.c_int, base.qmoe_gather_qmm_sorted_tiles.argtypes
    rd = L.qmoe_gemm_stamps_read
    rd.restype, rd.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    nu = int(L.qmoe_gemm_stamp_units())
    wl, x, sets, r, lhs, out = _prefill_common(args, dev, 3)
    t = r.tiles
    tsets = [ops.repack_tiles(w, s_, b) for (w, s_, b) in sets]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    units_max = t.maxt * (1024 // 256)
    P = min((2 * cus + 7) // 8 * 8, max(8, (units_max + 7) // 8 * 8))

    def launch(i):
        tw = tsets[i % len(tsets)]
        rc = fn(x.data_ptr(), lhs.data_ptr(), t.rows, 2048, tw.wp.data_ptr(), tw.sb.data_ptr(), 256, 1024,
                t.offsets.data_ptr(), t.tile_row.data_ptr(), t.tile_exp.data_ptr(), t.ntiles.data_ptr(), t.maxt,
                out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"stamped qmoe_gather_qmm_sorted_tiles failed ({rc})")

    for i in range(4):
        launch(i)
    torch.cuda.synchronize()
    times = np.zeros(P * nu * 2, np.uint64)
    uinfo = np.zeros(P * nu * 2, np.int32)
    counts = np.zeros(P, np.int32)
    recs, spans, ends_all, busy_all = [], [], [], []
    for k in range(samples):
        launch(k)
        torch.cuda.synchronize()
        if rd(times.ctypes.data, uinfo.ctypes.data, counts.ctypes.data, P) != 0:
            raise RuntimeError("qmoe_gemm_stamps_read failed")
        if counts.max() > nu:
            raise RuntimeError(f"a block ran {counts.max()} units, more than the {nu} recorded")
        tt = times.reshape(P, nu, 2).astype(np.int64)
        ui = uinfo.reshape(P, nu, 2)
        live = np.arange(nu)[None, :] < counts[:, None]
        t0 = tt[..., 0][live].min()
        blk = np.repeat(np.arange(P)[:, None], nu, axis=1)[live]
        d = (tt[..., 1] - tt[..., 0])[live] * 0.01
        msub = (ui[..., 1][live] + 31) // 32
        recs.append((blk, d, msub))
        end = np.where(live, tt[..., 1], 0).max(axis=1)
        ran = counts > 0
        ends_all.append((end[ran] - t0) * 0.01)
        busy_all.append(np.where(live, tt[..., 1] - tt[..., 0], 0).sum(axis=1)[ran] * 0.01)
        spans.append((end[ran].max() - t0) * 0.01)
    blk = np.concatenate([r_[0] for r_ in recs])
    d = np.concatenate([r_[1] for r_ in recs])
    ms = np.concatenate([r_[2] for r_ in recs])
    first = blk < P // 2
    per = {}
    for m in range(1, 5):
        sel = ms == m
        if sel.any():
            per[str(m)] = {"units_per_launch": int(sel.sum() // samples),
                           "median_us_first_half": round(float(np.median(d[sel & first])), 2) if (sel & first).any() else None,
                           "median_us_second_half": round(float(np.median(d[sel & ~first])), 2) if (sel & ~first).any() else None}
    pct = (0, 10, 50, 90, 100)
    ends = np.concatenate(ends_all)
    busy = np.concatenate(busy_all)
    return {"workload": "workload 3 (prefill bf16 grouped GEMM, 4096 tokens)", "blocks": P, "samples": samples,
            "unit_us_by_subtiles": per,
            "percentiles": list(pct),
            "block_end_us": [round(float(v), 1) for v in np.percentile(ends, pct)],
            "block_busy_us": [round(float(v), 1) for v in np.percentile(busy, pct)],
            "span_us_median": round(float(np.median(spans)), 1),
            "busy_fraction_of_span": round(float(busy.mean() / np.median(spans)), 3),
            "note": "eager launches of the stamped kernel; unit time from before the unit to after its "
                    "epilogue stores are issued (lane 0 of the block); first half = blocks 0..P/2-1"}


# ------------------------------------------------------------- CPU baseline


def cpu_threads():
    """Threads the CPU legs use: this process's CPU affinity, capped by
    OMP_NUM_THREADS when that is set (the host's share of cores)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def cpu_baseline(cfg, wl, budget_s):
    """The oracle (C, OpenMP, fp64 accumulation) on the same seeded inputs,
    timed on this host; the prefill workloads on a sample of their routed rows."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from titan_amd import synth

    oracle.build()
    nt = cpu_threads()
    if cfg == 1:
        def run():
            gu, _ = oracle.gather_qmm_rows(wl["x"], np.zeros(10, np.int32), wl["idx"].reshape(-1), wl["w"],
                                           wl["s"], wl["b"], n_threads=nt)
            oracle.swiglu(gu)
        work, unit, scale = synth.algorithmic_bytes(1), "GB/s", 1e9
        sample = "full workload: 10 experts x 1024 rows x 2048 + SwiGLU"
    elif cfg == 0:
        def run():
            oracle.gather_qmm_rows(wl["x"], None, np.zeros(1, np.int32), wl["w"][None], wl["s"][None],
                                   wl["b"][None], n_threads=nt)
        work, unit, scale = synth.algorithmic_bytes(0), "GB/s", 1e9
        sample = "full workload: 4096 rows x 2048"
    elif cfg == 2:
        def run():
            oracle.down_wsum(wl["h"], wl["idx"], wl["scores"], wl["w"], wl["s"], wl["b"], n_threads=nt)
        work, unit, scale = synth.algorithmic_bytes(2, wl), "GB/s", 1e9
        sample = "full workload: 8 tokens x 10 experts x 2048 rows x 512 + weighted sum"
    elif cfg in (3, 4):
        T, k = wl["idx"].shape
        rows = np.random.default_rng(cfg).choice(T * k, size=256, replace=False)
        order, _, srt = oracle.route_sort(wl["idx"], 256)
        xr = (order[rows] // k).astype(np.int32)
        ex = srt[rows]
        if cfg == 3:
            def run():
                oracle.gather_qmm_rows(wl["x"], xr, ex, wl["w"], wl["s"], wl["b"], deq="bf16", n_threads=nt)
            sample = "256 of the 40960 routed rows x 1024 columns x 2048 (bf16-dequantised weights)"
        else:
            toks = np.unique(xr)

            def run():
                xi, sx = oracle.quant_act_int8(wl["x"][toks])
                remap = np.searchsorted(toks, xr).astype(np.int32)
                oracle.gather_qmm_int8_rows(xi, sx, remap, ex, wl["w"], wl["s"], wl["b"], n_threads=nt)
            sample = "256 of the 40960 routed rows x 1024 columns x 2048, with their tokens' int8 quantisation"
        work, unit, scale = 2 * 256 * 1024 * 2048, "TFLOP/s" if cfg == 3 else "TOP/s", 1e12
    else:
        return None
    run()
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= 1000:
            break
    per = el / reps
    return {"value": round(work / per / scale, 4), "unit": unit, "cores": nt, "kind": "port",
            "affinity_cores": len(os.sched_getaffinity(0)),
            "sample": f"{sample}; {reps} repetitions in {el:.1f} s; {per * 1e3:.3f} ms per call",
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------- main


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this path runs on one GPU; --gpus must be 1 (expert-parallel "
                                   "sharding over several GPUs is not built)"}))
        return 2
    traffic = None
    if args.traffic and args.only is None:
        traffic = measure_traffic_live()  # child processes, before this one touches the GPU
    import torch
    from titan_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    cfgs = [int(c) for c in args.configs.split(",") if c != ""]
    if args.only == "copy":
        calibration_copy(dev)
        return 0
    if args.only is not None:
        cfgs = [int(args.only)]
    if args.decode_phases:
        print(json.dumps({"decode_phases": decode_phases(args, dev)}))
        return 0
    if args.gemm_units:
        print(json.dumps({"gemm_units": gemm_units(args, dev)}))
        return 0
    peaks = None
    if args.only is None and not args.no_peaks:
        print("[bench] measured peaks", file=sys.stderr, flush=True)
        peaks = measure_peaks(dev, power_seconds=args.power)
        print(f"[bench] peaks: {peaks}", file=sys.stderr, flush=True)
    results = {}
    head = None
    wls = {}
    for cfg in cfgs:
        print(f"[bench] workload {cfg}: setup", file=sys.stderr, flush=True)
        if cfg in (6, 7):
            results[cfg] = (run_widths if cfg == 6 else run_block)(args, dev)
            torch.cuda.empty_cache()
            continue
        wl, cycle, meta = SETUPS[cfg](args, dev)
        wls[cfg] = wl
        steps = meta.get("steps", args.steps)
        print(f"[bench] workload {cfg}: timing {len(cycle)} launches in windows of {steps}", file=sys.stderr,
              flush=True)
        sec, tinfo = timer(args)(cycle, steps, args.warmup, dev)
        res = {"workload": meta["workload"], "us_per_call": round(sec * 1e6, 3),
               "us_per_call_min": round(tinfo["min"] * 1e6, 3), "us_per_call_max": round(tinfo["max"] * 1e6, 3),
               "timed_rounds": tinfo["rounds"], "steps_per_round": steps, "cycle_launches": len(cycle),
               "kernel": meta["kernel"], "weight_sets": meta["sets"]}
        if "events_per_step" in tinfo:
            # the same replays timed by events around each window's graph launch
            res["us_per_call_with_graph_launch"] = round(tinfo["events_per_step"] * 1e6, 3)
        if meta["bound"] == "hbm":
            gbs = meta["bytes"] / sec / 1e9
            res.update(metric="HBM GB/s", value=round(gbs, 1), bytes_per_call=meta["bytes"],
                       pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 2),
                       touched_bytes_per_round=int(steps * meta["bytes"]),
                       rotation_bytes_per_cycle=int(meta["cycle_bytes"]))
            if peaks:
                res["pct_measured_hbm_read"] = round(100 * gbs / peaks["hbm_read_GBps"], 2)
        else:
            tf = meta["flops"] / sec / 1e12
            res.update(metric="TFLOP/s" if cfg == 3 else "TOP/s", value=round(tf, 1),
                       flops_per_call=meta["flops"], pct_peak=round(100 * tf / meta["peak_tflops"], 2),
                       pct_bf16_peak=round(100 * tf / BF16_PEAK_TFLOPS, 2))
            if peaks:
                res["pct_measured_peak"] = round(100 * tf / peaks[meta["peak_key"]], 2)
        for k_ in ("mean_distinct_experts",):
            if k_ in meta:
                res[k_] = meta[k_]
        if "alt" in meta:
            label, alt = meta["alt"]
            sec_alt, _ta = timer(args)(alt, steps, args.warmup, dev)
            res[label] = round(sec_alt * 1e6, 3)
            del alt, _ta
        if "floor" in meta:
            fl = meta.pop("floor")
            res["floor"] = {}
            if "launch" in fl:
                sec_l, _tl = timer(args)(fl["launch"], steps, args.warmup, dev)
                sec_c, _tc = timer(args)(fl["chain"], steps, args.warmup, dev)
                res["floor"].update(launch_us=round(sec_l * 1e6, 3), chain_us=round(sec_c * 1e6, 3),
                                    chain_bytes=fl["chain_bytes"])
                del _tl, _tc
            for wpb, (wl_, wc_) in fl.get("wider", {}).items():
                sl_, _x = timer(args)(wl_, steps, args.warmup, dev)
                sc_, _y = timer(args)(wc_, steps, args.warmup, dev)
                res["floor"][f"waves_per_block_{wpb}"] = {"launch_us": round(sl_ * 1e6, 3),
                                                          "chain_us": round(sc_ * 1e6, 3)}
                del _x, _y
            if "burst" in fl:
                sb_, _z = timer(args)(fl["burst"], steps, args.warmup, dev)
                res["floor"]["burst_us"] = round(sb_ * 1e6, 3)
                res["floor"]["burst_bytes"] = fl["burst_bytes"]
                res["floor"]["frac_of_burst"] = round(sb_ / sec, 4)
                del _z
            del fl
        for label, ex, ex_flops in meta.get("extras", ()):
            sec_ex, _te = timer(args)(ex, steps, args.warmup, dev)
            res[label] = {"us_per_call": round(sec_ex * 1e6, 3), "TOP/s": round(ex_flops / sec_ex / 1e12, 1),
                          "flops_per_call": ex_flops}
            del ex, _te
        if args.power > 0:
            graphs = tinfo.get("graphs")

            def run_once(graphs=graphs, cycle=cycle):
                if graphs:
                    for g in graphs:
                        g.replay()
                else:
                    for fn in cycle:
                        fn()
            res["power"] = sample_power(run_once, args.power)
            print(f"[bench] workload {cfg} power: {res['power']}", file=sys.stderr, flush=True)
        results[cfg] = res
        print(f"[bench] workload {cfg}: {res}", file=sys.stderr, flush=True)
        if cfg == 1:
            head = (wl, meta, sec)
        del cycle, tinfo
        torch.cuda.empty_cache()
    if args.only is not None:
        return 0
    peaks_after = None
    if peaks is not None:
        peaks_after = measure_peaks(dev)
        print(f"[bench] peaks after the workloads: {peaks_after}", file=sys.stderr, flush=True)
    if head is None:
        print(json.dumps({"configs": results, "peaks_measured": peaks}))
        return 0
    wl, meta, sec = head
    gbs = meta["bytes"] / sec / 1e9
    if traffic is None:
        traffic = traffic_from_profile()
    cpu, cpu_rows = None, {}
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(1, wl, args.cpu_seconds)
        for c in (0, 2, 3, 4):
            if c in cfgs:
                cpu_rows[c] = cpu_baseline(c, wls[c], args.cpu_seconds / 3)
                print(f"[bench] cpu baseline {c}: {cpu_rows[c]}", file=sys.stderr, flush=True)
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None if traffic is None else round(traffic["bytes"]),
            "kernel": TRAFFIC_KERNEL, "bytes_per_launch": meta["bytes"], "traffic_detail": traffic}
    if peaks:
        roof["peak_measured"] = peaks["hbm_read_GBps"]
        roof["frac_measured"] = round(gbs / peaks["hbm_read_GBps"], 4)
    fl = results.get(1, {}).get("floor")
    if fl is not None:
        # per-call floor of one launch that must learn its experts before
        # asking for their weights: the chain probe (launch, arguments, expert
        # id, first row, store) at the kernel's four waves per workgroup, plus
        # the remaining bytes at the measured read rate
        floor = dict(fl)
        if peaks:
            chain_us = fl.get("waves_per_block_4", {}).get("chain_us", fl["chain_us"])
            stream_us = (meta["bytes"] - fl["chain_bytes"]) / (peaks["hbm_read_GBps"] * 1e3)
            floor["stream_rest_us"] = round(stream_us, 3)
            floor["model_chain_us"] = chain_us
            floor["model_us"] = round(chain_us + stream_us, 3)
            floor["frac_of_model"] = round((chain_us + stream_us) / (sec * 1e6), 4)
        if "burst_us" in fl:
            # the same ids-then-weights memory work measured as one launch
            floor["frac_of_burst"] = round(fl["burst_us"] / (sec * 1e6), 4)
        roof["floor"] = floor
    line = {
        "metric": METRIC,
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": meta["workload"], "tokens": 1, "top_k": 10, "experts": 256, "hidden": 2048,
                   "intermediate": 512, "group_size": 64, "bits": 4, "weight_sets_rotated": meta["sets"],
                   "timing": "median per step over the timed windows of exactly `steps` launches"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "cpu_baseline_configs": cpu_rows,
        "peaks_measured": {"before": peaks, "after": peaks_after},
        "configs": results,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

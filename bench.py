#!/usr/bin/env python3
"""Forward-latency benchmark of the MI355X transformer-block path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]``

One step = one ``UserOptimizedTransformer.forward(x)`` call on the workload
(input copy into the captured graph's static buffer, hipGraph replay of the
layers, the final LayerNorm into a new output tensor), the unit the reference
times in ``benchmark_once`` (TTB:4824-4855).  The headline workload is
BASELINE.json's ``configs[1]`` (c2, fp16, "p50 latency over 1000 graph
replays"), so the default is K=1000 timed steps after W=20 warmups, each
bracketed by HIP events; ``value`` is their p50 in ms.

The same JSON line carries
* ``per_config`` (c1-c5): the reference's timing protocol (TTB:4857-4930):
  warmups, then ``--rounds`` rounds alternating the eager oracle on the same
  GPU with this build (the order flips every round), each round
  ``repeats`` event-timed calls; median / mean / p90 / min and tokens/s of
  both (``TimingResult``, TTB:4774-4822).  c2 runs 1000 replays and reports
  the replay time of an empty graph beside them (agent/tools/microbench.py:
  84-101).  Then FLOPs by the reference formula (run_bench.py:102-113),
  TFLOP/s and the fraction of the MI355X dense MFMA peak, the per-kernel
  times of exactly the launches the forward makes (recorded from the
  forward itself), and the eager oracle on the host cores (``cpu_baseline``,
  bounded sample, method stated);
* ``geomean_speedup_vs_eager_gpu_c2_c4``: the reference's headline
  statistic (geomean of eager-baseline median / this build's median);
* ``roofline``: the dominant kernel of the headline workload, its
  algorithmic FLOPs (or bytes) per launch over its average duration, timed
  with HIP events on the stream it is launched on;
* ``cpu_baseline``: the eager oracle on the host cores for the headline;
* ``range_ms`` / ``comparison``: the headline is measured ``--runs`` times
  (the first run is ``value``) and each config over ``--rounds`` alternating
  rounds; min / median / max of the per-run medians, and against the newest
  committed ``BENCH_rNN.json`` a verdict that counts only non-overlapping
  ranges (agent/tools/bench.py:78-119);
* ``provenance``: source hash and git head (from the checkout, or on a copy
  without git from the build record next to the library), torch / HIP
  versions, the device, the host CPU model and thread budget, the device's
  busy %, clocks, power and temperature before and after (amdgpu sysfs), an
  idle gate -- the run waits until the device has been below 10% busy for
  5 s and refuses to measure (exit status 3) if it is not within
  ``--idle-timeout-s`` -- and a sampler that marks the record untrusted if
  another compute process appears on the device while it measures
  (run_bench.py:314-532; agent/tools/_common.py:71-131, 217-311).  Nothing
  is forked once the GPU is initialised (git runs before).

Synthetic data: weights N(0, 0.02) from seed 0, x ~ N(0, 1) from seed 1
(transformer_optimization_amd/workloads.py).  One GPU only.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from transformer_optimization_amd import UserOptimizedTransformer, _C, workloads  # noqa: E402
from transformer_optimization_amd.flops import (  # noqa: E402
    MI355X_HBM_BYTES_PER_S, MI355X_PEAK_FLOPS, EXECUTED_PRECISION,
    attention_flops, count_dense_flops, gemm_flops,
)

# The reference CLI's defaults (TTB:5044-5060): 3 alternating rounds.
ROUNDS = 3
# Calls per round and config: c2 reaches 1000 replays over the rounds.
REPEATS = {"c1": 100, "c2": 334, "c3": 10, "c4": 8, "c5": 4}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_model(wl, dev):
    """The workload's model with default attributes (it picks its own numeric
    policy, as a caller of the drop-in API gets it)."""
    model = UserOptimizedTransformer(wl.config)
    workloads.init_parameters(model)
    model = model.to(dev, wl.dtype).eval()
    x = workloads.make_input(wl.config, wl.dtype).to(dev)
    return model, x


# ------------------------------------------------------------------- timing
def percentile(values, q: float) -> float:
    """Linear-interpolated percentile (TTB:4786-4799)."""
    ordered = sorted(values)
    if len(ordered) == 1:
        return ordered[0]
    pos = (len(ordered) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    if lo == hi:
        return ordered[lo]
    return ordered[lo] * (1.0 - (pos - lo)) + ordered[hi] * (pos - lo)


def summarize(samples, tokens: int):
    """TimingResult's statistics (TTB:4802-4822) plus tokens/s at the median."""
    med = statistics.median(samples)
    return {"n": len(samples), "median_ms": round(med, 5), "mean_ms": round(statistics.fmean(samples), 5),
            "p90_ms": round(percentile(samples, 0.9), 5), "min_ms": round(min(samples), 5),
            "tokens_per_s": round(tokens * 1000.0 / med, 1)}


def benchmark_once(model, x, iterations: int):
    """Per-call HIP-event timings (ms) on the current stream (TTB:4824-4846)."""
    with torch.inference_mode():
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
        torch.cuda.synchronize()
        for i in range(iterations):
            starts[i].record()
            model(x)
            ends[i].record()
        torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def warmup_model(model, x, iterations: int) -> None:
    with torch.inference_mode():
        for _ in range(iterations):
            model(x)
    torch.cuda.synchronize()


def benchmark_pair(baseline, ours, x, rounds: int, repeats: int, warmup: int):
    """Alternating rounds (TTB:4893-4907): baseline first in even rounds,
    this build first in odd ones.  baseline None: this build only.  Returns
    the per-round sample lists of both."""
    if baseline is not None:
        warmup_model(baseline, x, warmup)
    warmup_model(ours, x, warmup)
    base_r, ours_r = [], []
    for r in range(rounds):
        if baseline is not None and r % 2 == 0:
            base_r.append(benchmark_once(baseline, x, repeats))
        ours_r.append(benchmark_once(ours, x, repeats))
        if baseline is not None and r % 2 == 1:
            base_r.append(benchmark_once(baseline, x, repeats))
    return base_r, ours_r


def range_of(per_run):
    """min / median / max of the per-run medians (agent/tools/_common.py:330+)."""
    meds = [statistics.median(r) for r in per_run]
    return {"runs": len(meds), "min": round(min(meds), 5), "median": round(statistics.median(meds), 5),
            "max": round(max(meds), 5), "per_run_median_ms": [round(m, 5) for m in meds]}


def empty_graph_replay_us(replays: int = 1000):
    """Replay time of a graph with no device work: the scheduling cost every
    replay carries (agent/tools/microbench.py:84-101)."""
    try:
        g = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(g):
            pass
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        e1.synchronize()
        return round(e0.elapsed_time(e1) * 1000.0 / replays, 3)
    except RuntimeError as exc:  # an empty capture may be refused by the runtime
        log(f"[bench] empty graph replay not measurable: {exc}")
        return None


def config_record(wl):
    c = wl.config
    return {"workload": wl.name, "batch": c.batch_size, "seq_len": c.seq_len,
            "d_model": c.d_model, "heads": c.num_heads, "head_dim": c.d_model // c.num_heads,
            "layers": c.num_layers, "ffn_dim": c.ffn_dim, "causal": c.causal,
            "dtype": wl.dtype_name}


def mfu_fields(wl, ms):
    c = wl.config
    flops = count_dense_flops(c.batch_size, c.seq_len, c.d_model, c.ffn_dim, c.num_layers)
    peak = MI355X_PEAK_FLOPS[EXECUTED_PRECISION[wl.dtype_name]]
    tflops = flops / (ms / 1e3) / 1e12
    return {"gflop": round(flops / 1e9, 3), "tflop_s": round(tflops, 2),
            "mfu": round(tflops * 1e12 / peak, 4)}


# --------------------------------------------------------------- per-kernel
# Wrapper calls per layer of _forward_layers, in order (every policy).
LAYER_SCHEDULE = ("layernorm", "qkv_proj", "flash_attn", "gemm_out_proj", "layernorm_2",
                  "gemm_ffn_in_gelu", "gemm_ffn_out")


def forward_launches(model, x):
    """The launches of one forward, recorded from the forward itself:
    ``[(name, launch, work, unit, executed_work, launches_per_forward)]`` for
    layer 0's seven calls and the final LayerNorm.  ``work`` is the
    algorithmic FLOPs (mfma) or bytes (hbm) of one launch; ``executed_work``
    differs where the fp32-residual policy feeds a GEMM a hi/lo operand pair
    (K doubled)."""
    cfg = model.config
    policy = model.resolve_policy(x.shape[1], x.dtype, x.device)
    with _C.record_launches() as rec, torch.inference_mode():
        model._refresh_derived()
        model._forward_core(x, None, policy)
    torch.cuda.synchronize()
    per_layer = len(LAYER_SCHEDULE)
    if len(rec) != per_layer * cfg.num_layers + 1:
        raise RuntimeError(f"unexpected launch count {len(rec)} for {cfg.num_layers} layers")
    picked = list(zip(LAYER_SCHEDULE, rec[:per_layer])) + [("layernorm_final", rec[-1])]
    out = []
    for name, ln in picked:
        i = ln.info
        if i["op"] == "layernorm":
            split = 2 if i["flags"] & _C.LN_SPLIT_Y else 1
            work = i["rows"] * i["d"] * (i["x_bytes"] + split * i["y_bytes"]) + 2 * i["d"] * i["param_bytes"]
            executed, unit = work, "hbm"
        elif i["op"] in ("gemm", "qkv_proj"):
            executed = gemm_flops(i["m"], i["n"], i["k"])
            two_term = policy[1] == "fp32_residual" and name in ("gemm_ffn_in_gelu", "gemm_ffn_out")
            work = executed // 2 if two_term else executed
            unit = "mfma"
        else:
            work = executed = attention_flops(i["batch"], i["heads"], i["seq"], i["head_dim"])
            unit = "mfma"
        per_fwd = 1 if name == "layernorm_final" else cfg.num_layers
        out.append((name, ln, work, unit, executed, per_fwd))
    return out


def time_kernel(fn, reps: int) -> float:
    """Average duration (ms) of one launch.  The reps launches are captured
    into one hipGraph (so host launch cost is excluded, as in the forward's
    own graph) and the replay is bracketed by two HIP events recorded on the
    stream the kernels run on."""
    with torch.inference_mode():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph):
                for _ in range(reps):
                    fn()
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def kernel_breakdown(model, x, reps):
    rows = []
    for name, fn, work, bound, executed, per_fwd in forward_launches(model, x):
        ms = time_kernel(fn, reps)
        rows.append({"kernel": name, "avg_ms": ms, "work": work, "executed_work": executed,
                     "bound": bound, "launches_per_forward": per_fwd, "ms_per_forward": ms * per_fwd})
    return rows


def roofline_of(row, dtype_name, traffic=None):
    if row["bound"] == "mfma":
        achieved = row["work"] / (row["avg_ms"] / 1e3) / 1e12
        peak = MI355X_PEAK_FLOPS[EXECUTED_PRECISION[dtype_name]] / 1e12
        unit = "TFLOP/s"
    else:
        achieved = row["work"] / (row["avg_ms"] / 1e3) / 1e9
        peak = MI355X_HBM_BYTES_PER_S / 1e9
        unit = "GB/s"
    return {"kernel": row["kernel"], "bound": row["bound"], "achieved": round(achieved, 2),
            "peak": round(peak, 1), "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": traffic, "avg_us": round(row["avg_ms"] * 1e3, 3),
            "work_per_launch": row["work"]}


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summaries, if any."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        data = json.loads(p.read_text())
        return data.get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None


# --------------------------------------------------------------- provenance
def _run(cmd, timeout=20):
    try:
        out = subprocess.run(cmd, capture_output=True, text=True, errors="replace", timeout=timeout)
        return out.stdout if out.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        return None


def source_hash() -> str:
    """SHA-256 over the sources that define what runs (kernels, C ABI, host
    package, this file), so a record can be tied to a tree without git."""
    h = hashlib.sha256()
    files = sorted([*ROOT.glob("include/*.h"), *ROOT.glob("transformer_optimization_amd/csrc/*"),
                    *ROOT.glob("transformer_optimization_amd/*.py"), ROOT / "bench.py"])
    for f in files:
        if f.is_file():
            h.update(str(f.relative_to(ROOT)).encode())
            h.update(f.read_bytes())
    return h.hexdigest()


def kernel_sources_hash() -> str:
    """SHA-256 over the kernel sources and the C header, as the build records it."""
    h = hashlib.sha256()
    for f in sorted([*ROOT.glob("transformer_optimization_amd/csrc/*"), *ROOT.glob("include/*.h")]):
        if f.is_file():
            h.update(str(f.relative_to(ROOT)).encode())
            h.update(f.read_bytes())
    return h.hexdigest()


def git_state():
    if not (ROOT / ".git").exists():
        # A copy of the tree without git (the GPU box): the commit the library
        # was built from, as the build recorded it, and whether the kernel
        # sources here still match the ones it was built from.
        info_path = ROOT / "transformer_optimization_amd" / "_lib" / "build_info.json"
        try:
            info = json.loads(info_path.read_text())
        except (OSError, ValueError):
            return {"head": None, "dirty": None, "note": "no git checkout and no build record"}
        return {"head": info.get("git_head"), "dirty": info.get("git_dirty"),
                "note": f"from the build record ({info.get('built_utc')}); no git checkout here",
                "kernel_sources_match_build": info.get("kernel_sources_sha256") == kernel_sources_hash()}
    head = _run(["git", "-C", str(ROOT), "rev-parse", "HEAD"])
    status = _run(["git", "-C", str(ROOT), "status", "--porcelain", "--untracked-files=no"])
    branch = _run(["git", "-C", str(ROOT), "rev-parse", "--abbrev-ref", "HEAD"])
    return {"head": head.strip() if head else None, "branch": branch.strip() if branch else None,
            "dirty": bool(status.strip()) if status is not None else None}


def cpu_info():
    """Host CPU model and thread budget from /proc/cpuinfo (no subprocess:
    nothing may be forked from a process that has initialised the GPU)."""
    info = {"model": None, "logical_cpus": None, "sockets": None,
            "affinity_cores": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}
    try:
        text = Path("/proc/cpuinfo").read_text()
    except OSError:
        text = ""
    procs, sockets = 0, set()
    for line in text.splitlines():
        k, _, v = line.partition(":")
        k, v = k.strip(), v.strip()
        if k == "processor":
            procs += 1
        elif k == "model name" and info["model"] is None:
            info["model"] = v
        elif k == "physical id":
            sockets.add(v)
    info["logical_cpus"] = procs or None
    info["sockets"] = len(sockets) or None
    if info["model"] is None:
        info["model"] = platform.processor() or None
    return info


# ---------------------------------------------------------------- GPU state
# Read from the amdgpu driver's sysfs files of this process's device and from
# the KFD process list, in-process: a forked rocm-smi from a process that has
# initialised the GPU is refused on the GPU boxes (and is the kind of exec
# that can take a machine down).
def _read(path: Path):
    try:
        return path.read_text().strip()
    except OSError:
        return None


def gpu_sysfs_dir(dev):
    """``/sys/bus/pci/devices/<domain:bus:dev.0>`` of a torch device, or None."""
    props = torch.cuda.get_device_properties(dev)
    dom, bus, slot = (getattr(props, a, None) for a in ("pci_domain_id", "pci_bus_id", "pci_device_id"))
    if bus is None:
        return None
    d = Path(f"/sys/bus/pci/devices/{int(dom or 0):04x}:{int(bus):02x}:{int(slot or 0):02x}.0")
    return d if d.exists() else None


def kfd_gpu_id(sysdir):
    """KFD's gpu_id of the device at sysdir (topology node whose PCI location
    matches), or None."""
    if sysdir is None:
        return None
    try:
        dom, bus, devfn = sysdir.name.split(":")
        dev_, fn = devfn.split(".")
        loc = (int(bus, 16) << 8) | (int(dev_, 16) << 3) | int(fn, 16)
        for node in Path("/sys/class/kfd/kfd/topology/nodes").iterdir():
            props = _read(node / "properties") or ""
            kv = dict(ln.split()[:2] for ln in props.splitlines() if len(ln.split()) >= 2)
            if kv.get("location_id") == str(loc) and kv.get("domain", "0") == str(int(dom, 16)):
                return _read(node / "gpu_id")
    except (OSError, ValueError):
        return None
    return None


def kfd_pids(gpu_id=None):
    """Host PIDs holding a KFD (compute) context, restricted to those with
    memory on gpu_id when given; None if the list is not visible here.
    (The names are host PIDs: inside a container they do not match
    os.getpid(), so callers compare sets over time instead.)"""
    base = Path("/sys/class/kfd/kfd/proc")
    try:
        pids = [p for p in base.iterdir() if p.name.isdigit()]
    except OSError:
        return None
    if gpu_id:
        pids = [p for p in pids if (p / f"vram_{gpu_id}").exists() or (p / f"stats_{gpu_id}").exists()]
    return sorted(int(p.name) for p in pids)


def gpu_state(sysdir, gpu_id=None):
    """Busy %, current shader / memory clocks, power and temperature of the
    device, and the processes holding compute contexts on it."""
    st = {"sysfs": str(sysdir) if sysdir else None, "busy_pct": None, "sclk": None, "mclk": None,
          "power_w": None, "temp_c": None}
    if sysdir is not None:
        busy = _read(sysdir / "gpu_busy_percent")
        st["busy_pct"] = float(busy) if busy and busy.lstrip("-").isdigit() else None
        for key, fname in (("sclk", "pp_dpm_sclk"), ("mclk", "pp_dpm_mclk")):
            txt = _read(sysdir / fname)
            if txt:
                cur = [ln for ln in txt.splitlines() if ln.rstrip().endswith("*")]
                st[key] = (cur[0].split(":", 1)[-1].replace("*", "").strip() if cur else None)
        for hw in sorted((sysdir / "hwmon").glob("hwmon*")) if (sysdir / "hwmon").exists() else []:
            for fname in ("power1_average", "power1_input"):
                v = _read(hw / fname)
                if v and v.isdigit() and st["power_w"] is None:
                    st["power_w"] = round(int(v) / 1e6, 1)
            v = _read(hw / "temp2_input") or _read(hw / "temp1_input")
            if v and v.lstrip("-").isdigit() and st["temp_c"] is None:
                st["temp_c"] = int(v) / 1000.0
    st["compute_pids"] = kfd_pids(gpu_id)
    return st


IDLE_BUSY_PCT = 10.0   # agent/tools/_common.py:217 (util_threshold)
IDLE_HOLD_S = 5.0      # agent/tools/_common.py:217 (hold_s)


def wait_for_idle(sysdir, timeout_s: float, hold_s: float = IDLE_HOLD_S, poll_s: float = 0.25, gpu_id=None):
    """Block until the device has been below IDLE_BUSY_PCT busy for hold_s
    (agent/tools/_common.py:217-240).  Returns the gate record; ``idle``
    False on timeout, when the caller must refuse to measure.  Where the
    device's busy counter is not visible the gate cannot wait: it records
    ``measurable`` False and passes, and the record says so."""
    t0 = time.time()
    below_since = None
    samples = []
    while True:
        st = gpu_state(sysdir, gpu_id)
        now = time.time()
        busy = st["busy_pct"]
        samples.append(busy)
        if busy is None:
            return {"idle": True, "measurable": False, "waited_s": round(now - t0, 2),
                    "compute_pids": st["compute_pids"],
                    "note": "device busy counter not readable here; gate not enforced"}
        if busy < IDLE_BUSY_PCT:
            below_since = below_since if below_since is not None else now
            if now - below_since >= hold_s:
                return {"idle": True, "measurable": True, "waited_s": round(now - t0, 2),
                        "threshold_pct": IDLE_BUSY_PCT, "hold_s": hold_s,
                        "max_busy_pct_in_hold": max(samples[-int(hold_s / poll_s) - 1:]),
                        "compute_pids": st["compute_pids"]}
        else:
            below_since = None
        if now - t0 > timeout_s:
            return {"idle": False, "measurable": True, "waited_s": round(now - t0, 2),
                    "last_busy_pct": busy, "compute_pids": st["compute_pids"],
                    "reason": f"device not below {IDLE_BUSY_PCT}% busy for {hold_s} s within {timeout_s} s"}
        time.sleep(poll_s)


class ForeignLoadSampler:
    """Samples the device state in a thread while measurements run; the run
    is untrusted if a compute process that was not there at the start (this
    process included) appears on the device meanwhile (agent/tools/
    _common.py:243-311)."""

    def __init__(self, sysdir, gpu_id=None, poll_s: float = 0.5):
        import threading

        self.sysdir, self.gpu_id, self.poll_s = sysdir, gpu_id, poll_s
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)
        self.max_busy = None
        self.baseline = None
        self.foreign = set()

    def _run(self):
        while not self._stop.is_set():
            st = gpu_state(self.sysdir, self.gpu_id)
            if st["busy_pct"] is not None:
                self.max_busy = max(self.max_busy or 0.0, st["busy_pct"])
            if st["compute_pids"] is not None and self.baseline is not None:
                self.foreign.update(set(st["compute_pids"]) - self.baseline)
            self._stop.wait(self.poll_s)

    def __enter__(self):
        pids = kfd_pids(self.gpu_id)
        self.baseline = set(pids) if pids is not None else None
        self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._thread.join(timeout=5)

    def report(self):
        return {"trusted": not self.foreign, "process_list_visible": self.baseline is not None,
                "baseline_compute_pids": sorted(self.baseline) if self.baseline is not None else None,
                "max_busy_pct": self.max_busy, "new_compute_pids": sorted(self.foreign)}


def ranges_overlap(a, b) -> bool:
    """Whether two [min, max] ranges overlap (agent/tools/_common.py:318-327):
    only non-overlapping ranges count as a change."""
    return not (max(a) < min(b) or max(b) < min(a))


def previous_record():
    """The newest committed driver record (BENCH_rNN.json at the repository
    root), as ``(file name, parsed bench line)``, or (None, None)."""
    best = None
    for p in ROOT.glob("BENCH_r*.json"):
        tag = p.stem[len("BENCH_r"):]
        if tag.isdigit() and (best is None or int(tag) > best[0]):
            best = (int(tag), p)
    if best is None:
        return None, None
    try:
        data = json.loads(best[1].read_text())
    except (OSError, ValueError):
        return best[1].name, None
    return best[1].name, data.get("parsed", data)


RANGES_PATH = ROOT / "profiles" / "bench_ranges.json"


def committed_ranges():
    """Per-config latency ranges of an earlier measured run, committed in
    the repository (the driver's records keep only the headline fields), as
    ``(label, {config: [min, max]})`` or (None, {})."""
    try:
        data = json.loads(RANGES_PATH.read_text())
    except (OSError, ValueError):
        return None, {}
    label = f"{RANGES_PATH.relative_to(ROOT)} ({data.get('git_head', '?')[:12]}, {data.get('measured_utc', '?')})"
    return label, data.get("per_config", {})


def compare_range(new_range, old_range, source):
    """Verdict of a new [min, max] latency range against an old one (lower is
    better; agent/tools/bench.py:101-116)."""
    overlap = ranges_overlap(new_range, old_range)
    verdict = "noise" if overlap else ("improved" if max(new_range) < min(old_range) else "regressed")
    return {"source": source, "old_range_ms": [round(v, 5) for v in old_range],
            "new_range_ms": [round(v, 5) for v in new_range], "ranges_overlap": overlap,
            "verdict": verdict,
            "median_delta_pct": round(100.0 * (statistics.median(new_range) / statistics.median(old_range) - 1.0), 2)}


def old_range_of(rec):
    """[min, max] of a record's repeated measurements (a single median when
    the record carries none)."""
    if rec is None:
        return None
    rng = rec.get("range_ms")
    if rng:
        return [rng["min"], rng["max"]]
    v = rec.get("value", rec.get("latency_ms_p50"))
    return [v, v] if v is not None else None


def provenance_host():
    """Everything of the provenance that does not touch the GPU.  Collected
    before the first GPU call: git runs as a subprocess, and nothing may be
    forked once the process has initialised the GPU."""
    lib = _C.LIB_PATH
    return {
        "source_sha256": source_hash(),
        "git": git_state(),
        "library_sha256": hashlib.sha256(lib.read_bytes()).hexdigest() if lib.exists() else None,
        "torch": torch.__version__, "hip": torch.version.hip,
        "cpu": cpu_info(),
        "python": platform.python_version(),
        "timestamp_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
    }


def device_record(dev):
    props = torch.cuda.get_device_properties(dev)
    return {"name": props.name, "arch": getattr(props, "gcnArchName", None),
            "compute_units": props.multi_processor_count,
            "memory_gib": round(props.total_memory / 2**30, 1),
            "pci": [getattr(props, a, None) for a in ("pci_domain_id", "pci_bus_id", "pci_device_id")]}


# -------------------------------------------------------------- CPU baseline
def cpu_threads():
    """Threads for the CPU baseline: every core of the process's affinity
    set, bounded by OMP_NUM_THREADS when the host sets it (the GPU box sets
    its per-GPU CPU share there)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(wl, budget_s: float):
    """The eager oracle (the reference's BaselineTransformer, restated) on the
    host cores, in the workload's dtype, timed with perf_counter_ns per call
    (TTB:4848-4853).  Bounded sample: one block of the stack is timed
    (repeated until ~budget_s, median) and the forward is that times the
    layer count plus the final LayerNorm, since every block has the same
    cost.  For sequences with no dense baseline (S = 100000) the block is
    timed on a subset of query rows -- LN1 and the K/V projections of all
    rows, attention and the block tail of the subset -- and the row-dependent
    part is extrapolated linearly to all rows."""
    import oracle  # the checker's restatement; timed here as the CPU baseline only
    from oracle.chunked import _attention_rows, head_split_kv

    threads = cpu_threads()
    torch.set_num_threads(threads)
    c = wl.config
    model = oracle.BaselineTransformer(c)
    workloads.init_parameters(model)
    model = model.to(wl.dtype).eval()
    x = workloads.make_input(c, wl.dtype)
    block = model.layers[0]

    def timed(fn, reps_max=50):
        t0 = time.perf_counter_ns()
        fn()
        first = (time.perf_counter_ns() - t0) / 1e6
        times = [first]
        reps = max(0, min(reps_max, int(budget_s * 1e3 / max(first, 1e-3)) - 1))
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            fn()
            times.append((time.perf_counter_ns() - t0) / 1e6)
        return statistics.median(times), len(times)

    with torch.inference_mode():
        t_ln, _ = timed(lambda: model.final_norm(x), 5)
        if c.seq_len <= 16384:
            t_blk, n = timed(lambda: block(x, None, c.causal))
            value = t_blk * c.num_layers + t_ln
            sample = (f"{wl.name}: eager oracle block 0 of {c.num_layers}, {wl.dtype_name} on CPU, "
                      f"median of {n} calls, x{c.num_layers} layers + final LayerNorm")
            kind_note = "measured per block"
        else:
            rows_n = 512
            rows = torch.arange(0, c.seq_len, c.seq_len // rows_n)[:rows_n]

            def all_rows_part():
                xn = block.norm1(x)
                return xn, head_split_kv(block.attention, xn)

            t_all, _ = timed(all_rows_part, 3)
            xn, kv = all_rows_part()

            def subset_part():
                xr = x[:, rows, :] + _attention_rows(block.attention, xn, rows, None, c.causal, 64, kv)
                xr = xr + block.ffn_out(torch.nn.functional.gelu(block.ffn_in(block.norm2(xr))))
                return model.final_norm(xr)

            t_sub, n = timed(subset_part, 3)
            value = (t_all + t_sub * c.seq_len / rows_n) * c.num_layers
            sample = (f"{wl.name}: eager oracle, {wl.dtype_name} on CPU; LN1 + K/V projections of all "
                      f"{c.seq_len} rows ({t_all:.0f} ms) + attention and block tail of {rows_n} "
                      f"query rows ({t_sub:.0f} ms, median of {n}) extrapolated linearly to all rows")
            kind_note = "extrapolated"
    return {"value": round(value, 4), "unit": "ms", "cores": threads, "kind": "port",
            "sample": sample, "method": kind_note}


def eager_gpu_model(wl, dev):
    """The eager oracle on the same GPU and dtype (the reference's baseline
    model); None where its dense scores cannot exist (S = 100000: 320 GB)."""
    import oracle

    c = wl.config
    if c.seq_len > 16384:
        return None
    model = oracle.BaselineTransformer(c)
    workloads.init_parameters(model)
    return model.to(dev, wl.dtype).eval()


# ---------------------------------------------------------------------- main
def per_config_record(key, dev, args, prev=None):
    cw = workloads.workload(key)
    c = cw.config
    log(f"[bench] per-config {cw.name}")
    ours, x = build_model(cw, dev)
    base = eager_gpu_model(cw, dev)
    repeats = REPEATS.get(key.partition(":")[0], 10)
    base_r, ours_r = benchmark_pair(base, ours, x, args.rounds, repeats, warmup=3)
    base_s = [t for r in base_r for t in r]
    ours_s = [t for r in ours_r for t in r]
    tokens = c.batch_size * c.seq_len
    mine = summarize(ours_s, tokens)
    ms = mine["median_ms"]
    rng = range_of(ours_r)
    krows = kernel_breakdown(ours, x, 10 if c.seq_len >= 8192 else 50)
    kd = max(krows, key=lambda r: r["ms_per_forward"])
    policy = ours.resolve_policy(c.seq_len, cw.dtype, dev)
    rec = {"config": key, **config_record(cw), "softmax": policy[0], "precision": policy[1],
           "latency_ms_p50": ms, "timing": mine, "range_ms": rng, **mfu_fields(cw, ms),
           "kernels_us": {r["kernel"]: round(r["avg_ms"] * 1e3, 2) for r in krows},
           "kernels_ms_per_forward": {r["kernel"]: round(r["ms_per_forward"], 4) for r in krows},
           "dominant_kernel": roofline_of(kd, cw.dtype_name, load_traffic(kd["kernel"], cw.name))}
    executed = sum(r["executed_work"] * r["launches_per_forward"] for r in krows if r["bound"] == "mfma")
    if c.causal:
        # Executed attention work is about half the dense figure: key tiles
        # past the diagonal are skipped (README.md:158-163 reports both).
        att = attention_flops(c.batch_size, c.num_heads, c.seq_len, c.d_model // c.num_heads)
        executed -= c.num_layers * att // 2
        rec["mfu_note"] = "tflop_s/mfu count dense (no causal discount); executed_tflop_s halves attention"
    rec["executed_tflop_s"] = round(executed / (ms / 1e3) / 1e12, 2)
    if key == "c2":
        rec["empty_graph_replay_us"] = empty_graph_replay_us()
    old = None
    if prev is not None:
        old = next((r for r in prev[1].get("per_config", []) if r.get("config") == key), None)
    if old is not None and old_range_of(old):
        rec["comparison"] = compare_range([rng["min"], rng["max"]], old_range_of(old), prev[0])
    else:
        label, ranges = committed_ranges()
        if key in ranges:
            rec["comparison"] = compare_range([rng["min"], rng["max"]], ranges[key], label)
    if base is not None:
        eager = summarize(base_s, tokens)
        rec["eager_gpu"] = eager
        rec["eager_gpu_ms"] = eager["median_ms"]
        rec["speedup_vs_eager_gpu"] = round(eager["median_ms"] / ms, 3)
    else:
        rec["eager_gpu_ms"] = None
        rec["speedup_vs_eager_gpu"] = None
    del ours, base, x
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        if ":" not in key:
            cb = cpu_baseline(cw, args.cpu_budget_s if key == args.workload else args.cpu_config_budget_s)
            rec["cpu_baseline"] = cb
            rec["speedup_vs_cpu"] = round(cb["value"] / ms, 2)
    log(f"  {ms:.4f} ms (p90 {mine['p90_ms']}, min {mine['min_ms']}, rounds {rng['min']}-{rng['max']})  "
        f"{rec['tflop_s']} TFLOP/s  "
        f"MFU {rec['mfu']:.2%}  eager-GPU {rec['eager_gpu_ms']} ms"
        + (f"  CPU {rec['cpu_baseline']['value']} ms ({rec['cpu_baseline']['method']})"
           if "cpu_baseline" in rec else ""))
    return rec


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(workloads.WORKLOADS))
    ap.add_argument("--per-config", default="c1,c2,c3,c4,c5,c3:causal,c4:causal",
                    help="comma list of configs to report in per_config ('' = none); "
                         "cN:causal = config N with causal masking")
    ap.add_argument("--rounds", type=int, default=ROUNDS,
                    help="alternating eager/optimised rounds per config (TTB --benchmark-rounds); "
                         "their per-round medians give each config's range")
    ap.add_argument("--runs", type=int, default=3,
                    help="repeated headline measurements of --steps each (agent/tools/bench.py --runs); "
                         "the first is the reported value, all give the range")
    ap.add_argument("--write-ranges", default=None,
                    help="also write the measured per-config ranges to this JSON file "
                         "(the format of profiles/bench_ranges.json)")
    ap.add_argument("--idle-timeout-s", type=float, default=120.0,
                    help="longest wait for an idle GPU before refusing to measure")
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--cpu-budget-s", type=float, default=15.0,
                    help="CPU-baseline time budget of the headline workload")
    ap.add_argument("--cpu-config-budget-s", type=float, default=4.0,
                    help="CPU-baseline time budget per other config")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB "
                         "(a known-size kernel for scaling HBM counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "this build has no multi-GPU path.", file=sys.stderr)
        return 2
    if args.runs < 1:
        print("--runs must be at least 1", file=sys.stderr)
        return 2
    # Host-side provenance first: it forks git, which must happen before the
    # process touches the GPU.
    prov = provenance_host()
    prev = previous_record()
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    _C.load_library()
    prov["device"] = device_record(dev)
    sysdir = gpu_sysfs_dir(dev)
    gpu_id = kfd_gpu_id(sysdir)
    prov["device"]["sysfs"] = str(sysdir) if sysdir else None
    prov["device"]["kfd_gpu_id"] = gpu_id

    # Idle gate: refuse to measure on a busy GPU (agent/tools/bench.py:29-33).
    gate = wait_for_idle(sysdir, args.idle_timeout_s, gpu_id=gpu_id)
    prov["idle_gate"] = gate
    prov["gpu_before"] = gpu_state(sysdir, gpu_id)
    log(f"[bench] idle gate: {gate}")
    if not gate["idle"]:
        print(f"bench refused: {gate['reason']}", file=sys.stderr)
        return 3

    wl = workloads.WORKLOADS[args.workload]
    c = wl.config
    log(f"[bench] headline workload {wl.name}: {args.warmup} warmup + {args.steps} timed steps, "
        f"{args.runs} runs")
    sampler = ForeignLoadSampler(sysdir, gpu_id)
    with sampler:
        model, x = build_model(wl, dev)
        warmup_model(model, x, args.warmup)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        per = benchmark_once(model, x, args.steps)
        wall = time.perf_counter() - t0
        head = summarize(per, c.batch_size * c.seq_len)
        p50 = head["median_ms"]
        ms_per_step = wall * 1e3 / args.steps
        log(f"[bench] run 1: p50 {p50:.4f} ms (p90 {head['p90_ms']}, min {head['min_ms']}), "
            f"wall {ms_per_step:.4f} ms/step")
        # Repeated measurements of the same workload, for the range only.
        runs = [per]
        for r in range(1, args.runs):
            warmup_model(model, x, args.warmup)
            runs.append(benchmark_once(model, x, args.steps))
            log(f"[bench] run {r + 1}: p50 {statistics.median(runs[-1]):.4f} ms")
        head_range = range_of(runs)

        log("[bench] per-kernel breakdown (HIP events, the forward's own launches)")
        rows = kernel_breakdown(model, x, args.kernel_reps)
        for r in rows:
            log(f"  {r['kernel']:18s} {r['avg_ms'] * 1e3:9.2f} us x{r['launches_per_forward']}")
        dom = max(rows, key=lambda r: r["ms_per_forward"])
        roof = roofline_of(dom, wl.dtype_name, load_traffic(dom["kernel"], wl.name))
        del model, x
        torch.cuda.empty_cache()

        per_config = [per_config_record(key, dev, args, prev if prev[1] else None)
                      for key in [k for k in args.per_config.split(",") if k]]

        if args.calibration_copy_mib > 0:
            n = args.calibration_copy_mib * (1 << 20) // 4
            src = torch.ones(n, dtype=torch.float32, device=dev)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            log(f"[bench] calibration copy: {args.calibration_copy_mib} MiB read + written")
            del src, dst

    cpu = None
    if not args.no_cpu_baseline:
        cpu = next((r["cpu_baseline"] for r in per_config if r["config"] == args.workload), None)
        if cpu is None:
            log(f"[bench] CPU baseline ({wl.name})")
            cpu = cpu_baseline(wl, args.cpu_budget_s)
        log(f"[bench] CPU baseline {wl.name}: {cpu['value']} ms on {cpu['cores']} threads")
    sp = [r["speedup_vs_eager_gpu"] for r in per_config
          if r["config"] in ("c2", "c3", "c4") and r.get("speedup_vs_eager_gpu")]
    geomean = round(math.exp(sum(math.log(v) for v in sp) / len(sp)), 3) if sp else None
    prov["gpu_after"] = gpu_state(sysdir, gpu_id)
    prov["load_during_measurement"] = sampler.report()

    out = {
        "metric": "forward latency (ms), p50 over graph replays; MFU vs MI355X dense MFMA peak per config",
        "value": round(p50, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float16": "fp16", "bfloat16": "bf16"}.get(wl.dtype_name, wl.dtype_name),
        "data": "synthetic (weights N(0,0.02) seed 0, x ~ N(0,1) seed 1)",
        "config": config_record(wl),
        "timing": head,
        "range_ms": head_range,
        **mfu_fields(wl, p50),
        "roofline": roof,
        "cpu_baseline": cpu,
        "geomean_speedup_vs_eager_gpu_c2_c4": geomean,
        "trusted": sampler.report()["trusted"],
        "per_config": per_config,
        "provenance": prov,
    }
    # A headline range is only compared with one of the same workload.
    prev_wl = ((prev[1] or {}).get("config") or {}).get("workload")
    if prev[1] is not None and prev_wl == wl.name:
        old_rng = old_range_of(prev[1])
        if old_rng:
            out["comparison"] = compare_range([head_range["min"], head_range["max"]], old_rng, prev[0])
            log(f"[bench] vs {prev[0]}: {out['comparison']['verdict']} "
                f"({out['comparison']['median_delta_pct']:+.2f}% median)")
    if args.write_ranges:
        Path(args.write_ranges).write_text(json.dumps({
            "note": "per-config latency ranges (min / max of per-round medians, ms) of one bench.py run",
            "git_head": (prov.get("git") or {}).get("head"), "measured_utc": prov["timestamp_utc"],
            "device": prov["device"]["name"], "headline": [head_range["min"], head_range["max"]],
            "per_config": {r["config"]: [r["range_ms"]["min"], r["range_ms"]["max"]] for r in per_config},
        }, indent=1) + "\n")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

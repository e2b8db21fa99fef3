#!/usr/bin/env python3
"""Weaver decode benchmark on one MI355X.

Metric: decode attention tokens/s per GPU and achieved HBM GB/s for a hot pool
of 2048 f16 tokens plus a cold pool of 32768 SparseCodes per kv head
(32 q / 8 kv heads, head_dim 128, one shared 4096 x 128 dictionary), swept
over batch B = 1..64.  `value` is tokens/s at B = 64; every B of the sweep is
reported beside it.  One step = one full decode (q . D^T, hot split-K, cold
bins, bins . D and merge) over the whole batch, inputs resident in HBM.

Pools are replicated over several disjoint block sets ("copies") and the steps
rotate through them, so every step reads at least ~512 MB of distinct data and
the 256 MB Infinity Cache cannot serve repeats.  The cold pool sits in HBM in
the head-blocked order [blocks][kv_heads][16] (how the .aether fabric keeps it
on the device: same codes, one kv head's 16 codes of a block contiguous); the
reference's file order [blocks][16][kv_heads] is measured beside it, with
output bits checked identical (`--cold-layout` swaps the two).

Also measured in the same run:
  * per-kernel durations with HIP events on the stream each kernel runs on
    (roofline of the dominant kernel at B = 64);
  * the reference's own --bench configuration (nexus-core/src/bench.rs:27-36,
    113-133: 64 hot + 16 cold blocks, 512-atom per-kv-head dictionary, B = 1),
    beside its published 389.6 tok/s on an M1 Pro;
  * the CPU baseline: the oracle's multi-threaded fp32 restatement of the
    reference kernel on this host, on a bounded sample of B = 1 steps;
  * the SparseCode encoder on 8192 Llama8B hot blocks, and the Llama8B
    `.aether` fabric: upload of its pools into HBM, write-back of its cold pool,
    and one Distiller cycle on the device (each beside the CPU oracle).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode attn tokens/s per GPU + achieved HBM GB/s (hot 2k + cold 32k, B=1..64)"
PEAK_HBM_GBPS = 8000.0
MALL_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--batches", default="1,2,4,8,16,32,64")
    p.add_argument("--no-graph", action="store_true", help="launch each step from the host (no HIP graph)")
    p.add_argument("--steps-per-graph", type=int, default=8,
                   help="besides a graph per step, time graphs of this many decode steps (one host launch for "
                        "all of them) and report the faster of the two (1: a graph per step only)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--stage-sweep", action="store_true", help="per-kernel times at every batch size")
    p.add_argument("--cold-layout", choices=("reference", "head_blocked"), default="head_blocked",
                   help="cold pool order in HBM of the main measurement: head_blocked ([blocks][kv_heads][16], "
                        "how the fabric keeps it on the device) or reference ([blocks][16][kv_heads], the file order)")
    p.add_argument("--skip-encoder", action="store_true", help="skip the SparseCode encoder measurement")
    p.add_argument("--skip-fabric", action="store_true", help="skip the .aether fabric residency measurement")
    p.add_argument("--skip-attention", action="store_true", help="skip the inference-attention measurement")
    p.add_argument("--skip-ops", action="store_true", help="skip the dense-ops measurement (products, decode forward)")
    p.add_argument("--skip-projection", action="store_true", help="skip the projection-path table (MFMA vs VALU)")
    p.add_argument("--only-ops", action="store_true", help="time only the dense ops and print them")
    p.add_argument("--only-products", action="store_true",
                   help="time only the dense products (no decode forwards: short enough for counter runs)")
    p.add_argument("--configs", default="2,4,5",
                   help="BASELINE configurations timed beside the sweep (comma list of 2, 4, 5; empty for none)")
    p.add_argument("--only-configs", action="store_true",
                   help="time only the --configs lines (no sweep, no other measurement) and print them")
    p.add_argument("--skip-alt-layout", action="store_true",
                   help="skip the extra B-max run with the other cold pool order (for clean profiles)")
    p.add_argument("--rocpd-summary", metavar="DB", help="print a per-kernel summary of a rocprofv3 database and exit")
    p.add_argument("--kernel-filter", default="aw::", help="kernel-name filter for --rocpd-summary")
    p.add_argument("--copy-calibration", type=int, metavar="MIB", default=0,
                   help="first run a plain device copy of MIB MiB (counter calibration)")
    p.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                   help="print HBM traffic per launch from a FETCH_SIZE and a WRITE_SIZE rocprofv3 database and exit")
    p.add_argument("--traffic-command", default="", help="command line recorded in --traffic-summary output")
    p.add_argument("--traffic-title", default="", help="workload named in --traffic-summary output")
    p.add_argument("--only-projection", action="store_true",
                   help="time only q . D^T on MFMA and on the VALU at several row counts and print them")
    p.add_argument("--only-attention", action="store_true",
                   help="time only the inference attention (dense and tiered caches) and print it")
    p.add_argument("--trace-phase", choices=("all", "pipeline", "serial"), default="all",
                   help="for kernel traces: 'pipeline' launches only the concurrent pipeline (no per-kernel "
                        "event timing), 'serial' runs every decode with its kernels one at a time and no graph")
    return p.parse_args()


def copies_for(geom) -> int:
    per_copy = geom.algorithmic_bytes()["total"]
    return max(1, min(256, math.ceil(2 * MALL_BYTES / per_copy)))


class Runner:
    """One workload resident on the GPU, its descriptors and (optionally) graphs."""

    def __init__(self, engine, geom, seed, use_graph, wl=None, cold_head_blocked=False, steps_per_graph=1):
        import torch
        from aether_nexus_amd import workloads as W
        self.torch = torch
        self.engine = engine
        self.geom = geom
        self.wl = wl if wl is not None else W.generate(geom, seed=seed, device="cuda:0")
        self.out = torch.empty(self.wl.out_shape(), dtype=torch.float16, device="cuda:0")
        # Optionally the same codes in the head-blocked pool layout (AW_F_COLD_HEAD_BLOCKED).
        self.cold_hb = W.head_blocked(self.wl.cold) if cold_head_blocked else None
        self.descs = [W.device_desc(self.wl, self.out, copy=c, cold_head_blocked=self.cold_hb)
                      for c in range(geom.copies)]
        self.stream = torch.cuda.Stream()
        # The inputs were written on the current stream: order the side stream after them.
        self.stream.wait_stream(torch.cuda.current_stream())
        self.graphs = None
        sh = self.stream.cuda_stream
        with torch.cuda.stream(self.stream):
            for d in self.descs:  # first calls size the workspace
                engine.decode_device(d, stream=sh)
        engine.check_device_errors(sh)
        if use_graph:
            self.graphs = []
            for d in self.descs:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream):
                    engine.decode_device(d, stream=torch.cuda.current_stream().cuda_stream)
                self.graphs.append(g)
        # Graphs of m consecutive steps (copies in rotation), the way a serving
        # loop captures a whole decode step: a replay's host launch cost is paid
        # once per m steps, so a short step is timed on the GPU, not on the host.
        self.m = steps_per_graph if use_graph else 1
        self.multi = []
        if self.m > 1:
            C = len(self.descs)
            for k in range(max(1, C // self.m)):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream):
                    for j in range(self.m):
                        engine.decode_device(self.descs[(k * self.m + j) % C],
                                             stream=torch.cuda.current_stream().cuda_stream)
                self.multi.append(g)

    def step(self, i):
        if self.graphs is not None:
            self.graphs[i % len(self.graphs)].replay()
        else:
            self.engine.decode_device(self.descs[i % len(self.descs)], stream=self.stream.cuda_stream)

    def time_best(self, steps, warmup):
        """ms per step of the faster way to replay the same steps: a graph per step,
        or graphs of m steps (whose one host launch covers m steps).  Returns
        (ms, steps per graph of that mode, {steps per graph: ms} of both)."""
        by = {1: self.time_steps(steps, warmup, one_step_graphs=True)}
        if self.multi:
            by[self.m] = self.time_steps(steps, warmup)
        m = min(by, key=by.get)
        return by[m], m, {str(k): round(v, 5) for k, v in by.items()}

    def time_steps(self, steps, warmup, one_step_graphs=False):
        """ms per step over exactly `steps` decode steps after `warmup` untimed
        ones: replays of the m-step graphs (and one-step graphs for a remainder),
        or of one-step graphs only."""
        torch = self.torch
        m = 1 if one_step_graphs or not self.multi else self.m
        with torch.cuda.stream(self.stream):
            for i in range(warmup):
                self.step(i)
            for g in self.multi:
                g.replay()
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(self.stream)
            for k in range(steps // m if m > 1 else 0):
                self.multi[k % len(self.multi)].replay()
            for i in range(steps % m if m > 1 else steps):
                self.step(warmup + i)
            b.record(self.stream)
            torch.cuda.synchronize()
        return a.elapsed_time(b) / steps  # ms per step

    def stage_times(self, steps, mode=1):
        """Average duration per kernel stage: HIP events bracket each launch on
        the stream it runs on.  mode 1 keeps the concurrent pipeline of the timed
        steps (launched from the host, same rotation); mode 2 serializes it."""
        torch = self.torch
        eng = self.engine
        eng.reset_stage_stats()
        eng.set_profiling(mode)
        try:
            with torch.cuda.stream(self.stream):
                torch.cuda.synchronize()
                for i in range(steps):
                    eng.decode_device(self.descs[i % len(self.descs)], stream=self.stream.cuda_stream)
                torch.cuda.synchronize()
            st = eng.stage_stats()
        finally:
            eng.set_profiling(0)
        return {k: (ms / n if n else None, n) for k, (ms, n) in st.items()}


def stage_pair(r, args):
    """Per-kernel event times in the pipeline and serialized, or none (a kernel
    trace of one phase: --trace-phase pipeline / serial)."""
    if args.trace_phase != "all":
        none = {k: (None, 0) for k in ("project", "hot", "cold", "finish", "merge")}
        return none, dict(none)
    return r.stage_times(args.steps, mode=1), r.stage_times(args.steps, mode=2)


def kernel_bytes(geom) -> dict:
    """Algorithmic HBM bytes per launch of the hot and cold kernels."""
    from aether_nexus_amd.types import BLOCK_SIZE
    B, Hkv, D = geom.batch * geom.layers, geom.kv_heads, geom.head_dim
    nh, nc = geom.hot_count * BLOCK_SIZE, geom.cold_count * BLOCK_SIZE
    q = B * geom.queries * geom.q_heads * D * 2
    return {
        "hot": B * nh * Hkv * D * 2 + q + B * geom.hot_count * 4,
        "cold": B * nc * Hkv * 16 + B * geom.cold_count * 4,
    }


def cpu_baseline(seconds: float, seed: int):
    """Oracle fp32 restatement of weaver_kernel.metal on this host: B = 1 steps of
    the metric's workload (hot 2048 + cold 32768), q_latent computed on the CPU."""
    import numpy as np
    from aether_nexus_amd import workloads as W
    from oracle import oracle
    build = native_oracle()
    geom = W.hot_cold(batch=1)
    wl = W.generate(geom, seed=seed, device="cpu")
    arrs = W.host_arrays(wl)
    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.decode_ref32(geom, arrs, threads)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.decode_ref32(geom, arrs, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 1000:
            break
    # One thread, briefly, beside the multi-threaded figure.
    n1, t1 = 0, time.perf_counter()
    while True:
        oracle.decode_ref32(geom, arrs, 1)
        n1 += 1
        el1 = time.perf_counter() - t1
        if el1 >= min(4.0, seconds / 3) or n1 >= 100:
            break
    del np
    return {"value": n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} B=1 decode steps of hot 2048 + cold 32768 (32q/8kv d128, 4096 atoms, q_latent "
                      f"computed on the CPU) in {el:.1f} s, fp32 restatement of weaver_kernel.metal, "
                      f"{threads} threads",
            "single_thread_value": round(n1 / el1, 3), "cpu_model": cpu_model(),
            "host_cpus": os.cpu_count(), "build": build}


_NATIVE = {}


def native_oracle() -> str:
    """The timed CPU port built for this host (-O3 -march=native) into a scratch
    directory and bound in place of the shipped portable build (x86-64-v3, used
    by the tests); the shipped build is kept if no compiler is here."""
    if "build" not in _NATIVE:
        import tempfile
        from oracle import oracle
        try:
            out = Path(tempfile.mkdtemp(prefix="weaver_oracle_")) / "libweaver_oracle_native.so"
            oracle.use_lib(oracle.build_native(out))
            _NATIVE["build"] = "gcc -O3 -march=native -ffp-contract=off, built on this host"
        except Exception as exc:  # no gcc/make on the host: the portable build times it
            _NATIVE["build"] = f"gcc -O3 -march=x86-64-v3 -ffp-contract=off (shipped; native build failed: {exc})"
    return _NATIVE["build"]


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its family/model/stepping and
    widest vector extension (a virtualised host may report only the brand)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                info.setdefault(k, v)
            elif info:
                break  # first processor only
    except OSError:
        return "unknown"
    flags = set(info.get("flags", "").split())
    isa = next((f for f in ("avx512f", "avx2", "avx") if f in flags), "sse")
    return (f"{info.get('model name', 'unknown')} (vendor {info.get('vendor_id', '?')}, family "
            f"{info.get('cpu family', '?')}, model {info.get('model', '?')}, stepping {info.get('stepping', '?')}, "
            f"{isa})")


def hbm_copy_peak(mib: int = 1024, reps: int = 10) -> dict:
    """A device-to-device copy of `mib` MiB: bytes read + written per second, the
    attainable HBM rate beside the 8 TB/s nominal peak."""
    import torch
    src = torch.empty((mib << 20) // 4, dtype=torch.int32, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    gbps = 2 * src.numel() * 4 * reps / (a.elapsed_time(b) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return {"gbps": round(gbps, 1), "frac_of_nominal": round(gbps / PEAK_HBM_GBPS, 4),
            "copy": f"torch copy_ of {mib} MiB int32 on one device, read + write counted"}


def hbm_read_peak(engine, mib: int = 2048, reps: int = 10) -> dict:
    """The library's read-only stream kernel (aw_debug_read_stream: 16-byte loads,
    8 in flight per lane, nothing written) over `mib` MiB, eight times the
    Infinity Cache: bytes read per second at 8, 16 and 32 waves per CU, the best
    beside the 8 TB/s nominal peak."""
    import torch
    nbytes = mib << 20
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device="cuda:0")
    sink = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    rates = {}
    for wpc in (8, 16, 32):
        with torch.cuda.stream(s):
            engine.read_stream(buf, nbytes, wpc, sink, stream=s.cuda_stream)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(s)
            for _ in range(reps):
                engine.read_stream(buf, nbytes, wpc, sink, stream=s.cuda_stream)
            b.record(s)
        torch.cuda.synchronize()
        rates[wpc] = nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9
    best = max(rates, key=rates.get)
    del buf, sink
    torch.cuda.empty_cache()
    return {"gbps": round(rates[best], 1), "frac_of_nominal": round(rates[best] / PEAK_HBM_GBPS, 4),
            "waves_per_cu": best, "by_waves_per_cu": {str(k): round(v, 1) for k, v in rates.items()},
            "read": f"aw_debug_read_stream over {mib} MiB, {reps} passes, bytes read counted"}


def pool_gather_rate(engine, runner, reps: int = 20) -> dict:
    """The attainable rate of the decode's own pool reads (aw_debug_read_pools):
    every hot row and cold code of the runner's request through its block table,
    in the pools' layouts, nothing computed, rotating over the same pool copies
    as the timed steps.  Bytes counted: the hot rows, the codes and the block
    refs of both pools."""
    import torch
    from aether_nexus_amd.types import BLOCK_SIZE
    g = runner.geom
    B, Hkv, D = g.batch * g.layers, g.kv_heads, g.head_dim
    nbytes = B * Hkv * (g.hot_count * BLOCK_SIZE * D * 2 + g.cold_count * BLOCK_SIZE * 16) + \
        B * (g.hot_count + g.cold_count) * 4
    sink = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    s = runner.stream
    with torch.cuda.stream(s):
        for d in runner.descs:
            engine.read_pools(d, sink, stream=s.cuda_stream)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        for i in range(reps):
            engine.read_pools(runner.descs[i % len(runner.descs)], sink, stream=s.cuda_stream)
        b.record(s)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / reps
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"gbps": round(gbps, 1), "frac_of_nominal": round(gbps / PEAK_HBM_GBPS, 4), "us": round(us, 2),
            "bytes": int(nbytes),
            "read": f"aw_debug_read_pools over the B={g.batch} request's hot rows, codes and block refs "
                    f"({'head-blocked' if runner.cold_hb is not None else 'reference-order'} cold pool, "
                    f"{len(runner.descs)} pool copies), {reps} passes"}


# BASELINE configurations timed beside the sweep (config 3 is the sweep at B = 1).
CONFIGS = {
    "2": "hot-only exact f16 decode, 32q/8kv heads, head_dim 128, hot 4096 tokens, no cold pool, B=1, "
         "one query, scale 1/sqrt(128)",
    "4": "batched hot+cold decode, B=64, hot 1024 f16 tokens + cold 131072 SparseCodes per kv head "
         "(Zipf(1.1) atom indices), shared 4096x128 dictionary, 32q/8kv, head_dim 128",
    "5": "speculative-verify decode over 32 layers, B=8 x 8 causal draft queries, hot 2048 + cold 65536 "
         "per kv head, per-layer 4096x128 dictionary, 32q/8kv, head_dim 128",
}


def config_geom(key: str):
    from aether_nexus_amd import workloads as W
    return {"2": W.hot_only, "4": W.batched, "5": W.spec_verify}[key]()


def config_line(engine, key: str, args) -> dict:
    """One BASELINE configuration, timed like the sweep (HIP graph replay, pools
    rotated past the Infinity Cache), with its dominant bandwidth-bound kernel."""
    import torch
    from dataclasses import replace
    g0 = config_geom(key)
    geom = replace(g0, copies=copies_for(g0))
    hb = args.cold_layout == "head_blocked" and g0.cold_count > 0
    r = Runner(engine, geom, args.seed, not args.no_graph, cold_head_blocked=hb, steps_per_graph=args.steps_per_graph)
    ms, spg, by_spg = r.time_best(args.steps, args.warmup)
    ab = geom.algorithmic_bytes()["total"]
    gbps = ab / (ms * 1e-3) / 1e9
    stages, serial = stage_pair(r, args)
    kb = kernel_bytes(geom)
    dom = max((k for k in ("hot", "cold") if serial[k][0]), key=lambda k: serial[k][0], default="hot")
    pipe, alone = stages[dom][0] or math.nan, serial[dom][0] or math.nan
    row = {"config": key, "workload": CONFIGS[key], "layers": geom.layers, "batch": geom.batch,
           "queries": geom.queries, "tokens_per_step": geom.tokens, "ms_per_step": round(ms, 5),
           "steps_per_graph": spg, "ms_per_step_by_steps_per_graph": by_spg,
           "tokens_per_s": round(geom.tokens / (ms * 1e-3), 1), "alg_bytes_per_step": int(ab),
           "achieved_gbps": round(gbps, 1), "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4),
           "cold_layout": ("head_blocked" if hb else "reference") if g0.cold_count else None,
           "copies": geom.copies,
           "dominant_kernel": {"kernel": f"{dom}_kernel", "alg_bytes_per_launch": int(kb[dom]),
                               "avg_launch_us": round(pipe * 1e3, 2),
                               "frac": round(kb[dom] / (pipe * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                               "serialized_launch_us": round(alone * 1e3, 2),
                               "serialized_frac": round(kb[dom] / (alone * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)},
           "stages_us": {k: (round(v * 1e3, 2) if v else None) for k, (v, n) in stages.items()},
           "stages_serial_us": {k: (round(v * 1e3, 2) if v else None) for k, (v, n) in serial.items()}}
    del r
    torch.cuda.empty_cache()
    return row


VALU_FP32_FMA_TFLOPS = 78.6  # 256 CUs x 128 fp32 FMA lanes x 2.4 GHz x 2 (no packed fp32 here)
MFMA_F16_TFLOPS = 2500.0     # dense f16 MFMA
VALU_DOT2_F16_TFLOPS = 157.3  # v_dot2_f32_f16: two f16 products per lane and cycle


def projection_table(engine, seed, steps=50):
    """q_latent = q . D^T (YELLOWPAPER.md:86-92) on MFMA tiles (project_kernel)
    and on the vector ALUs (project_valu_kernel), serialized stage time of each
    path over `steps` decodes, at several rows per dictionary group; `planner`
    is the path aw_engine_set_projection(AUTO) takes there."""
    import torch
    from aether_nexus_amd import workloads as W
    from aether_nexus_amd.types import AW_PROJECT_AUTO, AW_PROJECT_MFMA, AW_PROJECT_VALU
    from aether_nexus_amd.weaver import plan
    cases = [("4 rows per group: one query, 8 per-kv-head dictionaries of 512 atoms",
              W.hot_cold(batch=1, dict_size=512, dict_heads=8)),
             ("16 rows per group: 4 queries, 8 per-kv-head dictionaries of 512 atoms",
              W.hot_cold(batch=1, queries=4, causal=True, dict_size=512, dict_heads=8)),
             ("32 rows: B = 1, shared 4096-atom dictionary", W.sweep(1)),
             ("256 rows: B = 8, shared 4096-atom dictionary", W.sweep(8)),
             ("2048 rows: B = 64, shared 4096-atom dictionary", W.sweep(64))]
    st = torch.cuda.current_stream().cuda_stream
    rows = []
    try:
        for name, geom in cases:
            wl = W.generate(geom, seed=seed, device="cuda:0")
            out = torch.empty(wl.out_shape(), dtype=torch.float16, device="cuda:0")
            desc = W.device_desc(wl, out)
            per_group = geom.batch * geom.queries * (geom.q_heads if geom.dict_heads == 1 else
                                                       geom.q_heads // geom.kv_heads)
            flops = 2.0 * geom.layers * geom.batch * geom.queries * geom.q_heads * geom.dict_size * geom.head_dim
            row = {"case": name, "rows_per_group": per_group, "groups": geom.layers * geom.dict_heads,
                   "atoms": geom.dict_size, "gflop": round(flops / 1e9, 4)}
            for key, mode in (("mfma", AW_PROJECT_MFMA), ("valu", AW_PROJECT_VALU)):
                engine.set_projection(mode)
                engine.decode_device(desc, stream=st)
                engine.reset_stage_stats()
                engine.set_profiling(2)
                for _ in range(steps):
                    engine.decode_device(desc, stream=st)
                torch.cuda.synchronize()
                engine.set_profiling(0)
                ms, n = engine.stage_stats()["project"]
                us = ms / n * 1e3
                tf = flops / (us * 1e-6) / 1e12
                peak = MFMA_F16_TFLOPS if key == "mfma" else VALU_DOT2_F16_TFLOPS
                row[key] = {"us": round(us, 2), "tflops": round(tf, 2), "frac_of_peak": round(tf / peak, 4),
                            "peak_tflops": peak}
            row["planner"] = "valu" if plan(desc).projection == AW_PROJECT_VALU else "mfma"
            rows.append(row)
            log(json.dumps(row))
            del wl, out, desc
            torch.cuda.empty_cache()
    finally:
        engine.set_projection(AW_PROJECT_AUTO)
        engine.set_profiling(0)
    return {"note": "serialized stage time (HIP events) of the projection alone; peaks: f16 MFMA dense for "
                    "project_kernel, v_dot2_f32_f16 on every lane for project_valu_kernel",
            "rows": rows}


def encoder_bench(engine, seed, reps, cpu_blocks):
    """SparseCode encoder (distiller.rs:171-246) on the reference geometry
    (Llama8B: 8 kv heads, head_dim 128, 512 atoms per kv head) over 8192 hot
    blocks, the most one find_candidates pass hands over (distiller.rs:107), with
    the entropy proxy; the CPU oracle is timed on `cpu_blocks` of them."""
    import numpy as np
    import torch
    from aether_nexus_amd.weaver import make_encode_desc
    hkv, hd, a, nb = 8, 128, 512, 8192
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    hot = torch.randn((nb, 16, hkv, hd), generator=g, device="cuda:0").to(torch.float16)
    dd = torch.randn((hkv, a, hd), generator=g, device="cuda:0", dtype=torch.float64)
    dic = (dd / dd.norm(dim=-1, keepdim=True)).to(torch.float16)
    src = torch.randperm(nb, generator=g, device="cuda:0").to(torch.int32)
    cold = torch.zeros((nb, 16, hkv, 8), dtype=torch.int16, device="cuda:0")
    ent = torch.zeros(nb, dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream()

    def timed(full_scan):
        desc = make_encode_desc(kv_heads=hkv, head_dim=hd, dict_size=a, dict_heads=hkv, hot_blocks=nb, cold_blocks=nb,
                                hot=hot, dictionary=dic, src_blocks=src, cold=cold, entropy=ent, full_scan=full_scan)
        engine.encode_device(desc, stream=st.cuda_stream)
        engine.check_device_errors(st.cuda_stream)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(st)
        for _ in range(reps):
            engine.encode_device(desc, stream=st.cuda_stream)
        ev[1].record(st)
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / reps

    scan_ms = timed(True)
    scan_codes = cold.clone()
    ms = timed(False)
    tok_heads = nb * 16 * hkv
    flops = 2.0 * tok_heads * a * hd  # the projection x . D^T, counted once
    # CPU oracle on the first blocks of the same pools (one thread), checked against the GPU's codes.
    from oracle import oracle
    hot_h = hot.cpu().numpy().view(np.uint16)
    dic_h = dic.cpu().numpy().view(np.uint16)
    src_h = src.cpu().numpy().astype(np.uint32)[:cpu_blocks]
    t0 = time.perf_counter()
    want = oracle.encode_blocks(hot_h, dic_h, src_h, cold=np.zeros((nb, 16, hkv, 8), np.uint16))
    cpu_s = time.perf_counter() - t0
    got = cold.cpu().numpy().view(np.uint16)
    same = bool((got[src_h] == want[src_h]).all()) and bool(torch.equal(cold, scan_codes))
    tf = flops / (ms * 1e-3) / 1e12
    scan_tf = flops / (scan_ms * 1e-3) / 1e12
    return {"workload": f"{nb} blocks x 16 tokens x {hkv} kv heads, head_dim {hd}, {a} atoms per kv head, "
                        "entropy proxy included (on a side stream beside the encoder)",
            "ms_per_call": round(ms, 4), "blocks_per_s": round(nb / (ms * 1e-3), 1),
            "token_heads_per_s": round(tok_heads / (ms * 1e-3), 1),
            "achieved_tflops": round(tf, 2),
            "roofline": {"bound": "mfma", "peak_tflops": MFMA_F16_TFLOPS, "frac": round(tf / MFMA_F16_TFLOPS, 4),
                         "note": "the projection x . D^T (counted once) runs twice on MFMA, f16 in, f32 out, then the "
                                 "candidate atoms are rescored in the reference's fp32 order; the per-score bound and "
                                 "top-4 bookkeeping on the VALU bounds the kernel, not the matrix cores"},
            "full_scan": {"ms_per_call": round(scan_ms, 4), "achieved_tflops": round(scan_tf, 2),
                          "valu_frac": round(scan_tf / VALU_FP32_FMA_TFLOPS, 4), "valu_peak_tflops": VALU_FP32_FMA_TFLOPS,
                          "note": "AW_F_ENCODE_FULL_SCAN: one exact fp32 FMA per (token, kv head, atom, dim); same codes"},
            "cpu_baseline": {"value": round(cpu_blocks / cpu_s, 2), "unit": "blocks/s", "cores": 1, "kind": "port",
                             "build": native_oracle(),
                             "sample": f"{cpu_blocks} blocks through the oracle's restatement of distiller.rs:171-246"},
            "codes_match_cpu": same}


def attention_bench(engine, seed, reps, cpu_seconds):
    """The Weaver as the inference loop's attention (Ops::multihead_attention,
    ops.metal:528-616): one forward's attention over the 32 layers of
    Llama-3.1-8B (32q/8kv, head_dim 128) with every layer's K and V caches at
    MAX_SEQ_LEN = 4096 tokens (inference.rs:219), for a decode step (1 new token)
    and a verify step (last token + 3 drafts, agent.rs:337-355), captured in a
    HIP graph.  Algorithmic bytes per layer: the K and V rows read (4096 x 8 x 128
    x 2 bytes each) plus q and out."""
    import numpy as np
    import torch
    from types import SimpleNamespace
    layers, hq, hkv, hd, kv_len = 32, 32, 8, 128, 4096
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    kc = [torch.randn((kv_len, hkv, hd), generator=g, device="cuda:0").to(torch.float16) for _ in range(layers)]
    vc = [torch.randn((kv_len, hkv, hd), generator=g, device="cuda:0").to(torch.float16) for _ in range(layers)]
    res = {"workload": f"{layers} layers x multihead_attention over K and V caches of {kv_len} tokens, "
                       f"{hq}q/{hkv}kv heads, head_dim {hd} (Llama-3.1-8B at MAX_SEQ_LEN)"}
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    for name, nq in (("decode", 1), ("verify_3_drafts", 4)):
        q = torch.randn((nq, hq, hd), generator=g, device="cuda:0").to(torch.float16)
        outs = [torch.empty((nq, hq, hd), dtype=torch.float16, device="cuda:0") for _ in range(layers)]
        with torch.cuda.stream(st):
            def forward(s):
                for l in range(layers):
                    engine.multihead_attention(q, kc[l], vc[l], outs[l], kv_len, hd, hq, hkv, nq,
                                               cache_tokens=kv_len, stream=s)
            forward(st.cuda_stream)  # sizes the workspace and the block table before capture
            engine.check_device_errors(st.cuda_stream)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=st):
                forward(torch.cuda.current_stream().cuda_stream)
            for _ in range(3):
                graph.replay()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record(st)
            for _ in range(reps):
                graph.replay()
            ev[1].record(st)
        torch.cuda.synchronize()
        ms = ev[0].elapsed_time(ev[1]) / reps
        alg = layers * (kv_len * hkv * hd * 2 * 2 + 2 * nq * hq * hd * 2)
        gbps = alg / (ms * 1e-3) / 1e9
        res[name] = {"new_tokens": nq, "ms_per_forward": round(ms, 4), "us_per_layer": round(ms * 1e3 / layers, 2),
                     "alg_bytes_per_forward": alg, "achieved_gbps": round(gbps, 1),
                     "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4)}
        log(f"attention: {name} {res[name]['us_per_layer']} us per layer")
        del graph
    res["tiered"] = tiered_attention_bench(engine, seed, reps)
    res["dense_at_tiered_length"] = dense_attention_at(engine, seed, reps, kv_len=2048 + 32768)
    log(f"attention: dense cache of {2048 + 32768} tokens {res['dense_at_tiered_length']['us_per_layer']} us per layer")
    # CPU: the oracle's fp32 restatement of the same attention (a hot pool of
    # 16-token blocks, identity block table, causal) on one layer of the decode step.
    from oracle import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
    geom = SimpleNamespace(layers=1, batch=1, queries=1, q_heads=hq, kv_heads=hkv, head_dim=hd, dict_size=16,
                           dict_heads=1, hot_count=kv_len // 16, cold_count=0, refs_stride=kv_len // 16, causal=True,
                           scale=1.0 / math.sqrt(hd), hot_blocks=kv_len // 16, cold_blocks=0)
    arrs = {"q": q[:1].cpu().numpy().view(np.uint16), "hot_k": kc[0].cpu().numpy().view(np.uint16),
            "hot_v": vc[0].cpu().numpy().view(np.uint16), "refs": np.arange(kv_len // 16, dtype=np.uint32)}
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.decode_ref32(geom, arrs, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= cpu_seconds or n >= 2000:
            break
    res["cpu_baseline"] = {"value": round(n / el / layers, 3), "unit": "decode forwards/s (32 layers)",
                           "cores": threads, "kind": "port", "build": native_oracle(),
                           "sample": f"{n} single-layer decode attentions ({kv_len} cached tokens) through the "
                                     f"oracle's fp32 restatement in {el:.1f} s, {threads} threads"}
    res["gpu_forwards_per_s"] = round(1e3 / res["decode"]["ms_per_forward"], 1)
    return res


def dense_attention_at(engine, seed, reps, kv_len, layers=32, distinct=8):
    """The contiguous-cache attention (multihead_attention, one decode token) at the
    tiered cache's total length: what the same 32 layers cost when every token
    stays exact f16 K and V (8 distinct caches of 143 MB rotated over the layers,
    so no layer finds the previous one's in the MALL)."""
    import torch
    hq, hkv, hd = 32, 8, 128
    g = torch.Generator(device="cuda:0").manual_seed(seed + 2)
    kc = [torch.randn((kv_len, hkv, hd), generator=g, device="cuda:0").to(torch.float16) for _ in range(distinct)]
    vc = [torch.randn((kv_len, hkv, hd), generator=g, device="cuda:0").to(torch.float16) for _ in range(distinct)]
    q = torch.randn((1, hq, hd), generator=g, device="cuda:0").to(torch.float16)
    outs = [torch.empty((1, hq, hd), dtype=torch.float16, device="cuda:0") for _ in range(layers)]
    st = torch.cuda.Stream()

    def forward(s):
        for l in range(layers):
            engine.multihead_attention(q, kc[l % distinct], vc[l % distinct], outs[l], kv_len, hd, hq, hkv, 1,
                                       cache_tokens=kv_len, stream=s)
    ms = _graph_time(forward, st, reps)
    alg = layers * (kv_len * hkv * hd * 2 * 2 + 2 * hq * hd * 2)
    gbps = alg / (ms * 1e-3) / 1e9
    del kc, vc
    torch.cuda.empty_cache()
    return {"workload": f"{layers} layers x multihead_attention, one decode token over contiguous K and V caches of "
                        f"{kv_len} tokens ({distinct} distinct caches rotated), 32q/8kv heads, head_dim 128",
            "us_per_layer": round(ms * 1e3 / layers, 2), "alg_bytes_per_forward": alg,
            "achieved_gbps": round(gbps, 1), "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4),
            "cache_bytes_per_token_and_layer": hkv * hd * 2 * 2}


def tiered_attention_bench(engine, seed, reps, layers=32, hot=2048, cold=32768):
    """The same forward's attention over WeaverKvCache: per layer a hot window of
    2048 exact K and V tokens plus 32768 cold tokens distilled into SparseCodes of
    the layer's 512-atom per-kv-head dictionaries (the reference's Llama8B
    geometry), one hot+cold aw_decode_device per layer with q_latent computed on
    the device, the 32 layers captured in a HIP graph; the cold kernel's value
    partials (the planner's path here) and its bins + finish path, each timed.
    Algorithmic bytes per layer: hot K and V rows, cold codes, the dictionary,
    block refs, q and out."""
    import torch
    from aether_nexus_amd.inference import WeaverKvCache
    hq, hkv, hd, atoms = 32, 8, 128, 512
    g = torch.Generator(device="cuda:0").manual_seed(seed + 1)
    dd = torch.randn((layers, hkv, atoms, hd), generator=g, device="cuda:0", dtype=torch.float32)
    dicts = (dd / dd.norm(dim=-1, keepdim=True)).to(torch.float16)
    n = hot + cold
    cache = WeaverKvCache(layers, hkv, hd, dicts, hot_window=hot, max_seq_len=n + 64)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):  # a prompt of n tokens per layer (K rows reused as V rows)
        ks = [torch.randn((n, hkv, hd), generator=g, device="cuda:0").to(torch.float16) for _ in range(layers)]
        cache.extend(engine, ks, ks, stream=st.cuda_stream)
    torch.cuda.synchronize()
    del ks
    log(f"tiered: prompt of {n} tokens per layer loaded ({cache.cold_tokens} cold)")
    res = {"workload": f"{layers} layers x Weaver attention over a hot window of {hot} f16 K/V tokens + {cold} "
                       f"cold SparseCodes per kv head ({atoms}-atom per-kv-head dictionaries), {hq}q/{hkv}kv "
                       f"heads, head_dim {hd}",
           "cold_tokens": cache.cold_tokens, "hot_tokens": cache.hot_tokens()}
    p0 = cache.position
    from aether_nexus_amd.types import AW_COLD_OUT_AUTO, AW_COLD_OUT_BINS
    for name, nq in (("decode", 1), ("verify_3_drafts", 4)):
        q = torch.randn((nq, hq, hd), generator=g, device="cuda:0").to(torch.float16)
        rows = torch.randn((nq, hkv, hd), generator=g, device="cuda:0").to(torch.float16)
        outs = [torch.empty((nq, hq, hd), dtype=torch.float16, device="cuda:0") for _ in range(layers)]
        with torch.cuda.stream(st):
            for l in range(layers):
                cache.append(l, rows, rows)

        def forward(s):
            for l in range(layers):
                cache.attend(engine, l, q, outs[l], stream=s)
        # The planner's path (value partials at these 512-atom heads), then the
        # bins + finish path on the same cache for comparison.
        by_mode = {}
        for mode in (AW_COLD_OUT_AUTO, AW_COLD_OUT_BINS):
            engine.set_cold_output(mode)
            try:
                with torch.cuda.stream(st):
                    forward(st.cuda_stream)  # sizes the workspace and the block table before capture
                    engine.check_device_errors(st.cuda_stream)
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=st):
                        forward(torch.cuda.current_stream().cuda_stream)
                    for _ in range(3):
                        graph.replay()
                    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                    ev[0].record(st)
                    for _ in range(reps):
                        graph.replay()
                    ev[1].record(st)
                torch.cuda.synchronize()
            finally:
                engine.set_cold_output(AW_COLD_OUT_AUTO)
            by_mode[mode] = ev[0].elapsed_time(ev[1]) / reps
            log(f"tiered: {name}, cold output {'auto' if mode == AW_COLD_OUT_AUTO else 'bins'}: "
                f"{by_mode[mode] * 1e3 / layers:.2f} us per layer")
            del graph
        ms = by_mode[AW_COLD_OUT_AUTO]
        n_hot = hot + nq
        alg = layers * (n_hot * hkv * hd * 2 * 2 + cold * hkv * 16 + hkv * atoms * hd * 2
                        + (-(-n_hot // 16) + cold // 16) * 4 + 2 * nq * hq * hd * 2)
        gbps = alg / (ms * 1e-3) / 1e9
        res[name] = {"new_tokens": nq, "ms_per_forward": round(ms, 4), "us_per_layer": round(ms * 1e3 / layers, 2),
                     "alg_bytes_per_forward": alg, "achieved_gbps": round(gbps, 1),
                     "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4),
                     "bins_path_us_per_layer": round(by_mode[AW_COLD_OUT_BINS] * 1e3 / layers, 2)}
        cache.pop_loom(p0)
    del cache
    torch.cuda.empty_cache()
    return res


# Llama-3.1-8B, the dense shapes of the inference loop (inference.rs:13-159 presets).
LLAMA8B = dict(hidden=4096, q_heads=32, kv_heads=8, head_dim=128, inter=14336, vocab=128256, layers=32, eps=1e-5,
               theta=500000.0, max_seq=4096)
PEAK_F16_TFLOPS = 2500.0


def _graph_time(fn, st, reps):
    """ms per replay of `fn(stream)` captured in a HIP graph (one eager call first),
    after the work already queued on torch's current stream (the inputs)."""
    import torch
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn(st.cuda_stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            fn(torch.cuda.current_stream().cuda_stream)
        for _ in range(2):
            graph.replay()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(st)
        for _ in range(reps):
            graph.replay()
        ev[1].record(st)
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    del graph
    return ms


def ops_bench(engine, seed, read_peak_gbps, reps=10, forwards=True):
    """The dense ops (ops.metal:16-635) on MI355X at Llama-3.1-8B shapes.

    * Each product of a layer, one launch at a time: decode (M = 1) and verify
      (M = 16, forward_batch's MAX_BATCH) are bound by the weight bytes (N*K*2,
      plus activations and output), measured against 8 TB/s and the read-only
      stream peak; prefill-sized M = 2048 by the matrix cores (2*M*N*K flops
      against 2.5 PFLOP/s f16).  The weights are rotated over copies that
      together exceed the 256 MiB Infinity Cache, so the bytes come from HBM.
    * One whole decode forward (InferenceEngine::forward_batch,
      inference.rs:456-634): embedding, 32 layers of RMSNorm, q/k/v products,
      RoPE, the cache append, multihead attention over 4096 cached tokens, the
      output product, residual, RMSNorm, gated MLP and residual, then the final
      norm and the f32 lm_head, captured in one HIP graph, random weights.
      Bytes per forward: every weight once plus the K and V caches read.  The
      "_fused" forwards make the same computation with the fused products (q/k/v
      in one launch, the residual adds and the SiLU gate in the products'
      stores) and must give the same logits bit for bit."""
    import torch
    from aether_nexus_amd.ops import OpsEngine
    c = LLAMA8B
    ops = OpsEngine(engine)
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())

    def randn(*shape, std=1.0):
        return (torch.randn(shape, generator=g, device="cuda:0") * std).to(torch.float16)

    H, I, V = c["hidden"], c["inter"], c["vocab"]
    kvd = c["kv_heads"] * c["head_dim"]
    shapes = [("q_proj, o_proj", H, H), ("k_proj, v_proj", kvd, H), ("gate_proj, up_proj", I, H),
              ("down_proj", H, I), ("lm_head (f32, scaled)", V, H)]
    products = []
    for name, n, k in shapes:
        copies = max(1, min(16, math.ceil(2 * MALL_BYTES / (n * k * 2))))
        ws = [randn(n, k, std=k ** -0.5) for _ in range(copies)]
        scaled = name.startswith("lm_head")
        for m in (1, 16, 2048):
            if m == 2048 and scaled:
                continue
            a = randn(m, k)
            outs = [torch.empty((m, n), dtype=torch.float32 if scaled else torch.float16, device="cuda:0")
                    for _ in range(copies)]
            launches = copies * max(1, 64 // copies) if m < 2048 else copies * 2

            def fn(s, ws=ws, a=a, outs=outs, m=m, n=n, k=k, scaled=scaled, launches=launches):
                for i in range(launches):
                    j = i % len(ws)
                    if scaled:
                        ops.matmul_scaled(a, ws[j], outs[j], m, n, k, 1.0 / 8.0, stream=s)
                    else:
                        ops.matmul(a, ws[j], outs[j], m, n, k, stream=s)
            us = _graph_time(fn, st, 3) * 1e3 / launches
            row = {"product": name, "m": m, "n": n, "k": k, "us": round(us, 2)}
            if m < 2048:
                nbytes = n * k * 2 + m * k * 2 + m * n * (4 if scaled else 2)
                gbps = nbytes / (us * 1e-6) / 1e9
                row.update(bound="hbm", bytes=nbytes, achieved_gbps=round(gbps, 1),
                           frac_of_peak=round(gbps / PEAK_HBM_GBPS, 4), frac_of_read_peak=round(gbps / read_peak_gbps, 4))
            else:
                tf = 2.0 * m * n * k / (us * 1e-6) / 1e12
                row.update(bound="mfma", flops=2 * m * n * k, achieved_tflops=round(tf, 1),
                           frac_of_peak=round(tf / PEAK_F16_TFLOPS, 4))
            products.append(row)
            log(json.dumps(row))
            del outs, a
        del ws
        torch.cuda.empty_cache()
    res = {"workload": "Llama-3.1-8B shapes: hidden 4096, 32q/8kv heads x 128, MLP 14336, vocab 128256",
           "products": products}
    if not forwards:
        return res

    # One decode forward of 32 layers.
    L, hq, hkv, hd, S = c["layers"], c["q_heads"], c["kv_heads"], c["head_dim"], c["max_seq"]
    lw = [{"ln1": randn(H, std=0.1) + 1, "ln2": randn(H, std=0.1) + 1, "wq": randn(H, H, std=H ** -0.5),
           "wk": randn(kvd, H, std=H ** -0.5), "wv": randn(kvd, H, std=H ** -0.5), "wo": randn(H, H, std=H ** -0.5),
           "wg": randn(I, H, std=H ** -0.5), "wu": randn(I, H, std=H ** -0.5), "wd": randn(H, I, std=I ** -0.5),
           "kc": randn(S, hkv, hd), "vc": randn(S, hkv, hd)} for _ in range(L)]
    embed, lm_head, final_ln = randn(V, H), randn(V, H, std=H ** -0.5), randn(H, std=0.1) + 1
    res["forward"] = {}
    ref_logits = {}
    # decode, then verify: each fused run directly after the separate calls it must equal (a
    # forward rewrites the cache rows at its own positions, which the other step type reads).
    for name, t, fused in (("decode", 1, False), ("decode_fused", 1, True), ("verify_3_drafts", 4, False),
                           ("verify_3_drafts_fused", 4, True)):
        pos = S - t  # the new tokens fill the cache's last positions: attention over all 4096
        ids = torch.arange(t, dtype=torch.int32, device="cuda:0") * 7919 + 11
        hid, norm = (torch.empty((t, H), dtype=torch.float16, device="cuda:0") for _ in range(2))
        q, k, v = (torch.empty((t, n), dtype=torch.float16, device="cuda:0") for n in (H, kvd, kvd))
        att, proj, down = (torch.empty((t, H), dtype=torch.float16, device="cuda:0") for _ in range(3))
        gate, up, ffn = (torch.empty((t, I), dtype=torch.float16, device="cuda:0") for _ in range(3))
        logits = torch.empty((t, V), dtype=torch.float32, device="cuda:0")

        def forward(s, t=t, pos=pos, ids=ids, hid=hid, norm=norm, q=q, k=k, v=v, att=att, proj=proj, down=down,
                    gate=gate, up=up, ffn=ffn, logits=logits):
            ops.embed_lookup(ids, embed, hid, H, t, V, stream=s)
            for w in lw:
                if fused:  # the same bits in 10 launches per layer instead of 16
                    ops.rms_norm(hid, w["ln1"], norm, H, t, c["eps"], stream=s)
                    ops.matmul_qkv(norm, w["wq"], w["wk"], w["wv"], q, k, v, t, H, kvd, H, stream=s)
                    ops.rope(q, k, t, hq, hkv, hd, pos, c["theta"], stream=s)
                    ops.copy_buffer(k, w["kc"], kvd * t, 0, pos * kvd, stream=s)
                    ops.copy_buffer(v, w["vc"], kvd * t, 0, pos * kvd, stream=s)
                    ops.multihead_attention(q, w["kc"], w["vc"], att, pos + t, hd, hq, hkv, t, cache_tokens=S,
                                            stream=s)
                    ops.matmul_add_residual(att, w["wo"], hid, t, H, H, 1.0, stream=s)
                    ops.rms_norm(hid, w["ln2"], norm, H, t, c["eps"], stream=s)
                    ops.matmul_silu_gate(norm, w["wg"], w["wu"], ffn, t, I, H, stream=s)
                    ops.matmul_add_residual(ffn, w["wd"], hid, t, H, I, 1.0, stream=s)
                    continue
                ops.rms_norm(hid, w["ln1"], norm, H, t, c["eps"], stream=s)
                ops.matmul(norm, w["wq"], q, t, H, H, stream=s)
                ops.matmul(norm, w["wk"], k, t, kvd, H, stream=s)
                ops.matmul(norm, w["wv"], v, t, kvd, H, stream=s)
                ops.rope(q, k, t, hq, hkv, hd, pos, c["theta"], stream=s)
                ops.copy_buffer(k, w["kc"], kvd * t, 0, pos * kvd, stream=s)
                ops.copy_buffer(v, w["vc"], kvd * t, 0, pos * kvd, stream=s)
                ops.multihead_attention(q, w["kc"], w["vc"], att, pos + t, hd, hq, hkv, t, cache_tokens=S, stream=s)
                ops.matmul(att, w["wo"], proj, t, H, H, stream=s)
                ops.add_residual(hid, proj, H * t, stream=s)
                ops.rms_norm(hid, w["ln2"], norm, H, t, c["eps"], stream=s)
                ops.matmul(norm, w["wg"], gate, t, I, H, stream=s)
                ops.matmul(norm, w["wu"], up, t, I, H, stream=s)
                ops.silu_gate(gate, up, ffn, I * t, stream=s)
                ops.matmul(ffn, w["wd"], down, t, H, I, stream=s)
                ops.add_residual(hid, down, H * t, stream=s)
            ops.rms_norm(hid, final_ln, norm, H, t, c["eps"], stream=s)
            ops.matmul_scaled(norm, lm_head, logits, t, V, H, 1.0, stream=s)
        ms = _graph_time(forward, st, reps)
        ops.check_device_errors(st.cuda_stream)
        assert torch.isfinite(logits).all(), "non-finite logits"
        # Every replay starts from the same embedding rows and rewrites the same cache
        # positions, so the fused forward must give the unfused one's logits bit for bit.
        base = name.replace("_fused", "")
        if fused:
            same = bool(torch.equal(logits, ref_logits[base]))
            assert same, f"{name}: logits differ from the separate calls"
        else:
            ref_logits[name] = logits.clone()
        nbytes = L * (2 * H * H + 2 * kvd * H + 3 * I * H + 2 * H) * 2 + V * H * 2 + L * 2 * S * kvd * 2
        gbps = nbytes / (ms * 1e-3) / 1e9
        res["forward"][name] = {"new_tokens": t, "fused": fused, "launches_per_layer": 10 if fused else 16,
                                "ms_per_forward": round(ms, 4), "tokens_per_s": round(t / (ms * 1e-3), 1),
                                "bytes_per_forward": nbytes, "achieved_gbps": round(gbps, 1),
                                "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4),
                                "frac_of_read_peak": round(gbps / read_peak_gbps, 4)}
        log(json.dumps({name: res["forward"][name]}))
    res["forward"]["workload"] = (f"InferenceEngine::forward_batch at Llama-3.1-8B: {L} layers, random f16 weights, "
                                  f"K/V caches of {S} tokens per layer, f32 lm_head over {V} tokens, one HIP graph")
    del lw, embed, lm_head
    torch.cuda.empty_cache()
    return res


PCIE_GEN5_X16_GBPS = 63.0  # per direction: 32 GT/s x 16 lanes x 128/130 encoding / 8 bits


def fabric_bench(engine, seed, cpu_blocks):
    """The Llama8B `.aether` fabric (hot pool 256 MiB, cold pool 64 MiB, dictionary
    1 MiB; fabric.rs:124-186): upload of its three pools into HBM, write-back of the
    cold pool into the mapping, and one Distiller REM cycle (distiller.rs:60-120)
    over its 8192 hot blocks, all of them candidates (rows ~ N(0, 0.3): variance
    proxy ~0.09 < 0.15).  The CPU oracle is timed on `cpu_blocks` blocks of the cycle."""
    import tempfile

    import numpy as np
    from aether_nexus_amd import fabric as F
    from oracle import oracle
    dims = F.model_dims("llama8b")
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "llama8b.aether")
        F.create_genesis(path, dims)
        fab = F.Fabric(path, dims)
        try:
            rng = np.random.default_rng(seed)
            hot = fab.hot_pool_blocks(writable=True)
            for b0 in range(0, hot.shape[0], 512):
                hot[b0:b0 + 512] = (rng.standard_normal((512,) + hot.shape[1:], dtype=np.float32) * 0.3).astype(
                    np.float16).view(np.uint16)
            dd = rng.standard_normal(fab.dictionary_atoms().shape)
            fab.dictionary_atoms(writable=True)[...] = (dd / np.linalg.norm(dd, axis=-1, keepdims=True)).astype(
                np.float16).view(np.uint16)
            # A fabric in service holds codes in its cold pool (its file blocks exist).
            codes = fab.cold_pool_blocks(writable=True)
            codes["indices"] = rng.integers(0, dims.dict_size, codes["indices"].shape)
            codes["coeffs"] = (rng.standard_normal(codes["coeffs"].shape) * 0.5).astype(np.float16)
            del codes
            fab.force_checkpoint()
            pools = ("hot", "cold", "dict")
            r = fab.regions
            nbytes = r.hot_pool_size + r.cold_pool_size + r.dict_size
            t0 = time.perf_counter()
            fab.attach_device(0, pools)
            first = time.perf_counter() - t0
            t0 = time.perf_counter()
            for _ in range(3):
                for name in pools:
                    fab.push(name)
            up = (time.perf_counter() - t0) / 3
            t0 = time.perf_counter()
            for _ in range(3):
                fab.pull("cold")
            down = (time.perf_counter() - t0) / 3
            # The device cold pool kept head-blocked: copies reorder whole blocks on the device.
            fab.attach_device(0, ("cold",), cold_head_blocked=True)
            t0 = time.perf_counter()
            for _ in range(3):
                fab.push("cold")
            up_hb = (time.perf_counter() - t0) / 3
            t0 = time.perf_counter()
            for _ in range(3):
                fab.pull("cold")
            down_hb = (time.perf_counter() - t0) / 3
            fab.force_checkpoint()
            time.sleep(0.31)  # the cycle's checkpoint then flushes, as the reference's does after a REM pass
            t0 = time.perf_counter()
            n, ent = fab.distill(engine, F.DISTILL_ENTROPY_THRESHOLD)
            cycle = time.perf_counter() - t0
            hot_h = fab.hot_pool_blocks()
            sample = np.arange(cpu_blocks, dtype=np.uint32)
            t0 = time.perf_counter()
            want_ent = [oracle.block_entropy(hot_h[b]) for b in sample]
            cands = [int(b) for b, e in zip(sample, want_ent) if 0 < e < np.float32(F.DISTILL_ENTROPY_THRESHOLD)]
            want = oracle.encode_blocks(hot_h, fab.dictionary_atoms(), cands)
            cpu_s = time.perf_counter() - t0
            got = fab.cold_pool().view(np.uint16).reshape(-1, 16, dims.kv_heads, 8)
            same = bool(np.array_equal(np.float32(want_ent).view(np.uint32), ent[:cpu_blocks].view(np.uint32))
                        and np.array_equal(got[cands], want[cands]))
            del hot, hot_h, got
        finally:
            fab.close()
    return {"workload": "Llama8B fabric: hot pool 8192 x 16 x 8 x 128 f16 (256 MiB), cold pool 32768 x 16 x 8 "
                        "SparseCodes (64 MiB), dictionary 8 x 512 x 128 f16 (1 MiB); every pool written, file in the page cache",
            "pool_bytes": int(nbytes),
            "first_attach_ms": round(first * 1e3, 2),
            "upload_ms": round(up * 1e3, 2), "upload_gbps": round(nbytes / up / 1e9, 2),
            "writeback_cold_ms": round(down * 1e3, 2), "writeback_cold_gbps": round(r.cold_pool_size / down / 1e9, 2),
            "cold_head_blocked": {"upload_gbps": round(r.cold_pool_size / up_hb / 1e9, 2),
                                  "writeback_gbps": round(r.cold_pool_size / down_hb / 1e9, 2),
                                  "note": "device cold pool in [blocks][kv_heads][16]; the REM cycle below runs on it"},
            "roofline": {"bound": "pcie", "peak_gbps": PCIE_GEN5_X16_GBPS,
                         "upload_frac": round(nbytes / up / 1e9 / PCIE_GEN5_X16_GBPS, 4),
                         "writeback_frac": round(r.cold_pool_size / down / 1e9 / PCIE_GEN5_X16_GBPS, 4)},
            "distill_cycle_ms": round(cycle * 1e3, 2), "distilled_blocks": int(n),
            "distill_blocks_per_s": round(n / cycle, 1),
            "cpu_baseline": {"value": round(cpu_blocks / cpu_s, 2), "unit": "blocks/s", "cores": 1, "kind": "port",
                             "build": native_oracle(),
                             "sample": f"entropy proxy and encoding of hot blocks 0..{cpu_blocks - 1} "
                                       "through the oracle (distiller.rs:97-246)"},
            "cycle_matches_cpu": same}


def reference_bench_config(engine, seed, steps):
    """The reference's --bench shape through the reference-compatible host API."""
    import numpy as np
    from aether_nexus_amd.types import SPARSE_CODE_DTYPE, WeaverParams
    rng = np.random.default_rng(seed)
    qh, kvh, hd, ds, hot, cold = 32, 8, 128, 512, 64, 16
    val = np.float16(0.01)
    params = WeaverParams(q_heads=qh, kv_heads=kvh, head_dim=hd, block_size=16, gqa_group=4, hot_count=hot,
                          cold_count=cold, dict_size=ds, sparsity_k=4)
    args = (np.full(qh * hd, val), np.full(qh * ds, val), np.full(hot * 16 * kvh * hd, val),
            np.zeros((hot + cold) * 16 * kvh, SPARSE_CODE_DTYPE), np.arange(hot + cold, dtype=np.uint32),
            np.full(kvh * ds * hd, val), params)
    del rng
    for _ in range(10):
        engine.decode(*args)
    t0 = time.perf_counter()
    for _ in range(steps):
        engine.decode(*args)
    el = time.perf_counter() - t0
    tps = steps / el
    return {"tokens_per_s": round(tps, 1), "ms_per_token": round(1e3 * el / steps, 4),
            "published_m1pro_tokens_per_s": 389.6, "ratio_vs_published": round(tps / 389.6, 2),
            "note": "wall clock of aw_decode incl. host->device copies of every pool and the blocking wait, "
                    "as in bench.rs:149-168; cold pool sized 80 blocks (the reference's refs 64..79 index "
                    "past its 16-block pool)"}


def rocpd_summary(db: str, name_filter: str) -> str:
    """Per-kernel summary of a rocprofv3 database (kernel trace and, when
    present, counters averaged per dispatch), grouped by kernel and grid."""
    import collections
    import sqlite3
    c = sqlite3.connect(db)
    lines = []
    dur = collections.defaultdict(list)
    try:  # grid_z separates launches that differ only in layers x dictionary groups
        rows = c.execute("select name, duration, grid_x, grid_y, grid_z, workgroup_x, vgpr_count, accum_vgpr_count, "
                         "lds_size from kernels").fetchall()
    except sqlite3.Error:
        rows = [(n, d, gx, gy, 1, w, v, a, l) for n, d, gx, gy, w, v, a, l in c.execute(
            "select name, duration, grid_x, grid_y, workgroup_x, vgpr_count, accum_vgpr_count, lds_size from kernels")]
    for name, d, gx, gy, gz, wgx, vg, ag, lds in rows:
        if name_filter in name:
            dur[(name, gx, gy, gz, wgx, vg, ag, lds)].append(d / 1e3)
    lines.append("kernel | grid | wg | vgpr | agpr | lds | launches | avg_us | min_us | max_us")
    for k, v in sorted(dur.items(), key=lambda x: -sum(x[1])):
        grid = f"{k[1]}x{k[2]}" + (f"x{k[3]}" if k[3] != 1 else "")
        lines.append(f"{k[0][:60]} | {grid} | {k[4]} | {k[5]} | {k[6]} | {k[7]} | {len(v)} | "
                     f"{sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f}")
    try:
        rows = list(c.execute("select kernel_name, grid_size, dispatch_id, counter_name, value from counters_collection"))
    except sqlite3.Error:
        rows = []
    if rows:
        per = collections.defaultdict(lambda: collections.defaultdict(float))
        nd = collections.defaultdict(set)
        for kn, gs, did, cn, v in rows:
            if name_filter in kn:
                per[(kn, gs)][cn] += v
                nd[(kn, gs)].add(did)
        lines.append("counters (average per dispatch)")
        for key in per:
            n = len(nd[key])
            lines.append(f"{key[0][:60]} | grid {key[1]} | dispatches {n} | " +
                         " ".join(f"{cn}={v / n:.0f}" for cn, v in sorted(per[key].items())))
    return "\n".join(lines)


def traffic_file(layout: str) -> Path:
    """The committed FETCH/WRITE traffic profile of the B = 64 pipeline with `layout`."""
    return ROOT / "profiles" / f"traffic_b64_{layout}.txt"


def sources_digest() -> str:
    """sha256 over the decode path's HIP sources (the kernels and their
    launches), so a traffic profile is only used for the kernels it was
    measured on.  Comments, trailing blanks and blank lines are left out, so a
    comment edit keeps a profile's digest; these sources hold no string
    literal with `//` or `/*` in it."""
    import hashlib
    import re
    h = hashlib.sha256()
    for name in ("weaver_engine.hip", "weaver_kernels.hpp"):
        f = ROOT / "aether_nexus_amd" / "csrc" / name
        code = re.sub(r"/\*.*?\*/", "", f.read_text(), flags=re.S)
        lines = (re.sub(r"//.*", "", ln).rstrip() for ln in code.splitlines())
        h.update(f.name.encode())
        h.update("\n".join(ln for ln in lines if ln).encode())
    return h.hexdigest()[:16]


def copy_calibration(mib: int, reps: int = 10):
    """A plain elementwise copy of known size (torch's bitwise_not over int32:
    reads and writes `mib` MiB once), for scaling the FETCH_SIZE / WRITE_SIZE
    counters to bytes."""
    import torch
    n = (mib << 20) // 4
    src = torch.empty(n, dtype=torch.int32, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    log(f"copy calibration: {reps} x {4 * n} bytes, {8 * n * reps / el / 1e9:.0f} GB/s read+write")
    del src, dst
    torch.cuda.empty_cache()


def _counters(db: str) -> dict:
    """(kernel name, grid) -> {counter: average per dispatch} of a rocprofv3 database."""
    import collections
    import sqlite3
    c = sqlite3.connect(db)
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    nd = collections.defaultdict(set)
    for kn, gs, did, cn, v in c.execute(
            "select kernel_name, grid_size, dispatch_id, counter_name, value from counters_collection"):
        per[(kn, gs)][cn] += v
        nd[(kn, gs)].add(did)
    return {k: {cn: v / len(nd[k]) for cn, v in d.items()} for k, d in per.items()}


def traffic_summary(fetch_db: str, write_db: str, copy_mib: int, command: str, layout: str,
                    title: str = "hot 2048 + cold 32768 per kv head, B = 64 (32q/8kv, d128, 4096 atoms)") -> str:
    """HBM bytes per launch of each aw:: kernel (largest grid = the B = 64 launch)
    from a FETCH_SIZE and a WRITE_SIZE pass, each scaled by what the counter
    reads for the calibration copy of `copy_mib` MiB in the same pass."""
    copy_bytes = copy_mib << 20
    f, w = _counters(fetch_db), _counters(write_db)

    def copy_kib(d, cn):
        cands = [(k, v[cn]) for k, v in d.items() if "bitwise_not" in k[0] and cn in v]
        if not cands:
            raise SystemExit(f"no bitwise_not calibration kernel with {cn} in the database")
        return max(cands, key=lambda kv: kv[0][1])  # the largest grid: the calibration copy
    (ck_f, cf), (ck_w, cw) = copy_kib(f, "FETCH_SIZE"), copy_kib(w, "WRITE_SIZE")
    ff, fw = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    lines = [f"# HBM traffic per launch, {title}",
             f"# command: {command}",
             f"# cold_layout: {layout}",
             f"# sources: {sources_digest()}",
             f"copy_bytes {copy_bytes} kernel {ck_f[0][:48]!r} fetch_kib {cf:.0f} write_kib {cw:.0f}",
             f"factor_fetch {ff:.4f} factor_write {fw:.4f}"]
    best = {}
    for (kn, gs), v in f.items():
        if "aw::" in kn and "FETCH_SIZE" in v:
            short = kn.split("(")[0].split("::")[-1].split("<")[0]
            if short not in best or gs > best[short][1]:
                best[short] = (kn, gs)
    for short, key in sorted(best.items()):
        fk = f[key]["FETCH_SIZE"]
        wk = w.get(key, {}).get("WRITE_SIZE", float("nan"))
        tb = fk * 1024 * ff + wk * 1024 * fw
        lines.append(f"kernel {short} grid {key[1]} fetch_kib {fk:.0f} write_kib {wk:.0f} traffic_bytes {tb:.0f}")
    return "\n".join(lines)


def read_traffic(kernel: str, layout: str):
    """Traffic bytes per launch of `kernel` from the committed profile of the
    cold-pool `layout`, or (None, reason) when absent or measured on other sources."""
    f = traffic_file(layout)
    if not f.exists():
        return None, f"no traffic profile for the {layout} cold layout"
    txt = f.read_text().splitlines()
    digest = next((ln.split()[-1] for ln in txt if ln.startswith("# sources:")), None)
    measured = next((ln.split()[-1] for ln in txt if ln.startswith("# cold_layout:")), None)
    if measured != layout:
        return None, f"traffic profile measured with the {measured} cold layout"
    if digest != sources_digest():
        return None, "traffic profile measured on other kernel sources"
    for ln in txt:
        p = ln.split()
        if len(p) >= 10 and p[0] == "kernel" and p[1] == kernel:
            return int(float(p[p.index("traffic_bytes") + 1])), None
    return None, f"{kernel} missing from traffic profile"


def main():
    args = parse()
    if args.rocpd_summary:
        print(rocpd_summary(args.rocpd_summary, args.kernel_filter))
        return 0
    if args.traffic_summary:
        extra = {"title": args.traffic_title} if args.traffic_title else {}
        print(traffic_summary(args.traffic_summary[0], args.traffic_summary[1], args.copy_calibration or 256,
                              args.traffic_command, args.cold_layout, **extra))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the Weaver path shards by sequence / kv head with no exchange)",
              file=sys.stderr)
        return 2
    import torch
    from aether_nexus_amd import workloads as W
    from aether_nexus_amd.weaver import WeaverEngine

    batches = [int(x) for x in args.batches.split(",") if x]
    if not args.no_cpu:
        log(f"CPU port: {native_oracle()}")
    engine = WeaverEngine()
    if args.trace_phase == "serial":
        engine.set_profiling(2)  # every decode's kernels one at a time on the caller's stream
        args.no_graph = True
    log(f"device: {engine.device_name()}")
    config_keys = [k for k in args.configs.split(",") if k]
    for k in config_keys:
        if k not in CONFIGS:
            print(f"unknown config {k} (choose from {', '.join(CONFIGS)})", file=sys.stderr)
            return 2
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
    if args.only_configs:
        rows = []
        for k in config_keys:
            rows.append(config_line(engine, k, args))
            log(json.dumps(rows[-1]))
        engine.close()
        print(json.dumps({"configs": rows}), flush=True)
        return 0
    if args.only_projection:
        out = projection_table(engine, args.seed)
        engine.close()
        print(json.dumps({"projection_paths": out}), flush=True)
        return 0
    if args.only_attention:
        out = attention_bench(engine, args.seed, 20, 0.5 if args.no_cpu else 3.0)
        engine.close()
        print(json.dumps({"inference_attention": out}), flush=True)
        return 0
    if args.only_ops or args.only_products:
        rp = hbm_read_peak(engine)
        out = ops_bench(engine, args.seed, rp["gbps"], forwards=not args.only_products)
        engine.close()
        print(json.dumps({"hbm_read_peak": rp, "dense_ops": out}), flush=True)
        return 0
    sweep = []
    head = None
    for B in batches:
        g0 = W.sweep(B)
        geom = W.sweep(B, copies=copies_for(g0))
        r = Runner(engine, geom, args.seed, not args.no_graph, cold_head_blocked=args.cold_layout == "head_blocked",
                   steps_per_graph=args.steps_per_graph)
        ms, spg, by_spg = r.time_best(args.steps, args.warmup)
        ab = geom.algorithmic_bytes()["total"]
        gbps = ab / (ms * 1e-3) / 1e9
        row = {"batch": B, "ms_per_step": round(ms, 5), "steps_per_graph": spg,
               "ms_per_step_by_steps_per_graph": by_spg, "tokens_per_s": round(B / (ms * 1e-3), 1),
               "alg_bytes_per_step": int(ab), "achieved_gbps": round(gbps, 1),
               "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4), "copies": geom.copies}
        if args.stage_sweep:
            row["stages_us"] = {k: (round(v * 1e3, 2) if v else None)
                                for k, (v, n) in r.stage_times(max(args.steps, 10)).items()}
        log(json.dumps(row))
        sweep.append(row)
        if B == max(batches):
            head = (geom, r, row)
        else:
            del r
            torch.cuda.empty_cache()

    geom, r, row = head
    # Per-kernel durations over the same steps, launched from the host with
    # events around each kernel on its own stream (pipeline unchanged).
    stages, serial = stage_pair(r, args)
    if serial["cold"][0] is None:  # a kernel trace of one phase: nothing timed per kernel
        serial = {k: (v or math.nan, n) for k, (v, n) in serial.items()}
        stages = {k: (v or math.nan, n) for k, (v, n) in stages.items()}
    kb_per_launch = kernel_bytes(geom)
    # Dominant of the two bandwidth-bound kernels by its own (serialized) cost; its
    # duration in the pipeline of the timed steps (where the hot kernel runs
    # beside it) gives `achieved`, the serialized duration is reported beside it.
    dom = max(("hot", "cold"), key=lambda k: serial[k][0] or 0.0)
    dur_ms = stages[dom][0]
    achieved = kb_per_launch[dom] / (dur_ms * 1e-3) / 1e9
    alone = kb_per_launch[dom] / (serial[dom][0] * 1e-3) / 1e9
    traffic, why = read_traffic(f"{dom}_kernel", args.cold_layout)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic, "kernel": f"{dom}_kernel",
                "alg_bytes_per_launch": int(kb_per_launch[dom]), "avg_launch_us": round(dur_ms * 1e3, 2),
                "serialized_launch_us": round(serial[dom][0] * 1e3, 2),
                "serialized_frac": round(alone / PEAK_HBM_GBPS, 4)}
    if why:
        roofline["traffic_note"] = why
    # The phase the two bandwidth-bound kernels share: hot beside cold, from the
    # cold launch to the later of the two ends (both event pairs start together).
    phase_ms = max(stages["cold"][0] or 0.0, stages["hot"][0] or 0.0)
    if phase_ms:
        pb = kb_per_launch["hot"] + kb_per_launch["cold"]
        roofline["hot_cold_phase"] = {"alg_bytes": int(pb), "us": round(phase_ms * 1e3, 2),
                                      "achieved": round(pb / (phase_ms * 1e-3) / 1e9, 1),
                                      "frac": round(pb / (phase_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
    stages_us = {k: (round(v * 1e3, 2) if v else None) for k, (v, n) in stages.items()}
    serial_us = {k: (round(v * 1e3, 2) if v else None) for k, (v, n) in serial.items()}
    # MFMA utilisation of the two dense contractions (serialized durations): the
    # projection q . D^T and the finish bins . D (two f16 products per term: hi + lo).
    proj_flops = 2.0 * geom.layers * geom.batch * geom.queries * geom.q_heads * geom.dict_size * geom.head_dim
    mfma = {}
    for k, fl in (("project", proj_flops), ("finish", 2 * proj_flops)):
        if serial[k][0]:
            tf = fl / (serial[k][0] * 1e-3) / 1e12
            mfma[k] = {"gflop": round(fl / 1e9, 3), "tflops": round(tf, 1), "frac": round(tf / MFMA_F16_TFLOPS, 4)}
    proj_paths = None if args.skip_projection else projection_table(engine, args.seed)
    copy_peak = hbm_copy_peak()
    read_peak = hbm_read_peak(engine)
    log(json.dumps({"hbm_read_peak": read_peak}))
    gather_peak = pool_gather_rate(engine, r)
    log(json.dumps({"hbm_gather_peak": gather_peak}))
    if "hot_cold_phase" in roofline:
        ph = roofline["hot_cold_phase"]
        ph["frac_of_gather_peak"] = round(ph["achieved"] / gather_peak["gbps"], 4)
    # The same workload with the cold pool in the other order (by default the
    # reference's file order [blocks][16][kv_heads], where one kv head's code is
    # 16 bytes of every 128-byte token line): output bits must be identical.
    alt = None
    if not args.skip_alt_layout:
        other = "head_blocked" if args.cold_layout == "reference" else "reference"
        rh = Runner(engine, geom, args.seed, not args.no_graph, wl=r.wl, cold_head_blocked=other == "head_blocked",
                    steps_per_graph=args.steps_per_graph)
        ms_hb = rh.time_best(args.steps, args.warmup)[0]
        same = bool(torch.equal(rh.out.view(torch.int16), r.out.view(torch.int16)))
        gb_hb = geom.algorithmic_bytes()["total"] / (ms_hb * 1e-3) / 1e9
        alt_st = rh.stage_times(args.steps, mode=1)
        alt = {"cold_layout": other, "ms_per_step": round(ms_hb, 5),
               "tokens_per_s": round(geom.batch / (ms_hb * 1e-3), 1), "achieved_gbps": round(gb_hb, 1),
               "frac_of_peak": round(gb_hb / PEAK_HBM_GBPS, 4), "output_bit_identical": same,
               "stages_us": {k: (round(v * 1e3, 2) if v else None) for k, (v, n) in alt_st.items()}}
        if alt_st["cold"][0]:
            ach = kb_per_launch["cold"] / (alt_st["cold"][0] * 1e-3) / 1e9
            tr, why_alt = read_traffic("cold_kernel", other)
            alt["cold_roofline"] = {"achieved": round(ach, 1), "frac": round(ach / PEAK_HBM_GBPS, 4),
                                    "avg_launch_us": round(alt_st["cold"][0] * 1e3, 2), "traffic": tr}
            if why_alt:
                alt["cold_roofline"]["traffic_note"] = why_alt
        log(json.dumps({"other_cold_layout": alt}))
        del rh
        torch.cuda.empty_cache()
    configs = []
    for k in config_keys:
        configs.append(config_line(engine, k, args))
        log(json.dumps(configs[-1]))
    ref_cfg = reference_bench_config(engine, args.seed, 200)
    enc = None if args.skip_encoder else encoder_bench(engine, args.seed, 5, 8 if args.no_cpu else 32)
    if enc:
        log(json.dumps({"encoder": enc}))
    fab = None if args.skip_fabric else fabric_bench(engine, args.seed, 8 if args.no_cpu else 24)
    dense = None if args.skip_ops else ops_bench(engine, args.seed, read_peak["gbps"])
    if fab:
        log(json.dumps({"fabric": fab}))
    att = None if args.skip_attention else attention_bench(engine, args.seed, 20, 0.5 if args.no_cpu else 3.0)
    if att:
        log(json.dumps({"inference_attention": att}))
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds, args.seed)

    result = {
        "metric": METRIC,
        "value": row["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": row["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"Weaver decode, hot 2048 f16 tokens + cold 32768 SparseCodes per kv head, "
                               f"32q/8kv heads, head_dim 128, shared 4096x128 f16 dictionary, B={geom.batch}, "
                               f"one query token, scale 1/sqrt(128), cold pool {args.cold_layout} in HBM",
                   "batch": geom.batch, "hot_tokens": geom.hot_count * 16, "cold_tokens": geom.cold_count * 16,
                   "q_heads": geom.q_heads, "kv_heads": geom.kv_heads, "head_dim": geom.head_dim,
                   "dict_atoms": geom.dict_size, "cold_layout": args.cold_layout, "hip_graph": not args.no_graph,
                   "steps_per_graph": row["steps_per_graph"]},
        "achieved_gbps": row["achieved_gbps"],
        "frac_of_peak": row["frac_of_peak"],
        "frac_of_copy_peak": round(row["achieved_gbps"] / copy_peak["gbps"], 4),
        "frac_of_read_peak": round(row["achieved_gbps"] / read_peak["gbps"], 4),
        "sweep": sweep,
        "stages_us": stages_us,
        "stages_serial_us": serial_us,
        "roofline": roofline,
        "hbm_copy_peak": copy_peak,
        "hbm_read_peak": read_peak,
        "hbm_gather_peak": gather_peak,
        "configs": configs,
        "mfma_kernels": mfma,
        "projection_paths": proj_paths,
        "other_cold_layout": alt,
        "encoder": enc,
        "fabric": fab,
        "dense_ops": dense,
        "inference_attention": att,
        "cpu_baseline": cpu,
        "reference_bench_config": ref_cfg,
    }
    engine.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

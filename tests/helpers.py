"""Shared helpers of the parity tests: run a workload on the GPU through the C
ABI and compare with the CPU oracle at the attention tolerance
(max-abs 2e-3, rel-L2 1e-3 against the fp64 brute force)."""
from __future__ import annotations

import numpy as np

MAX_ABS = 2e-3
REL_L2 = 1e-3


def run_gpu(engine, wl, stream, copy: int = 0, q_latent_f32: bool = False):
    import torch
    from aether_nexus_amd import workloads as W
    dev = wl.to("cuda:0")
    out = torch.full(dev.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
    engine.decode_device(W.device_desc(dev, out, copy=copy, q_latent_f32=q_latent_f32), stream=stream)
    engine.check_device_errors(stream)
    return out.cpu().numpy()


def errors(got, ref) -> tuple[float, float]:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = got - ref
    return float(np.abs(d).max()), float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30))


def assert_close(got, ref, what: str = "", max_abs: float = MAX_ABS, rel_l2: float = REL_L2):
    assert np.all(np.isfinite(np.asarray(got, dtype=np.float64))), f"{what}: non-finite output"
    ma, rl = errors(got, ref)
    print(f"{what}: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max_abs {ma:.3e} (<= {max_abs}), rel_l2 {rl:.3e} (<= {rel_l2})"

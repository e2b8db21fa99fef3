"""One HIP runtime per process: the library opened before any torch import (a
fresh process) still shares PyTorch's runtime, so torch's own device work and a
decode on torch memory both run afterwards."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CODE = """
import sys
from aether_nexus_amd.weaver import WeaverEngine
e = WeaverEngine()  # before this script imports torch (the loader itself does)
import torch
from aether_nexus_amd import workloads as W
x = torch.randn(1024, device="cuda:0")
wl = W.generate(W.hot_cold(batch=1), seed=5, device="cuda:0")
out = torch.empty(wl.out_shape(), dtype=torch.float16, device="cuda:0")
e.decode_device(W.device_desc(wl, out), stream=torch.cuda.current_stream().cuda_stream)
e.check_device_errors(torch.cuda.current_stream().cuda_stream)
print("ok", bool(torch.isfinite(x).all()), bool(torch.isfinite(out.float()).all()), flush=True)
e.close()
"""


def test_engine_first_then_torch_in_a_fresh_process():
    print("runtime: engine before torch in a child process", flush=True)
    r = subprocess.run([sys.executable, "-c", CODE], cwd=ROOT, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.strip().splitlines()[-1] == "ok True True", r.stdout[-1000:]

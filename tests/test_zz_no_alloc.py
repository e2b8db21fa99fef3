"""aw_decode_device_noalloc on cuda:0 through the C ABI: the decode with its
scratch in the library's fixed per-GPU array gives the same output bits as
aw_decode_device (which takes its scratch from the engine workspace), on two
calls in a row, the second smaller; a request whose scratch exceeds the array
is rejected before anything runs."""
from __future__ import annotations

import pytest
import torch

from aether_nexus_amd import workloads as W
from aether_nexus_amd.types import AW_E_UNSUPPORTED, AW_NOALLOC_SCRATCH_BYTES
from aether_nexus_amd.weaver import WeaverError, plan

pytestmark = pytest.mark.gpu


def decode_both(engine, stream, geom, seed):
    wl = W.generate(geom, seed=seed, device="cuda:0")
    ref = torch.full(wl.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
    out = torch.full(wl.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
    info = plan(W.device_desc(wl, out))
    print(f"no-alloc: {geom.batch} seq, hot {geom.hot_count} + cold {geom.cold_count} blocks, "
          f"scratch {info.workspace_bytes} bytes", flush=True)
    engine.decode_device_noalloc(W.device_desc(wl, out), stream=stream)
    engine.check_device_errors(stream)
    engine.decode_device(W.device_desc(wl, ref), stream=stream)
    engine.check_device_errors(stream)
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    return info.cold_output


def test_noalloc_matches_decode_device(engine, stream):
    # 64 sequences at hot 2048 + cold 32768 tokens (55.1 MiB of scratch), then a
    # smaller ragged request: the second call reuses the array the first left behind.
    # The second one's 256-atom dictionary takes the cold kernel's value partials
    # (their cold splits in the hot partial arrays), the first the bins and a finish.
    from aether_nexus_amd.types import AW_COLD_OUT_BINS, AW_COLD_OUT_VALUES
    big = W.sweep(64)
    small = W.hot_cold(batch=3, hot_count=5, cold_count=40, dict_size=256, queries=2, causal=True)
    assert decode_both(engine, stream, big, seed=71) == AW_COLD_OUT_BINS
    assert decode_both(engine, stream, small, seed=72) == AW_COLD_OUT_VALUES


@pytest.mark.parametrize("layers", [2, 4])
def test_noalloc_rejects_requests_beyond_its_scratch(engine, stream, layers):
    geom = W.sweep(64, layers=layers)  # 106.2 and 212.4 MiB of scratch
    wl = W.generate(geom, seed=73, device="cuda:0")
    out = torch.full(wl.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
    desc = W.device_desc(wl, out)
    need = plan(desc).workspace_bytes
    print(f"no-alloc: {layers} layers need {need / 2**20:.1f} MiB", flush=True)
    assert need > AW_NOALLOC_SCRATCH_BYTES
    with pytest.raises(WeaverError) as e:
        engine.decode_device_noalloc(desc, stream=stream)
    assert e.value.status == AW_E_UNSUPPORTED and "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()  # nothing ran


def test_noalloc_graph_capture_on_a_fresh_engine():
    """The entry point's purpose: capture into a HIP graph with no eager call first
    (a fresh engine has no workspace, and aw_decode_device would refuse to grow
    one under capture), the hot branch forked onto the engine's side stream
    inside the capture.  Every replay, with eager decodes of another shape and
    torch work in between, gives aw_decode_device's output bits."""
    from aether_nexus_amd.weaver import WeaverEngine
    eng = WeaverEngine()  # fresh: no workspace
    try:
        geom = W.hot_cold(batch=8)
        wl = W.generate(geom, seed=74, device="cuda:0")
        other = W.generate(W.hot_cold(batch=2, queries=2, causal=True), seed=75, device="cuda:0")
        out = torch.full(wl.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
        out2 = torch.empty(other.out_shape(), dtype=torch.float16, device="cuda:0")
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        print("no-alloc: capture on a fresh engine", flush=True)
        with torch.cuda.stream(s):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                eng.decode_device_noalloc(W.device_desc(wl, out), stream=torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            assert torch.isnan(out.float()).all()  # captured, not run
            ref = torch.empty_like(out)
            eng.decode_device(W.device_desc(wl, ref), stream=s.cuda_stream)
            eng.check_device_errors(s.cuda_stream)
            for rep in range(4):
                out.fill_(float("nan"))
                g.replay()
                torch.cuda.synchronize()
                assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
                eng.decode_device_noalloc(W.device_desc(other, out2), stream=s.cuda_stream)
                _ = (out2.float() * 2).sum()
                torch.cuda.synchronize()
            eng.check_device_errors(s.cuda_stream)
        del g
    finally:
        torch.cuda.synchronize()
        eng.close()

"""Decode captured in a HIP graph (as the benchmark replays it): every replay
gives the eager call's output bits, with other eager decodes, torch work and
synchronisations between the replays.  The capture holds the engine's
stream fork / join (hot kernel on its side stream beside the cold kernel);
the last case is one sequence over 512-atom per-kv-head dictionaries, where
the cold kernel hands value partials to the merge."""
from __future__ import annotations

import pytest
import torch

from aether_nexus_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("geom,hb", [
    (W.hot_cold(batch=4), False),
    (W.hot_cold(batch=4), True),
    (W.spec_verify(layers=2, batch=2), False),
    (W.hot_cold(batch=1), False),
    (W.hot_cold(batch=1, dict_size=512, dict_heads=8, separate_v=True, causal=True), True),
], ids=["hot_cold_b4", "hot_cold_b4_head_blocked", "spec_verify_l2_b2", "hot_cold_b1", "value_partials_b1"])
def test_graph_replays_match_eager(engine, geom, hb):
    wl = W.generate(geom, seed=21, device="cuda:0")
    other = W.generate(W.hot_cold(batch=2), seed=22, device="cuda:0")
    cold_hb = W.head_blocked(wl.cold) if hb else None
    out = torch.empty(wl.out_shape(), dtype=torch.float16, device="cuda:0")
    out2 = torch.empty(other.out_shape(), dtype=torch.float16, device="cuda:0")
    desc = W.device_desc(wl, out, cold_head_blocked=cold_hb)
    desc2 = W.device_desc(other, out2)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        engine.decode_device(desc, stream=s.cuda_stream)  # sizes the workspace before capture
        engine.check_device_errors(s.cuda_stream)
        eager = out.clone()
        print(f"graph: capture {geom}", flush=True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            engine.decode_device(desc, stream=torch.cuda.current_stream().cuda_stream)
        for rep in range(4):
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
            # Eager work between the replays: another decode and unrelated torch kernels.
            engine.decode_device(desc2, stream=s.cuda_stream)
            _ = (out2.float() * 2).sum()
            torch.cuda.synchronize()
    engine.check_device_errors(s.cuda_stream)


def test_capture_refuses_workspace_growth():
    """A call being captured cannot grow the engine's workspace (hipMalloc is not
    capturable): it returns AW_E_UNSUPPORTED before enqueueing anything; after
    one eager call of that size the same capture works and replays the eager
    output bits."""
    from aether_nexus_amd.types import AW_E_UNSUPPORTED
    from aether_nexus_amd.weaver import WeaverEngine, WeaverError
    eng = WeaverEngine()  # a fresh engine: no workspace yet
    try:
        wl = W.generate(W.hot_cold(batch=2), seed=23, device="cuda:0")
        out = torch.full(wl.out_shape(), float("nan"), dtype=torch.float16, device="cuda:0")
        desc = W.device_desc(wl, out)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        print("graph: capture before any eager call", flush=True)
        with torch.cuda.stream(s):
            g0 = torch.cuda.CUDAGraph()
            with pytest.raises(WeaverError) as e:
                with torch.cuda.graph(g0, stream=s):
                    eng.decode_device(desc, stream=torch.cuda.current_stream().cuda_stream)
            assert e.value.status == AW_E_UNSUPPORTED and "eager" in str(e.value)
            del g0
            torch.cuda.synchronize()
            assert torch.isnan(out.float()).all()  # nothing ran
            eng.decode_device(desc, stream=s.cuda_stream)
            eng.check_device_errors(s.cuda_stream)
            eager = out.clone()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                eng.decode_device(desc, stream=torch.cuda.current_stream().cuda_stream)
            for _ in range(2):
                out.fill_(float("nan"))
                g.replay()
                torch.cuda.synchronize()
                assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        del g
    finally:
        torch.cuda.synchronize()
        eng.close()

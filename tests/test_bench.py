"""CPU checks of bench.py's host logic: the one-GPU refusal, the per-launch
algorithmic bytes of the roofline, and the traffic-profile reader's layout and
source checks."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from aether_nexus_amd import workloads as W  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and not r.stdout.strip()


@pytest.mark.parametrize("batch", [1, 64])
def test_kernel_bytes_match_the_step_bytes(batch):
    """The hot and cold kernels' bytes are the step's hot rows, cold codes, block
    refs and the hot kernel's q reads (everything but the dictionary and out)."""
    g = W.sweep(batch)
    kb = bench.kernel_bytes(g)
    ab = g.algorithmic_bytes()
    assert kb["cold"] == ab["cold"] + g.batch * g.cold_count * 4
    assert kb["hot"] == ab["hot"] + g.batch * g.hot_count * 4 + ab["q_out"] // 2
    assert kb["hot"] + kb["cold"] == ab["total"] - ab["dict"] - ab["q_out"] // 2
    if batch == 64:
        assert kb["cold"] == 268_959_744  # 64 x 32768 tokens x 8 kv heads x 16 B + refs


def test_traffic_reader_checks_layout_and_sources(tmp_path, monkeypatch):
    lines = ["# HBM traffic per launch", "# command: x", "# cold_layout: head_blocked",
             f"# sources: {bench.sources_digest()}", "copy_bytes 1 kernel 'k' fetch_kib 1 write_kib 1",
             "factor_fetch 2.0 factor_write 1.0",
             "kernel cold_kernel grid 131072 fetch_kib 140000 write_kib 32792 traffic_bytes 319700000"]
    files = {}

    def fake(layout):
        return files.setdefault(layout, tmp_path / f"traffic_b64_{layout}.txt")

    monkeypatch.setattr(bench, "traffic_file", fake)
    fake("head_blocked").write_text("\n".join(lines) + "\n")
    assert bench.read_traffic("cold_kernel", "head_blocked") == (319700000, None)
    assert bench.read_traffic("hot_kernel", "head_blocked")[0] is None
    # Measured with the other layout: not used.
    fake("reference").write_text("\n".join(lines) + "\n")
    v, why = bench.read_traffic("cold_kernel", "reference")
    assert v is None and "head_blocked" in why
    # Measured on other sources: not used.
    fake("head_blocked").write_text("\n".join(lines).replace(bench.sources_digest(), "0123456789abcdef") + "\n")
    v, why = bench.read_traffic("cold_kernel", "head_blocked")
    assert v is None and "other kernel sources" in why


def test_sources_digest_ignores_comments_but_not_code(tmp_path, monkeypatch):
    """A comment or blank-line edit of the kernel sources keeps the digest (a
    traffic profile stays valid for the same code); a code edit changes it."""
    csrc = tmp_path / "aether_nexus_amd" / "csrc"
    csrc.mkdir(parents=True)
    names = ("weaver_engine.hip", "weaver_kernels.hpp")
    for n in names:
        (csrc / n).write_text((ROOT / "aether_nexus_amd" / "csrc" / n).read_text())
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    base = bench.sources_digest()
    assert base == bench.sources_digest()
    k = csrc / "weaver_kernels.hpp"
    src = k.read_text()
    k.write_text("// a new comment line\n\n" + src.replace("\n", "  // trailing note\n", 1) + "/* block\ncomment */\n")
    assert bench.sources_digest() == base
    k.write_text(src + "constexpr int kDigestProbe = 1;\n")
    assert bench.sources_digest() != base
    k.write_text(src)
    (csrc / "weaver_engine.hip").write_text((csrc / "weaver_engine.hip").read_text().replace("AW_OK", "AW_OK ", 1) + "int x;\n")
    assert bench.sources_digest() != base

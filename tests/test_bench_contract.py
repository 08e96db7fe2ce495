"""bench.py's bookkeeping against the committed counter summaries (CPU only).

The bench reports a launch group's HBM traffic as the sum of its kernels'
bytes in profiles/traffic*.json.  A kernel renamed in the sources but not in
the bench would silently drop its bytes; these tests tie the names together.
"""

import json
import os

import pytest

import bench
from tests.conftest import ROOT

PROFILES = os.path.join(ROOT, "profiles")
CSRC = os.path.join(ROOT, "redpanda_amd", "csrc")


def _kernels(name):
    with open(os.path.join(PROFILES, name)) as fh:
        return json.load(fh)["kernels"]


def _sources():
    text = ""
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".h")):
            with open(os.path.join(CSRC, f)) as fh:
                text += fh.read()
    return text


@pytest.mark.parametrize("total", sorted(bench.TRAFFIC_SUMS))
def test_summed_kernels_exist_in_sources(total):
    src = _sources()
    for name in bench.TRAFFIC_SUMS[total]:
        assert f" {name}(" in src or f" {name}<" in src, f"{total}: no kernel {name} in csrc"


@pytest.mark.parametrize("summary", ["traffic.json", "traffic_long.json"])
def test_summed_kernels_exist_in_counter_summaries(summary):
    k = _kernels(summary)
    for total, parts in bench.TRAFFIC_SUMS.items():
        if parts[0] in k:
            assert all(p in k for p in parts), (summary, total, [p for p in parts if p not in k])


@pytest.mark.parametrize("summary", ["traffic.json", "traffic_long.json"])
def test_group_totals_equal_the_sum_of_their_kernels(summary):
    k = _kernels(summary)
    out = bench.measured_traffic(summary)
    assert "scan_bwd_kernel+reductions" in out
    for total, parts in bench.TRAFFIC_SUMS.items():
        if parts[0] in k:
            assert out[total] == pytest.approx(sum(k[p]["bytes"] for p in parts), rel=1e-12)
    # the backward's total includes both reductions
    bwd = out["scan_bwd_kernel+reductions"]
    assert bwd > k["scan_bwd_kernel"]["bytes"] + k["bwd_reduce_bc4"]["bytes"]


def test_renamed_kernel_is_an_error(tmp_path, monkeypatch):
    """A summary that has the group's first kernel but not the others is
    refused rather than summed short."""
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "t.json").write_text(json.dumps(
        {"kernels": {"scan_bwd_kernel": {"bytes": 1.0}, "bwd_reduce_par": {"bytes": 2.0},
                     "bwd_reduce_bc": {"bytes": 3.0}}}))
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    with pytest.raises(KeyError, match="bwd_reduce_bc4"):
        bench.measured_traffic("t.json")


def test_gpus_above_one_exit_with_a_message():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr)

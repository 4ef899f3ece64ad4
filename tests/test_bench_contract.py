"""bench.py's contract pieces that need no GPU: the refusal of more than one
GPU and the provenance of the measured-traffic figure."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_traffic_figure_names_the_build_it_was_recorded_on():
    traffic, prov = bench.measured_traffic("attn_dense_kernel<12, 1, 2, 32, 3>")
    assert isinstance(traffic, int) and traffic > 0
    # the summary records the commit and the kernel source hash of its counter runs
    assert prov["commit"] and re.fullmatch(r"[0-9a-f]{7,40}", prov["commit"])
    assert prov["kernel_source_sha256"] and re.fullmatch(r"[0-9a-f]{16}", prov["kernel_source_sha256"])
    assert re.fullmatch(r"[0-9a-f]{16}", prov["current_kernel_source_sha256"])
    assert prov["source_matches"] == (prov["kernel_source_sha256"] == prov["current_kernel_source_sha256"])
    # within a few percent of the algorithmic bytes of the 8 x 384 x 32-head launch
    algorithmic = 2 * (2 * 8 * 384 * 32 * 128 + 2 * 8 * 384 * 32 * 128)
    assert 0.95 < traffic / algorithmic < 1.10


def test_traffic_of_another_kernel_is_not_reported():
    traffic, prov = bench.measured_traffic("attn_dense_kernel<4, 1, 2, 32, 3>")
    assert traffic is None
    assert prov["commit"] is None


@pytest.mark.parametrize("kernel", ["attn_dense_kernel<12, 1, 2, 32, 3>"])
def test_summary_first_line_names_the_kernel(kernel):
    with open(bench.TRAFFIC_SUMMARY) as f:
        assert kernel in f.readline()

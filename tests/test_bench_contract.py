"""The bench line's fixed parts that need no GPU: the HBM traffic it reads from the committed
rocprofv3 summaries, and the refusal of more than one GPU."""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_module", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("workload,kernel", [("bf16-2m", "pool_kernel"), ("bf16-2m-int8", "pool_kernel"),
                                             ("lazy-32k", "pool_kernel"), ("hetero-bf16", "bin_mixed_long_kernels")])
def test_profiles_give_the_traffic(bench, workload, kernel):
    # every profile the bench line cites exists and carries its measured HBM bytes per launch,
    # which sit between the output bytes written and 4 GB
    t = bench.traffic_from_profiles(workload, kernel)
    assert t is not None and 2.9e7 < t < 4e9


def test_missing_profile_gives_null_traffic(bench):
    assert bench.traffic_from_profiles("no-such-workload") is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)

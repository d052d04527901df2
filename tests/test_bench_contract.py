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


# (workload, kernel, output bytes of one launch)
PROFILES = [("bf16-2m", "pool_kernel", 29_360_128), ("bf16-2m-int8", "pool_kernel", 29_360_128),
            ("fp32-1m", "pool_kernel", 58_720_256), ("small-fp32", "pool_kernel", 1_835_008),
            ("lazy-32k", "pool_kernel", 234_881_024), ("hetero-bf16", "bin_mixed_long_kernels", 33_554_432),
            ("reference-5m", "pool_kernel", 117_440_512), ("reference-5m", "pool_norm_kernel", 117_440_512),
            ("reference-5m-int8", "pool_kernel", 117_440_512)]


@pytest.mark.parametrize("workload,kernel,out_bytes", PROFILES)
def test_profiles_give_the_traffic(bench, workload, kernel, out_bytes):
    # every profile the bench line cites exists and carries its measured HBM bytes per launch,
    # which sit between the output bytes written and 4 GB
    t, source = bench.traffic_from_profiles(workload, kernel)
    assert t is not None and out_bytes <= t < 4e9
    assert source == f"profiles/{kernel}_{workload}.md" and os.path.exists(os.path.join(ROOT, source))


def test_missing_profile_gives_null_traffic(bench):
    assert bench.traffic_from_profiles("no-such-workload") == (None, None)


def test_roofline_frac_is_the_measured_hbm_fraction(bench):
    # achieved / frac: the profile's HBM bytes per launch over the launch time, against 8 TB/s;
    # the algorithmic bytes (every lookup's row) go to effective_*
    r = bench.roofline(240e6, 40e-6, "pool_kernel", ("bf16-2m", "pool_kernel"), compulsory_bytes=100e6)
    assert r["traffic_source"] == "profiles/pool_kernel_bf16-2m.md"
    assert r["achieved"] == pytest.approx(r["traffic"] / 40e-6 / 1e9)
    assert r["frac"] == pytest.approx(r["achieved"] / 8000.0)
    assert r["effective_gbs"] == pytest.approx(6000.0) and r["effective_frac"] == pytest.approx(0.75)
    assert r["compulsory_frac"] == pytest.approx(100e6 / 40e-6 / 1e9 / 8000.0)
    # no counter profile: no HBM figure, unless the kernel streams each byte once
    none = bench.roofline(1.0, 1.0, "k", None)
    assert none["achieved"] is None and none["frac"] is None and none["traffic"] is None
    streamed = bench.roofline(8e6, 1e-6, "k", None, streaming=True)
    assert streamed["frac"] == pytest.approx(1.0) and streamed["traffic"] == 8e6


def test_host_cpu_counts(bench):
    info = bench.host_cpus()
    assert info["logical"] == os.cpu_count()
    assert 1 <= info["affinity"] <= info["logical"]
    assert info["physical"] is None or 1 <= info["physical"] <= info["logical"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)

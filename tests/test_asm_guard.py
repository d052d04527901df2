"""Guard on the generated gfx950 code (CPU only, needs only hipcc): every HIP source compiles to
device assembly without scalar-cache stores, scalar atomics or scalar-cache write-back/discard,
and every atomic is a vector (global) atomic."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cti-inference-optimization_amd", "csrc")
FORBIDDEN = re.compile(r"^\s+s_(store|atomic|buffer_store|buffer_atomic|dcache_wb|dcache_discard|scratch_store)",
                       re.M)


SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def test_every_hip_source_is_guarded():
    assert {"ebag_pool.hip", "ebag_layout.hip", "ebag_status.hip", "ebag_norm.hip", "ebag_quant.hip",
            "ebag_static.hip", "ebag_linear.hip"} <= set(SOURCES)


@pytest.mark.parametrize("src", SOURCES)
def test_no_scalar_cache_writes(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-ffp-contract=off", f"-I{ROOT}/include", "--cuda-device-only", "-S",
           os.path.join(CSRC, src), "-o", str(out)]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    text = out.read_text()
    assert ".amdgcn_target" in text or "amdgcn" in text
    bad = FORBIDDEN.findall(text)
    assert not bad, f"{src}: scalar-cache writes in device code: {sorted(set(bad))}"
    assert not re.search(r"^\s+v_pk_(add|mul|fma)_f32", text, re.M), f"{src}: packed fp32 ops emitted"

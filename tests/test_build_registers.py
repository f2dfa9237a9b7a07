"""Register budget of the gfx950 kernels (CPU: hipcc cross-compiles).

The attention kernels run four waves per SIMD at <= 128 VGPRs (the
sliding-window kernels with a key mask three, at <= 168); a change that
pushes one past its budget makes the compiler spill to scratch memory, which
costs far more than the change saves and shows up in no parity test. This
test compiles each kernel source to AMD assembly and compares every kernel's
.vgpr_spill_count with the committed maximum: 0 for every kernel."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "vllm-factory_amd", "csrc")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")

# mangled kernel name -> largest accepted spill count
KNOWN_SPILLS: dict = {}


def _spills(src: str, tmp_path) -> dict:
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-mcode-object-version=5",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only",
           "-S", src, "-o", str(out)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
    res, name = {}, None
    for line in out.read_text().splitlines():
        m = re.match(r"\s+\.name:\s+(_Z\S+)", line)
        if m:
            name = m.group(1)
        m = re.match(r"\s+\.vgpr_spill_count:\s+(\d+)", line)
        if m and name:
            res[name] = int(m.group(1))
    return res


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", ["attn_varlen.hip", "attn_rpb.hip", "attn_deberta.hip",
                                 "gemm_glu.hip", "gemm_ln.hip", "colbert_head.hip"])
def test_no_new_register_spills(src, tmp_path):
    spills = _spills(os.path.join(CSRC, src), tmp_path)
    assert spills, "no kernels found"
    over = {k: v for k, v in spills.items() if v > KNOWN_SPILLS.get(k, 0)}
    assert not over, f"kernels spilling beyond their budget: {over}"

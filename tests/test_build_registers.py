"""Register budget of the gfx950 kernels (CPU: hipcc cross-compiles).

The attention kernels run four waves per SIMD at <= 128 VGPRs; a change that
pushes one past its budget makes the compiler spill to scratch memory, which
costs far more than the change saves and shows up in no parity test. This
test compiles each kernel source to AMD assembly and compares every kernel's
.vgpr_spill_count with the committed maximum: 0 for every kernel but the two
bf16 RPB kernels with a key mask, which hold their second, running-max pass
next to the first, and the sliding-window varlen kernels with a key mask:
1 or 2 registers stored before a tile loop and reloaded after it, never
inside one.

It also checks .private_segment_fixed_size, the per-lane scratch a kernel
reserves: a private array that the compiler cannot keep in registers (one
indexed by a loop that did not unroll) lands there without counting as a
spill, and its scratch loads and stores can halve a memory-bound kernel's
rate. Only the LayerNorm / RMSNorm kernels for 16-bit rows wider than 4096
values (12 and 16 chunks per lane, no configured model's width) use any,
besides those kernels' spill slots."""
import concurrent.futures as cf
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "vllm-factory_amd", "csrc")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")

# mangled kernel name -> largest accepted spill count
KNOWN_SPILLS: dict = {
    "_ZN3vfk14rpb_fwd_kernelINS_4BF16ELi1ELb0EEEvNS_7RpbArgsE": 2,
    "_ZN3vfk14rpb_fwd_kernelINS_4BF16ELi1ELb1EEEvNS_7RpbArgsE": 2,
    "_ZN3vfk17varlen_fwd_kernelINS_4BF16ELb1ELb1ELb1EEEvNS_10VarlenArgsE": 1,
    "_ZN3vfk17varlen_fwd_kernelINS_4BF16ELb0ELb1ELb1EEEvNS_10VarlenArgsE": 2,
    "_ZN3vfk17varlen_fwd_kernelINS_3F16ELb1ELb1ELb1EEEvNS_10VarlenArgsE": 1,
    "_ZN3vfk17varlen_fwd_kernelINS_3F16ELb0ELb1ELb1EEEvNS_10VarlenArgsE": 2,
}
# kernels allowed a private segment: norm_vec_kernel<16-bit dtype, lanes, 12 or 16 chunks, rms>
KNOWN_PRIVATE = re.compile(r"_ZN3vfk15norm_vec_kernelILi[12]ELi(32|64)ELi(12|16)ELb[01]EEEvNS_8NormArgsE")


SOURCES = ["attn_varlen.hip", "attn_rpb.hip", "attn_deberta.hip", "gemm_glu.hip", "gemm_ln.hip",
           "colbert_head.hip", "elementwise.hip", "packing.hip"]
_CACHE: dict = {}


def _compile(src: str, outdir: str) -> dict:
    """{kernel: (vgpr spill count, private segment bytes)} from the AMD assembly."""
    out = os.path.join(outdir, os.path.basename(src) + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-mcode-object-version=5",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only",
           "-S", src, "-o", out]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
    spill, priv, name = {}, {}, None
    with open(out) as f:
        for line in f:
            m = re.match(r"\s+\.name:\s+(_Z\S+)", line)
            if m:
                name = m.group(1)
            m = re.match(r"\s+\.vgpr_spill_count:\s+(\d+)", line)
            if m and name:
                spill[name] = int(m.group(1))
            m = re.match(r"\s+\.private_segment_fixed_size:\s+(\d+)", line)
            if m and name:
                priv[name] = int(m.group(1))
    return {k: (spill.get(k, 0), priv.get(k, 0)) for k in set(spill) | set(priv)}


def _resources(src: str, tmp_path_factory) -> dict:
    """Resources of one source; the first call compiles every source at once."""
    if not _CACHE:
        outdir = str(tmp_path_factory.mktemp("asm"))
        with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
            futs = {f: ex.submit(_compile, os.path.join(CSRC, f), outdir) for f in SOURCES}
            for f, fut in futs.items():
                _CACHE[f] = fut.result()
    return _CACHE[src]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", ["attn_varlen.hip", "attn_rpb.hip", "attn_deberta.hip",
                                 "gemm_glu.hip", "gemm_ln.hip", "colbert_head.hip"])
def test_no_new_register_spills(src, tmp_path_factory):
    res = _resources(src, tmp_path_factory)
    assert res, "no kernels found"
    over = {k: v[0] for k, v in res.items() if v[0] > KNOWN_SPILLS.get(k, 0)}
    assert not over, f"kernels spilling beyond their budget: {over}"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", SOURCES)
def test_no_scratch_memory(src, tmp_path_factory):
    res = _resources(src, tmp_path_factory)
    assert res, "no kernels found"
    scratch = {k: v[1] for k, v in res.items()
               if v[1] > 8 * KNOWN_SPILLS.get(k, 0) and not KNOWN_PRIVATE.fullmatch(k)}
    assert not scratch, f"kernels with a private segment (scratch memory): {scratch}"

"""Register and scratch budgets of the streaming kernels, read from the code
object metadata of the built library (the AMDGPU notes of its gfx950 code
objects).  The launch plans assume workgroups per CU: two 512-thread
workgroups (16 wavefronts, four per SIMD: at most 128 VGPRs each) for the
8-wavefront kernels, three 256-thread ones (three per SIMD: at most 168) for
the 4-wavefront kernels with one activation block, two (two per SIMD: 256)
with two activation blocks (M = 17..32).  Past its budget a kernel loses a
workgroup per CU (a MoE gather once went from 121 to 129 VGPRs and from 28.8
to 41.0 us per launch), so the budgets are checked here, along with no
spills.  CPU only: nothing runs on a GPU."""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "dflash-mlx_amd", "libdfmi.so")
LLVM = "/opt/rocm/llvm/bin"

# kernel families launched with the workgroups-per-CU budget above
STREAMING = ("qmm_stream_kernel", "qmm_stream_multi_kernel", "qmm_stream_fused_kernel",
             "lmhead_stream_kernel", "moe_stream_kernel")
# (threads per workgroup, activation blocks) -> VGPRs per lane
VGPR_BUDGET = {(512, 1): 128, (512, 2): 128, (256, 1): 168, (256, 2): 256}


def _kernels():
    objdump, readelf = os.path.join(LLVM, "llvm-objdump"), os.path.join(LLVM, "llvm-readelf")
    if not (os.path.exists(LIB) and os.path.exists(objdump) and os.path.exists(readelf)):
        pytest.skip("libdfmi.so or the ROCm LLVM tools not present")
    out = {}
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "l.so")
        shutil.copy(LIB, lib)
        subprocess.run([objdump, "--offloading", lib], cwd=d, capture_output=True, check=True)
        objs = [f for f in os.listdir(d) if f.endswith("gfx950")]
        assert objs, "no gfx950 code object in libdfmi.so"
        for f in objs:
            notes = subprocess.run([readelf, "--notes", os.path.join(d, f)], capture_output=True,
                                   text=True, check=True).stdout
            for blk in notes.split("  - .agpr_count")[1:]:
                name = re.search(r"\.name:\s+(\S+)", blk).group(1)
                out[name] = {
                    "vgpr": int(re.search(r"\.vgpr_count:\s+(\d+)", blk).group(1)),
                    "scratch": int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", blk).group(1)),
                    "threads": int(re.search(r"\.max_flat_workgroup_size:\s+(\d+)", blk).group(1)),
                }
    return out


def _activation_blocks(name: str, fam: str) -> int:
    """MT, the third integer template argument (Tag, GS, MT, WV, ...), of the
    kernels that have one; the MoE gathers run one activation block."""
    if fam == "moe_stream_kernel":
        return 1
    ints = [int(v) for v in re.findall(r"Li(\d+)E", name)]
    return ints[1]


def _family(name: str):
    for fam in STREAMING:
        if f"{len(fam)}{fam}" in name:  # Itanium-mangled identifier: <length><name>
            return fam
    return None


def test_streaming_kernels_fit_their_occupancy():
    ks = _kernels()
    seen = set()
    for name, r in sorted(ks.items()):
        fam = _family(name)
        if fam is None:
            continue
        seen.add(fam)
        key = (r["threads"], _activation_blocks(name, fam))
        assert key in VGPR_BUDGET, (name, r)
        assert r["vgpr"] <= VGPR_BUDGET[key], (name, r)
        assert r["scratch"] == 0, (name, r)
    assert seen == set(STREAMING), sorted(set(STREAMING) - seen)

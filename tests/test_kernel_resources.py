"""Every kernel of the built library keeps its data in registers: no scratch memory and no
register spills, read from the gfx950 code objects' kernel metadata (no GPU needed).

The 256x256 ring GEMMs hold 128 accumulator registers per lane and sit close to the
register limit; an epilogue or main-loop change that pushes them over spills the
accumulators to scratch and makes C3 an order of magnitude slower (a copy of the epilogue's
row sweep specialised for beta == 0 did exactly that: 0.80 -> 9.7 ms). This test catches such
a change on the CPU, before any GPU run."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "go-nngpu_amd", "lib", "libgonngpu.so")
LLVM = "/opt/rocm/llvm/bin"


def kernel_resources(lib):
    """{kernel name: (scratch bytes per lane, VGPR spills, SGPR spills)} for every gfx950 code
    object in the library's HIP fat binary."""
    objdump, readelf = os.path.join(LLVM, "llvm-objdump"), os.path.join(LLVM, "llvm-readelf")
    d = tempfile.mkdtemp()
    try:
        shutil.copy(lib, d)  # the bundles are written next to the input file
        name = os.path.basename(lib)
        subprocess.run([objdump, "--offloading", name], cwd=d, check=True, capture_output=True)
        out = {}
        for f in sorted(os.listdir(d)):
            if not f.endswith("gfx950"):
                continue
            notes = subprocess.run([readelf, "--notes", os.path.join(d, f)], check=True, capture_output=True,
                                   text=True).stdout
            for k in re.split(r"\n\s+- \.", notes):
                m = re.search(r"\.name:\s+(\S+)", k)
                if not m or ".symbol:" not in k:  # kernel entries carry their descriptor symbol
                    continue
                vals = []
                for key in ("private_segment_fixed_size", "vgpr_spill_count", "sgpr_spill_count"):
                    v = re.search(r"\.%s:\s+(\d+)" % key, k)
                    vals.append(int(v.group(1)) if v else 0)
                out[m.group(1)] = tuple(vals)
        return out
    finally:
        shutil.rmtree(d)


@pytest.mark.skipif(not os.path.exists(os.path.join(LLVM, "llvm-objdump")), reason="ROCm LLVM tools not installed")
def test_no_kernel_uses_scratch_or_spills():
    if not os.path.exists(LIB):
        pytest.skip("libgonngpu.so is not built (run __graft_entry__.build())")
    res = kernel_resources(LIB)
    assert len(res) > 100, len(res)
    # the kernels whose performance depends on it most must be among those checked
    for key in ("gemm_f16_ring_kernelILi256ELi256ELi2ELi4ELb0ELb0", "gemm_f32_ring_kernelILi256ELi256",
                "spmv_grouped_kernel", "spmm_band", "gemm_small_kernelIfLi4ELi1ELi1E",
                "gemm_small_kernelIDF16_Li16ELi1ELi1E"):
        assert any(key in k for k in res), key
    bad = {k: v for k, v in res.items() if any(v)}
    assert not bad, bad

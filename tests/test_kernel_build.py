"""Register and LDS budgets of the bf16 attention kernels, read from the compiler's kernel metadata
(device-only assembly of kernels_attn.hip with the library's flags; no GPU needed).

The two-wave kernel (64-query tiles) must fit three waves per SIMD (<= 168 VGPRs) without spills,
and the four-wave kernel (128-query tiles, global layers) four waves per SIMD (<= 128 VGPRs), where
it keeps one spilled register outside its key loops.  Both use 24 KB of LDS, so that six two-wave
or four four-wave workgroups share a CU.  A change to the kernel that pushes either over its budget
halves its occupancy or puts spills in the key loop, which the kernel tests would not notice (the
results stay right) but a launch runs up to a third slower."""
import os
import re
import shutil
import subprocess

import pytest

from layamd_amd import build

HIPCC = build.HIPCC


@pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which(HIPCC)), reason="hipcc not available")
def test_attention_kernels_fit_their_occupancy(tmp_path):
    out = tmp_path / "attn.s"
    src = os.path.join(build.CSRC, "kernels_attn.hip")
    flags = [f for f in build.HIP_FLAGS if f != "-fPIC"] + build.TU_FLAGS.get("kernels_attn.hip", [])
    r = subprocess.run([HIPCC] + flags + ["--cuda-device-only", "-S", "-o", str(out), src],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    meta = out.read_text()
    # the amdhsa.kernels metadata: one block per kernel, .name after the segment sizes
    blocks = re.split(r"\n  - \.", meta[meta.index("amdhsa.kernels:"):])
    seen = {}
    for b in blocks:
        name = re.search(r"\.name:\s+(\S+)", b)
        if not name or "k_attention_bf16" not in name.group(1):
            continue
        nw = 2 if "ILi2E" in name.group(1) else 4
        val = lambda key: int(re.search(r"\." + key + r":\s+(\d+)", b).group(1))
        seen[nw] = (val("vgpr_count"), val("vgpr_spill_count"), val("group_segment_fixed_size"))
    assert set(seen) == {2, 4}, seen
    vgpr, spill, lds = seen[2]
    assert vgpr <= 168 and spill == 0 and lds == 24576, seen[2]
    vgpr, spill, lds = seen[4]
    assert vgpr <= 128 and spill <= 1 and lds == 24576, seen[4]

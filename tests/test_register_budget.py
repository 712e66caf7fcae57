"""Every HIP kernel compiles for gfx950 without register spills.

The two prefill kernels sit at exactly 256 VGPRs, and small source changes
can tip them into spilling VGPRs to scratch or SGPRs through VGPR lanes,
each of which cost several percent of kernel time when it happened.  This
compiles each source to device assembly with the library's own flags and
reads the spill counts from the kernel metadata.  CPU only: hipcc
cross-compiles without a GPU.
"""

import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from microserve_amd import build as B

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


def _kernel_metadata(src, out_dir):
    name = os.path.basename(src)
    asm = os.path.join(out_dir, name + ".s")
    cmd = [HIPCC, *B.HIP_FLAGS, *B.FILE_FLAGS.get(name, []), "--cuda-device-only", "-S",
           src, "-o", asm]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    text = open(asm).read()
    # one metadata record per kernel: .name, then its counts
    kernels = {}
    for block in re.split(r"\n\s+- \.", text.split("amdhsa.kernels:", 1)[1]):
        m = re.search(r"\.name:\s+(\S+)", block)
        if not m or m.group(1).endswith(".kd"):
            continue
        counts = {k: int(v) for k, v in
                  re.findall(r"\.(vgpr_spill_count|sgpr_spill_count|vgpr_count):\s+(\d+)", block)}
        if counts:
            kernels[m.group(1)] = counts
    return name, kernels


@pytest.fixture(scope="module")
def metadata(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("asm"))
    srcs = [s for s in B.sources() if s.endswith(".hip")]
    with ThreadPoolExecutor(max_workers=min(6, len(srcs))) as pool:
        return dict(pool.map(lambda s: _kernel_metadata(s, out), srcs))


def test_every_source_has_kernels(metadata):
    assert set(metadata) == {"store.hip", "decode.hip", "prefill.hip", "dense_prefill.hip",
                             "qk_norm_rope.hip", "step_inputs.hip"}
    for name, kernels in metadata.items():
        assert kernels, name


def test_no_kernel_spills_registers(metadata):
    for name, kernels in metadata.items():
        for kernel, c in kernels.items():
            assert c.get("vgpr_spill_count", 0) == 0, (name, kernel, c)
            assert c.get("sgpr_spill_count", 0) == 0, (name, kernel, c)


def test_prefill_kernels_fit_two_waves_per_simd(metadata):
    for name in ("prefill.hip", "dense_prefill.hip"):
        for kernel, c in metadata[name].items():
            if "prefill" in kernel:
                assert c["vgpr_count"] <= 256, (kernel, c)

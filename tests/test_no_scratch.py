"""The built kernels use no scratch (private) memory: a kernel that does pays for the wave's scratch set-up at
every dispatch and for memory round trips where registers were meant (a staging array the compiler could not keep
in registers took 144 bytes a lane of the attention kernel and 3 us a layer). Reads each built object's gfx950 code
object (the .hip_fatbin section, unbundled) and its kernels' .private_segment_fixed_size. CPU only; skipped when
the objects or the ROCm tools are absent."""
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LLVM = "/opt/rocm/llvm/bin"
OBJS = sorted(glob.glob(os.path.join(ROOT, "geode_amd", "_build", "*.hip.o")))


def _tool(name):
    p = os.path.join(LLVM, name)
    if not os.path.exists(p):
        pytest.skip(f"{p} not found")
    return p


@pytest.mark.skipif(not OBJS, reason="the library is not built (python -m geode_amd.build)")
@pytest.mark.parametrize("obj", OBJS, ids=[os.path.basename(o) for o in OBJS])
def test_kernels_use_no_scratch(obj, tmp_path):
    objcopy, bundler, readelf = _tool("llvm-objcopy"), _tool("clang-offload-bundler"), _tool("llvm-readelf")
    fat, dev = tmp_path / "fat.bin", tmp_path / "dev.co"
    r = subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", obj, str(tmp_path / "host.o")],
                       capture_output=True)
    if r.returncode != 0 or not fat.exists():
        pytest.skip("no device code in this object (host code only)")
    subprocess.run([bundler, "--unbundle", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={dev}"], check=True, capture_output=True)
    notes = subprocess.run([readelf, "--notes", str(dev)], check=True, capture_output=True, text=True).stdout
    names = re.findall(r"^\s+\.name:\s+(\S+)", notes, re.M)
    sizes = [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)]
    assert len(names) == len(sizes), "kernel metadata not read"
    using = [(n, s) for n, s in zip(names, sizes) if s]
    assert not using, f"kernels with scratch: {using}"

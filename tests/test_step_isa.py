"""Properties of the compiled persistent step kernel that no GPU run can show reliably.

The step kernel reads its arguments through the kernel-argument segment pointer, which exists
only in the kernel function itself: a called function gets 0 and its argument loads fault. So
every step-kernel instance must be free of calls. Its buffers are all device memory accessed
through global instructions; a FLAT access would also count against lgkmcnt and make every
LDS wait wait for outstanding weight loads.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "llm-inference_amd", "csrc", "step_kernel.hip")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _makefile_flags():
    """The package Makefile's COMMON and DEVICE flags for HIP sources."""
    text = open(os.path.join(ROOT, "llm-inference_amd", "Makefile")).read()
    flags = []
    for var in ("COMMON", "DEVICE"):
        m = re.search(r"^%s\s*[:+]?=\s*(.*)$" % var, text, re.M)
        assert m, "%s not found in the package Makefile" % var
        flags += m.group(1).replace("$(ROOT)", ROOT).split()
    return flags


@pytest.fixture(scope="module")
def step_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "step.s"
    flags = [f for f in _makefile_flags() if f not in ("-fPIC",)]
    cmd = [HIPCC, *flags, "-I" + os.path.join(ROOT, "include"), "--cuda-device-only", "-S",
           "-o", str(out), SRC]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    return out.read_text()


def _functions(asm):
    """name -> body of every function in the device assembly."""
    bodies = {}
    for m in re.finditer(r"^(_Z\S+):.*?\n(.*?)^\.Lfunc_end", asm, re.M | re.S):
        bodies[m.group(1)] = m.group(2)
    return bodies


def test_step_kernels_have_no_calls_and_no_flat_access(step_asm):
    funcs = _functions(step_asm)
    kernels = {n: b for n, b in funcs.items() if "step_kernel" in n}
    assert len(kernels) >= 4, sorted(funcs)
    assert set(funcs) == set(kernels), "out-of-line device functions: %s" % sorted(
        set(funcs) - set(kernels))
    for name, body in kernels.items():
        assert "s_swappc_b64" not in body, name
        flat = re.findall(r"^\s*(flat_\w+)", body, re.M)
        assert not flat, (name, sorted(set(flat)))


def test_bench_shape_step_kernel_uses_no_scratch(step_asm):
    """The Qwen3-0.6B instance with one workgroup per query head (the bench's) and the small test
    shape's keep everything in registers and LDS: no spill and no private array (a local table
    indexed at run time is placed in scratch memory, whose loads cost a memory round trip). The
    0.6B split-attention instance is allowed a few bytes, reloaded once per token."""
    sizes = dict(re.findall(r"\.name:\s+(\S+)\n(?:.*\n)*?\s+\.private_segment_fixed_size:\s+(\d+)",
                            step_asm))
    checked = 0
    for name, size in sizes.items():
        if "ShapeILi1024ELi3072ELi16ELi8EELb0E" in name or "ShapeILi512ELi1024ELi8ELi4EELb0E" in name:
            assert int(size) == 0, (name, size)
            checked += 1
        elif "ShapeILi1024ELi3072ELi16ELi8EELb1E" in name:
            assert int(size) <= 32, (name, size)
    assert checked == 2, sizes

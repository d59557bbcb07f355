"""MI355X (gfx950) FP32 attention: a drop-in for ROCmKernels' attention entry points.

The product is the C-ABI shared library ``lib/libROCmKernels.Kernels.Shared.so`` (and its static twin
``lib/libROCmKernels.Kernels.a``) built from ``csrc/`` (hand-written HIP for gfx950) by the repository's CMake project.
``rocmkernels_amd.attention`` binds it with ctypes the way the reference's training loop does.
"""
import os
import shutil
import subprocess

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PACKAGE_DIR)
BUILD_DIR = os.path.join(ROOT, "build")


def build(jobs=8):
    """Configure and build the CMake project (gfx950 only) from scratch: both libraries and the wrapper test program
    land in lib/. Always rebuilds."""
    shutil.rmtree(BUILD_DIR, ignore_errors=True)
    subprocess.run(["cmake", "-S", ROOT, "-B", BUILD_DIR, "-G", "Ninja"], check=True, stdout=subprocess.DEVNULL)
    subprocess.run(["ninja", "-C", BUILD_DIR, f"-j{jobs}"], check=True, stdout=subprocess.DEVNULL)

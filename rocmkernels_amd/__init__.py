"""MI355X (gfx950) FP32 attention: a drop-in for ROCmKernels' attention entry points.

The product is the C-ABI shared library ``lib/libROCmKernels.Kernels.Shared.so`` built from ``csrc/`` (hand-written
HIP for gfx950). ``rocmkernels_amd.attention`` binds it with ctypes the way the reference's training loop does.
"""
import os
import subprocess

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))


def build(jobs=4):
    """Compile every HIP source for gfx950 and link the shared library (always rebuilds)."""
    subprocess.run(["make", "-B", f"-j{jobs}", "-C", os.path.join(PACKAGE_DIR, "csrc")], check=True,
                   stdout=subprocess.DEVNULL)

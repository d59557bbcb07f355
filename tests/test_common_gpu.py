"""GPU run of a C++ caller written in the reference's generic-test pattern (Generic/AttentionGenericTests.cpp:106-139):
ROCmKernels::DeviceBuffer<T> storage, AttentionGenericForward(..., DTypeOf<T>::value) and the device queries of
ROCmKernels.Common, compiled against the public headers (tests/cpp/common_consumer.cpp, built by the CMake project as
librocmkernels_common_consumer.so) and called in this process through ctypes. Its fp32 and fp16 cases are checked
against their closed form (constant Q and K: the output is the mean of the visible V rows, lse = {score, visible
keys}) to the reference's tolerances.
"""
import ctypes
import os

import pytest

from rocmkernels_amd import attention

pytestmark = pytest.mark.gpu

CHECK_LIBRARY = os.path.join(os.path.dirname(attention.library_path()), "librocmkernels_common_consumer.so")


def test_reference_style_cpp_caller_runs_on_device_buffers(device):
    if not os.path.exists(CHECK_LIBRARY):
        pytest.fail(f"{CHECK_LIBRARY} is missing: build it with __graft_entry__.build() (CMake)")
    attention.lib()
    check = ctypes.CDLL(CHECK_LIBRARY)
    check.common_consumer_gpu_check.argtypes = [ctypes.c_char_p, ctypes.c_int]
    check.common_consumer_gpu_check.restype = ctypes.c_int
    text = ctypes.create_string_buffer(8192)
    failures = check.common_consumer_gpu_check(text, len(text))
    report = text.value.decode()
    print(report)
    assert failures == 0, report
    assert report.count("fp16") == 3 and report.count("fp32") == 2

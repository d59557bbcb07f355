"""CPU-side checks of the drop-in boundary: the shared library loads, exports exactly what include/*.h declares,
rejects invalid arguments with the reference's return codes before touching a device, and the C and C++ headers
compile and behave like the reference's (throwing wrappers)."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

from rocmkernels_amd import attention

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_symbols():
    names = set()
    for header in glob.glob(os.path.join(INCLUDE, "*.h")):
        with open(header) as handle:
            names.update(re.findall(r"ROCMKERNELS_EXPORT\s+int\s+(\w+)\s*\(", handle.read()))
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", attention.library_path()], check=True, capture_output=True,
                         text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_header_declares_every_reference_entry_point():
    reference_names = {
        "attention_fp32_forward", "attention_fp32_forward_tiled", "attention_fp32_backward", "attention_fp32_backward_tiled",
        "attention_fp32_statistics", "attention_fp32_forward_tuned", "attention_fp32_forward_flash",
        "attention_fp32_forward_flash_tuned", "attention_fp32_backward_tuned", "attention_fp32_backward_profile",
        "attention_fp32_query_profile", "attention64_fp32_forward", "attention64_fp32_backward",
    }
    assert reference_names <= declared_symbols()


def test_library_exports_exactly_the_declared_symbols():
    declared = declared_symbols()
    exported = exported_symbols()
    assert declared == exported, (declared ^ exported)
    assert declared == set(attention.ENTRY_POINTS)


def test_library_loads_and_binds():
    lib = attention.lib()
    for name in attention.ENTRY_POINTS:
        assert getattr(lib, name).restype is ctypes.c_int


S0 = attention.Strides(0, 0, 0)


def _buf():
    return ctypes.c_void_p(1)  # never dereferenced: every call below fails validation first


FWD_OK = lambda: [_buf(), _buf(), _buf(), _buf(), _buf(), _buf()]  # noqa: E731
BWD_OK = lambda: [_buf()] * 11  # noqa: E731


@pytest.mark.parametrize("name,args", [
    ("attention_fp32_forward", [None] + FWD_OK()[1:] + [1, 1, 1, 1, -1, S0, S0, S0, S0, None]),
    ("attention_fp32_forward", FWD_OK() + [0, 1, 1, 1, -1, S0, S0, S0, S0, None]),
    ("attention_fp32_forward", FWD_OK() + [1, 1, 1, -5, -1, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_tiled", FWD_OK()[:5] + [None] + [1, 1, 64, 64, -1, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_flash", FWD_OK() + [1, 1, 1, 1, -2, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_flash_tuned", FWD_OK() + [1, 1, 1, 1, -1, 19, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_flash_tuned", FWD_OK() + [1, 1, 1, 1, -1, -1, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_tuned", FWD_OK() + [1, 1, 1, 1, -1, 16, S0, S0, S0, S0, None]),
    ("attention_fp32_statistics", [_buf(), _buf(), _buf(), None, 1, 1, 1, 1, -1, S0, S0, None]),
    ("attention_fp32_statistics", [_buf(), _buf(), _buf(), _buf(), 1, 1, 1, 1, -2, S0, S0, None]),
    ("attention_fp32_backward", BWD_OK()[:10] + [None] + [1, 1, 1, 1, -1, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_tiled", BWD_OK() + [1, 0, 1, 1, -1, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_tuned", BWD_OK() + [1, 1, 1, 1, -1, 7, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_profile", BWD_OK() + [1, 1, 64, 64, -1, 0, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_profile", BWD_OK() + [1, 1, 64, 64, -1, 4, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_profile", BWD_OK() + [1, 1, 31, 64, -1, 2, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_query_profile", BWD_OK() + [1, 1, 64, 64, -1, 15, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_query_profile", BWD_OK() + [1, 1, 16, 64, -1, 14, S0, S0, S0, S0, S0, None]),
    ("attention64_fp32_forward", FWD_OK() + [1, 1, 0, 1, -1, S0, S0, S0, S0, None]),
    ("attention64_fp32_backward", [None] + BWD_OK()[1:] + [1, 1, 1, 1, -1, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_flash_ex", FWD_OK() + [1, 1, 1, 1, -1, 2, S0, S0, S0, S0, None]),
    ("attention_fp32_forward_flash_ex", FWD_OK() + [1, 1, 1, 1, -7, 1, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_ex", BWD_OK() + [1, 1, 1, 1, -1, 8, S0, S0, S0, S0, S0, None]),   # unknown flag bit
    ("attention_fp32_backward_ex", BWD_OK() + [1, 1, 1, 1, -1, 6, S0, S0, S0, S0, S0, None]),   # fused + deterministic
    ("attention64_fp32_backward_ex", BWD_OK() + [1, 1, 1, 1, -1, 7, S0, S0, S0, S0, S0, None]),
    ("attention_fp32_backward_ex", BWD_OK() + [1, 1, 0, 1, -1, 3, S0, S0, S0, S0, S0, None]),
    ("attention64_fp32_backward_ex", BWD_OK()[:7] + [None] + BWD_OK()[8:] + [1, 1, 1, 1, -1, 2, S0, S0, S0, S0, S0, None]),
    ("attention64_fp32_forward_ex", FWD_OK() + [1, 1, 1, 1, -1, 2, S0, S0, S0, S0, None]),
    ("attention64_fp32_forward_ex", FWD_OK()[:3] + [None] + FWD_OK()[4:] + [1, 1, 1, 1, -1, 1, S0, S0, S0, S0, None]),
    ("attention64_fp32_backward_ex", BWD_OK() + [1, 1, 1, 1, -1, -1, S0, S0, S0, S0, S0, None]),
    ("attention_generic_forward", FWD_OK() + [1, 1, 1, 1, 48, -1, S0, S0, S0, S0, 0, None]),   # head width 48
    ("attention_generic_forward", FWD_OK() + [1, 1, 1, 1, 16, -2, S0, S0, S0, S0, 1, None]),   # radius < -1
    ("attention_generic_forward", FWD_OK() + [1, 1, 1, 1, 32, -1, S0, S0, S0, S0, 2, None]),   # unknown dtype
    ("attention_generic_forward", FWD_OK()[:5] + [None] + [1, 1, 1, 1, 64, -1, S0, S0, S0, S0, 0, None]),
    ("attention_generic_forward", FWD_OK() + [1, 1, 0, 1, 16, -1, S0, S0, S0, S0, 1, None]),
    ("rotary_fp32", [None] + FWD_OK()[1:] + [1, 1, 1, 0, S0, S0, S0, S0, None]),
    ("rotary_fp32", FWD_OK() + [1, 0, 1, 1, S0, S0, S0, S0, None]),
    ("rotary_fp32", FWD_OK() + [1, 1, -3, 0, S0, S0, S0, S0, None]),
    # token-reversed views (negative token stride) are outside the buffer-resource addressing: rejected up front
    ("attention_fp32_forward_flash", FWD_OK() + [1, 1, 8, 8, -1, attention.Strides(256, 256, -32), S0, S0, S0, None]),
    ("attention64_fp32_backward", BWD_OK() + [1, 1, 8, 8, -1, S0, S0, S0, S0, attention.Strides(512, 512, -64), None]),
])
def test_invalid_arguments_return_invalid_value(name, args):
    assert attention.call(name, *args) == attention.HIP_ERROR_INVALID_VALUE


def _compile_and_run(tmp_path, compiler, source, extra):
    binary = str(tmp_path / os.path.basename(source).split(".")[0])
    libdir = os.path.dirname(attention.library_path())
    cmd = [compiler, *extra, f"-I{INCLUDE}", "-I/opt/rocm/include", source, "-o", binary, f"-L{libdir}",
           f"-Wl,-rpath,{libdir}", "-l:libROCmKernels.Kernels.Shared.so", "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib",
           "-lamdhip64"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return subprocess.run([binary], capture_output=True, text=True, timeout=60)


def test_c_header_compiles_as_c_and_links(tmp_path):
    result = _compile_and_run(tmp_path, "gcc", os.path.join(ROOT, "tests", "cpp", "c_header_check.c"),
                              ["-std=c11", "-Wall", "-Wextra", "-Werror"])
    assert result.returncode == 0, result.stdout + result.stderr


def test_cpp_wrappers_throw_hip_error(tmp_path):
    result = _compile_and_run(tmp_path, "g++", os.path.join(ROOT, "tests", "cpp", "wrapper_check.cpp"),
                              ["-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__"])
    assert result.returncode == 0, result.stdout + result.stderr
    assert "0 failure(s)" in result.stdout


def test_persistent_work_partition_deals_every_item_once_and_balances(tmp_path):
    binary = str(tmp_path / "plan_check")
    source = os.path.join(ROOT, "tests", "cpp", "plan_check.cpp")
    csrc = os.path.join(ROOT, "rocmkernels_amd", "csrc")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{csrc}",
                    "-I/opt/rocm/include", source, "-o", binary], check=True, capture_output=True, text=True)
    result = subprocess.run([binary], capture_output=True, text=True, timeout=60)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "0 failure(s)" in result.stdout


def test_fused_backward_block_plan_covers_every_tile_once_and_balances(tmp_path):
    binary = str(tmp_path / "block_plan_check")
    source = os.path.join(ROOT, "tests", "cpp", "block_plan_check.cpp")
    csrc = os.path.join(ROOT, "rocmkernels_amd", "csrc")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{csrc}",
                    "-I/opt/rocm/include", source, "-o", binary], check=True, capture_output=True, text=True)
    result = subprocess.run([binary], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "0 failure(s)" in result.stdout


def test_band_backward_walk_covers_every_band_and_hands_dq_over_safely(tmp_path):
    binary = str(tmp_path / "band_walk_check")
    source = os.path.join(ROOT, "tests", "cpp", "band_walk_check.cpp")
    csrc = os.path.join(ROOT, "rocmkernels_amd", "csrc")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{csrc}",
                    "-I/opt/rocm/include", source, "-o", binary], check=True, capture_output=True, text=True)
    result = subprocess.run([binary], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "0 failure(s)" in result.stdout


def test_autograd_binding_rejects_host_tensors():
    import torch

    from rocmkernels_amd import autograd

    q = torch.zeros(1, 1, 4, 32)
    with pytest.raises(ValueError):
        autograd.attention_fp32(q, q, q, mask=torch.ones(1, 4, dtype=torch.uint8))


def test_static_library_defines_every_declared_symbol():
    archive = os.path.join(os.path.dirname(attention.library_path()), "libROCmKernels.Kernels.a")
    out = subprocess.run(["nm", "--defined-only", archive], check=True, capture_output=True, text=True).stdout
    defined = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared_symbols() <= defined


def test_static_library_links_into_a_cpp_consumer(tmp_path):
    # The reference's ROCmKernels.Kernels is a static library (CMakeLists.txt:117); a C++ program links this one the
    # same way (archive + HIP runtime) and gets the throwing wrappers' behaviour.
    archive = os.path.join(os.path.dirname(attention.library_path()), "libROCmKernels.Kernels.a")
    binary = str(tmp_path / "static_consumer")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}",
                    "-I/opt/rocm/include", os.path.join(ROOT, "tests", "cpp", "static_consumer.cpp"), archive, "-o", binary,
                    "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64"], check=True, capture_output=True, text=True)
    result = subprocess.run([binary], capture_output=True, text=True, timeout=60)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.count("HIP call failed") == 2


def test_cmake_project_targets_gfx950_only():
    # The configured build uses one offload arch, the reference's target names, and no other GPU toolchain.
    build = os.path.join(ROOT, "build", "build.ninja")
    with open(build) as handle:
        text = handle.read()
    arches = set(re.findall(r"--offload-arch=(\w+)", text))
    assert arches == {"gfx950"}
    assert "libROCmKernels.Kernels.a" in text and "libROCmKernels.Kernels.Shared.so" in text
    assert "nvcc" not in text and "cuda" not in text.lower().replace("--cuda-device-only", "")


def test_reference_style_cpp_caller_compiles_and_links_common(tmp_path):
    # A caller written as the reference's generic tests are (Generic/AttentionGenericTests.cpp:106-139): DeviceBuffer<__half>
    # storage, AttentionGenericForward(..., DTypeOf<__half>::value) and QueryDevice, linked against the static kernel
    # archive and ROCmKernels.Common (DeviceBuffer.hpp, Device.hpp, DType.hpp's DTypeOf). Without a GPU it checks the
    # empty buffer, the wrapper's invalid-argument throw and that the device queries report the missing device.
    lib_dir = os.path.dirname(attention.library_path())
    binary = str(tmp_path / "common_consumer")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", "-DCOMMON_CONSUMER_MAIN",
                    f"-I{INCLUDE}", "-I/opt/rocm/include", os.path.join(ROOT, "tests", "cpp", "common_consumer.cpp"),
                    os.path.join(lib_dir, "libROCmKernels.Kernels.a"), os.path.join(lib_dir, "libROCmKernels.Common.a"),
                    "-o", binary, "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64"],
                   check=True, capture_output=True, text=True)
    result = subprocess.run([binary], capture_output=True, text=True, timeout=60)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "0 failure(s)" in result.stdout
    assert "invalid argument" in result.stdout


def test_kernel_targets_link_common_publicly():
    # Both kernel targets carry ROCmKernels.Common to their consumers (the reference's CMakeLists.txt:120,133): the
    # GPU consumer, linked against ROCmKernels.Kernels.Shared alone, gets libROCmKernels.Common.a on its link line.
    with open(os.path.join(ROOT, "build", "build.ninja")) as handle:
        text = handle.read()
    links = [block for block in text.split("\nbuild ") if "librocmkernels_common_consumer.so" in block.split(":")[0]]
    assert links and "libROCmKernels.Common.a" in links[0]
    with open(os.path.join(ROOT, "CMakeLists.txt")) as handle:
        cmake = handle.read()
    assert "target_link_libraries(${target_name} PUBLIC ROCmKernels.Common" in cmake


def test_autograd_backward_mode_follows_torch_deterministic_mode_and_keeps_the_old_alias():
    import warnings

    import torch

    from rocmkernels_amd import autograd

    assert autograd.backward_mode(True) == (True, False)
    assert autograd.backward_mode(False) == (False, False)
    previous = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        assert autograd.backward_mode() == (True, False)
        torch.use_deterministic_algorithms(False)
        assert autograd.backward_mode() == (False, False)
    finally:
        torch.use_deterministic_algorithms(previous)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        assert autograd.backward_mode(fused_backward=True) == (False, True)
        assert autograd.backward_mode(fused_backward=False) == (True, False)
        assert autograd.backward_mode(False, fused_backward=True) == (False, True)
    assert len(caught) == 3 and all(issubclass(w.category, DeprecationWarning) for w in caught)
    with pytest.raises(ValueError), warnings.catch_warnings():
        warnings.simplefilter("ignore")
        autograd.backward_mode(True, fused_backward=True)

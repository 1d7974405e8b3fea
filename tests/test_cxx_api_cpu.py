"""The C++ layer/weights API (include/welvet/*.hpp) without a GPU: a C++
caller that includes only those headers links against libwelvet.so, the
library exports every declared entry point, and a call that needs the device
returns Unsupported (code 2) where none is visible, as the reference does for
a missing CUDA device."""
import os
import re
import subprocess

import numpy as np
import pytest

import cxx_probe
import pywelvet as pw

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADERS = ["weights.hpp", "dense.hpp", "dense_session.hpp", "swiglu.hpp", "mha.hpp",
           "dtype.hpp", "activate.hpp", "tensor.hpp", "device_state.hpp"]


def exported_cxx():
    out = subprocess.check_output(["nm", "-DC", "--defined-only", pw.LIB_PATH], text=True)
    return {l.split(" ", 2)[2] for l in out.splitlines() if " T " in l}


@pytest.mark.parametrize("name", [
    "welvet::WeightStore::make(int, int, welvet::DType, float const*, welvet::WeightStore*)",
    "welvet::WeightStore::decode_row_f64(int, double*) const",
    "welvet::WeightStore::export_f32(float*) const",
    "welvet::WeightStore::apply_sgd(double const*, double)",
    "welvet::dense::new_layer(int, int, welvet::Activation, welvet::DType, float const*, welvet::dense::Layer*)",
    "welvet::dense::forward_f32(welvet::dense::Layer const&, welvet::TensorF32 const&, welvet::TensorF32*, welvet::TensorF32*)",
    "welvet::dense::backward_f32(welvet::dense::Layer const&, welvet::TensorF32 const&, welvet::TensorF32 const&, welvet::TensorF32 const&, welvet::TensorF32*, welvet::TensorF32*)",
    "welvet::dense::session_mount(int, int, int, welvet::Activation, welvet::DType, float const*, double const*, unsigned long, welvet::dense::Session**)",
    "welvet::dense::session_execute(welvet::dense::Session*, float const*, float*, float*)",
    "welvet::dense::session_release(welvet::dense::Session*)",
    "welvet::swiglu::forward(welvet::swiglu::Layer&, welvet::TensorF32 const&, welvet::TensorF32*, welvet::TensorF32*)",
    "welvet::mha::forward(welvet::mha::Layer&, welvet::TensorF32 const&, welvet::TensorF32*, welvet::TensorF32*)",
    "welvet::TensorF32::zeros(long, long)",
    "welvet::dtype_name(welvet::DType)",
])
def test_library_exports_the_cxx_api(name):
    assert name in exported_cxx()


def test_every_header_is_self_contained(tmp_path):
    """Each public header compiles on its own (no torch, HIP or library
    internals needed by a caller)."""
    for h in HEADERS:
        src = tmp_path / "one.cpp"
        src.write_text(f'#include "welvet/{h}"\nint main() {{ return 0; }}\n')
        subprocess.check_call(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror",
                               "-I", os.path.join(ROOT, "include"), str(src)])


def test_dtype_names():
    import ctypes
    buf = ctypes.create_string_buffer(32)
    got = {}
    for i in range(-1, 35):
        served = cxx_probe.lib().probe_dtype(i, buf, 32)
        got[i] = (buf.value.decode(), served)
    assert got[4] == ("fp8e4m3", 1) and got[5] == ("fp8e5m2", 1) and got[16] == ("fp4", 1)
    assert got[1] == ("float32", 0) and got[33] == ("uint3", 0)
    assert got[-1] == ("unknown", 0) and got[34] == ("unknown", 0)


def test_new_layer_without_device_is_unsupported():
    if pw.lib().welvet_cuda_available():
        pytest.skip("a device is visible: the GPU suite covers this path")
    W = np.ones((4, 8), np.float32)
    x = np.ones((1, 8), np.float32)
    with pytest.raises(cxx_probe.ProbeError) as e:
        cxx_probe.dense_forward(8, 4, -1, 4, 0, W, x)
    assert e.value.code == 2


def test_argument_errors_before_the_device():
    """Shape and dtype errors are reported without touching a device."""
    W = np.ones((4, 8), np.float32)
    x = np.ones((1, 8), np.float32)
    with pytest.raises(cxx_probe.ProbeError) as e:
        cxx_probe.dense_forward(0, 4, -1, 4, 0, W, x)  # in = 0
    assert e.value.code == 1
    with pytest.raises(cxx_probe.ProbeError) as e:
        cxx_probe.dense_forward(8, 4, -1, 1, 0, W, x)  # float32 storage: not served
    assert e.value.code == 2

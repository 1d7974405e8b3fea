"""C-ABI checks that need no GPU: the library loads, exports every entry
point include/welvet_c.h declares, and rejects bad arguments before touching
a device (reference error convention, src/interop/c_abi.cpp:41-47, :125-137)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import pywelvet as pw

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def declared():
    text = open(os.path.join(ROOT, "include", "welvet_c.h")).read()
    return sorted(set(re.findall(r"WELVET_API[^;(]*?\b(welvet_\w+)\s*\(", text, re.S)))


def test_library_exports_every_declared_symbol():
    names = declared()
    assert len(names) >= 80
    out = subprocess.check_output(["nm", "-D", "--defined-only", pw.LIB_PATH], text=True)
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    L = pw.lib()
    for n in names:
        assert getattr(L, n) is not None


def test_version_and_abi():
    L = pw.lib()
    assert L.welvet_version() == b"0.79"
    assert L.welvet_model_abi_version() == 1
    assert L.welvet_gaps_count() + L.welvet_gaps_done() > 0


def test_seqmix_metadata():
    L = pw.lib()
    buf = ctypes.create_string_buffer(32)
    assert L.welvet_seqmix_kind_name(1, buf, 32).code == 0 and buf.value == b"ssm"
    assert L.welvet_seqmix_kind_name(9, buf, 32).code == 1
    assert (L.welvet_seqmix_mha_kind(), L.welvet_seqmix_mamba_kind(), L.welvet_seqmix_gdn_kind()) == (0, 1, 2)


def test_invalid_arguments_return_code_1():
    L = pw.lib()
    W = np.ones(4, np.float32)
    x = np.ones(2, np.float32)
    y = np.zeros(2, np.float32)
    st = L.welvet_dense_forward_f32(0, 2, 2, -1, 4, 0, pw.fptr(W), None, 0, pw.fptr(x), pw.fptr(y), pw.fptr(y))
    assert st.code == 1
    h = ctypes.c_void_p()
    assert L.welvet_dense_mount(1, 2, 2, -1, 4, None, None, 0, ctypes.byref(h)).code == 1
    assert L.welvet_dense_execute(None, pw.fptr(x), pw.fptr(y), pw.fptr(y)).code == 1
    assert L.welvet_swiglu_forward_f32(1, 0, 2, 2, 16, 0, pw.fptr(W), pw.fptr(W), pw.fptr(W), pw.fptr(x), pw.fptr(y), pw.fptr(y)).code == 1
    assert L.welvet_mha_forward_f32(1, 1, 0, 1, 1, 0, 0, 1, 0, 4, 0, *[pw.fptr(W)] * 5, pw.fptr(y), pw.fptr(y)).code == 1
    out = np.zeros(2, np.int64)
    assert L.welvet_codec_sweep(4, 4095, 2, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))).code == 1
    loss = np.zeros(1)
    assert L.welvet_dense_normalbp_f32(0, 2, 2, -1, 4, 0, pw.fptr(W), None, 0, pw.fptr(W), pw.fptr(W), 0, 0.0,
                                       *[pw.fptr(y)] * 5, pw.dptr(loss)).code == 1


def test_out_of_path_entry_points_report_gap():
    L = pw.lib()
    f = np.zeros(4, np.float32)
    st = L.welvet_rmsnorm_forward_f32(1, 1, 2, ctypes.c_double(1e-6), 1, 0, pw.fptr(f), pw.fptr(f), pw.fptr(f), pw.fptr(f))
    assert st.code == 3 and st.message.startswith(b"gap?")
    assert L.welvet_model_train_mse(None, 0, ctypes.c_double(0.1), 1, None, 0, None).code == 3


def _model_status(desc):
    L = pw.lib()
    buf = np.frombuffer(desc, np.uint8).copy()
    h = ctypes.c_void_p()
    return L.welvet_model_mount(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), buf.size, ctypes.byref(h))


def _stack_descriptor(extra=b"", magic=0x314E4D57, root=0):
    w = pw.Wire()
    w.u32(magic)
    w.i32(root, 1, 1, 1, 1, 1)
    W = np.eye(2, dtype=np.float32)
    pw.dense_child(w, 2, 2, -1, 4, W)
    pw.empty_controls(w)  # root
    pw.empty_controls(w)  # child
    w.i32(1)
    pw.store_payload(w, 4, 2, 2, np.array([0x38, 0, 0, 0x38], np.uint8))
    return w.bytes() + extra


def test_model_descriptor_rejections_before_device():
    assert _model_status(_stack_descriptor(magic=0x12345678)).code == 1
    assert _model_status(_stack_descriptor(extra=b"\0")).code == 1  # trailing bytes
    d = _stack_descriptor()
    assert _model_status(d[:-3]).code == 1  # truncated
    assert _model_status(_stack_descriptor(root=1)).code == 3  # Parallel root: gap


def test_no_device_reports_unsupported():
    L = pw.lib()
    if L.welvet_cuda_available():
        pytest.skip("a GPU is visible here")
    assert L.welvet_cuda_init().code == 2
    assert pw.lib().welvet_runtime_identity() == b"hip:unavailable"


def test_prng_is_splitmix64_box_muller():
    # splitmix64 from state 0 yields 0xE220A8397B1DCDAF first (Vigna's
    # reference sequence); u = ((z >> 11) + 0.5) 2^-53; Box-Muller cos branch.
    z = 0xE220A8397B1DCDAF
    z2 = 0x6E789E6AA1B965F4
    u1 = ((z >> 11) + 0.5) * 2.0 ** -53
    u2 = ((z2 >> 11) + 0.5) * 2.0 ** -53
    want = np.float32(np.sqrt(-2 * np.log(u1)) * np.cos(2 * np.pi * u2))
    assert pw.normal(0, 2)[0] == want
    a = pw.normal(pw.seed_for(2), 1 << 16)
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02
    assert np.array_equal(a, pw.normal(pw.seed_for(2), 1 << 16))


def _one_dense(scheme, f, tag_extra=0):
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(0, 1, 1, 1, 1, 1)
    w.i32(19, 1)
    pw.dense_child(w, 40, 2, -1, 4, np.zeros((2, 40), np.float32))
    pw.empty_controls(w)
    pw.empty_controls(w)
    pw.empty_controls(w)
    w.i32(1)
    w.i32(4 | (scheme << 8) | tag_extra, 2, 40)
    w.f32([1.0])
    w.i32(len(f))
    if len(f):
        w.f32(np.asarray(f, np.float32))
    w.i32(80)
    w.u8(np.zeros(80, np.uint8))
    w.i32(0)
    return np.frombuffer(w.bytes(), np.uint8).copy()


@pytest.mark.parametrize("scheme,f,ok", [
    (2, [0.5, 3.0], True),
    (2, [0.5], False),                              # one scale per row
    (2, [0.5, float("inf")], False),                 # finite row scales
    (3, [2.0 ** -127, 1.0, 2.0 ** 127, 0.25], True),  # 2 rows x 2 blocks, powers of two
    (3, [1.0, 1.5, 1.0, 1.0], False),                # 1.5 is no power of two
    (3, [1.0, 1.0], False),                          # rows * ceil(40/32) scales
    (1, [], True),
    (4, [], False),                                  # no scheme 4
])
def test_scaled_store_payload_parse(scheme, f, ok):
    """The scaled store extension is checked while parsing, before any device
    work: malformed payloads give code 1; well-formed ones get past the parse
    (code 2 here, no device; 0 on a GPU host)."""
    L = pw.lib()
    buf = _one_dense(scheme, f)
    h = ctypes.c_void_p()
    st = L.welvet_model_mount(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), buf.size,
                              ctypes.byref(h))
    if ok:
        assert st.code in (0, 2), st.message
        if st.code == 0:
            L.welvet_model_release(h)
    else:
        assert st.code == 1, st.message


@pytest.mark.parametrize("backend,ok", [(0, True), (3, True), (16, True), (19, True), (32, True),
                                        (34, True), (4, False), (48, False), (64, False),
                                        (-1, False)])
def test_model_backend_bits(backend, ok):
    """backend: scale scheme 0-3 in bits 0-3, bit 4 (16) asks for two
    activation terms, bit 5 (32) for one; both bits together, or anything
    else, is code 1, found before device work."""
    L = pw.lib()
    buf = _one_dense(0, [])
    h = ctypes.c_void_p()
    st = L.welvet_model_mount_q(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), buf.size,
                                backend, ctypes.byref(h))
    if ok:
        assert st.code in (0, 2), st.message
        if st.code == 0:
            L.welvet_model_release(h)
    else:
        assert st.code == 1, st.message

"""CPU checks of the C ABI (no GPU): the library loads, exports every symbol the
header declares, and the host-side validation maps each failure to the status
code / exception of the reference's tensor layer."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g4hip.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g4_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    syms = header_symbols()
    for must in ["g4_open", "g4_close", "g4_upload", "g4_matmul", "g4_matmul_dev", "g4_matmul_batch",
                 "g4_matmul_argmax", "g4_dequant", "g4_ffn", "g4_moe_route", "g4_moe", "g4_last_error"]:
        assert must in syms


def test_library_exports_every_header_symbol(g4):
    L = g4.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", g4.LIB_PATH], stdout=subprocess.PIPE, text=True).stdout
    exported = set(re.findall(r"\bT (g4_\w+)$", out, flags=re.M))
    for s in header_symbols():
        assert s in exported, s
        assert hasattr(L, s)
    # the Python binding declares a signature for each of them
    assert set(g4.SIGNATURES) == set(header_symbols())


def test_library_binds_to_torchs_hip_runtime():
    """Loaded through g4hip in a fresh interpreter, the library's HIP calls resolve
    to torch's own libamdhip64 (the runtime torch's tensors and streams live in),
    not to a second runtime from the system path."""
    code = ("import sys; sys.path.insert(0, %r); import g4hip; g4hip.lib(); "
            "assert 'torch' in sys.modules" % os.path.join(ROOT, "gemma4.kt_amd"))
    env = dict(os.environ, LD_DEBUG="bindings")
    r = subprocess.run(["python3", "-c", code], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stderr.splitlines() if "libg4hip.so" in l and "`hipLaunchKernel'" in l]
    assert lines, "no binding record for hipLaunchKernel"
    assert all("torch/lib/libamdhip64" in l for l in lines), lines


def test_no_device_here(g4):
    assert g4.device_count() == 0
    with pytest.raises(g4.IllegalStateException):
        g4.Context(0)
    h = ctypes.c_void_p()
    assert g4.lib().g4_open(0, ctypes.byref(h)) == -4
    assert "no HIP device" in g4.last_error()


def test_type_table(g4):
    # GGMLType.kt:16-32
    expect = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210),
              30: (1, 2)}
    for t, (bs, ts) in expect.items():
        assert g4.GGMLType(t).block_size == bs and g4.GGMLType(t).type_size == ts
    assert g4.GGMLType.Q8_0.byte_size_for(2048 * 2048) == 4456448
    assert g4.GGMLType.Q4_0.byte_size_for(8192 * 2048) == 9437184
    assert g4.GGMLType.Q4_K.byte_size_for(8192 * 2048) == 9437184
    assert g4.GGMLType.Q5_K.byte_size_for(8192 * 2048) == 11534336
    assert g4.GGMLType.Q6_K.byte_size_for(8192 * 2048) == 13762560


@pytest.mark.parametrize("bad", [3, 6, 7, 9, 10, 11, 15, 39, 41, -1])
def test_unsupported_type_ids(g4, bad):
    with pytest.raises(g4.UnsupportedOperationException):
        g4.check_matmul(bad, 1024, 0, 1, 1024)
    bs = ctypes.c_int32()
    assert g4.lib().g4_type_info(bad, ctypes.byref(bs), None) == -2


def test_byte_size_rejects_partial_blocks(g4):
    with pytest.raises(g4.IllegalArgumentException):
        g4.GGMLType.Q4_K.byte_size_for(300)
    with pytest.raises(g4.IllegalArgumentException):
        g4.GGMLType.Q8_0.byte_size_for(-32)


def test_geometry_validation(g4):
    n = 64 * 2048
    g4.check_matmul(8, n, 0, 64, 2048)
    g4.check_matmul(8, n, 2048, 63, 2048)
    g4.check_matmul(8, n, 0, 0, 2048)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.check_matmul(8, n, 1, 64, 2048)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.check_matmul(8, n, -32, 1, 32)
    with pytest.raises(g4.IllegalArgumentException):
        g4.check_matmul(8, n, 0, -1, 2048)
    with pytest.raises(g4.IllegalArgumentException):
        g4.check_matmul(8, 33, 0, 1, 32)
    # offsets past the reference's Int range are representable (int64)
    g4.check_matmul(0, 3 << 31, (1 << 32), 2, 1 << 20)


def test_null_arguments(g4):
    L = g4.lib()
    assert L.g4_close(None) == -1
    assert L.g4_matmul(None, None, 0, None, None, 1, 1) == -1
    assert L.g4_upload(None, 8, None, 0, 0, None) == -1
    assert L.g4_weight_free(None) == -1
    assert L.g4_device_count(None) == -1
    assert L.g4_moe(None, None, None, None, 1, 1, 1, None, None, 1, None) == -1
    assert L.g4_argmax(None, None, 1, None) == -1
    assert "null" in g4.last_error()


def test_last_error_is_thread_local(g4):
    import threading
    g4.lib().g4_close(None)
    seen = {}

    def other():
        seen["msg"] = g4.last_error()

    th = threading.Thread(target=other)
    th.start()
    th.join()
    assert seen["msg"] == "" and "null" in g4.last_error()


def test_python_errors_map_to_reference_exceptions(g4):
    assert issubclass(g4.UnsupportedOperationException, NotImplementedError)
    assert issubclass(g4.IndexOutOfBoundsException, IndexError)
    assert issubclass(g4.IllegalArgumentException, ValueError)
    with pytest.raises(g4.IllegalArgumentException):
        g4._f32(np.zeros(3, np.float64), "x")


def _fake_tensor(g4):
    """A GpuFloatTensor shell with no device behind it: the wrappers' argument
    checks run before any library call, so a short array must raise here."""
    t = object.__new__(g4.GpuFloatTensor)
    t.ctx, t.handle, t.size = type("C", (), {"handle": None})(), None, 0
    return t


def test_short_host_arrays_raise_index_out_of_bounds(g4):
    ctx = type("C", (), {"handle": None})()
    w = _fake_tensor(g4)
    short = np.zeros(7, np.float32)
    with pytest.raises(g4.IndexOutOfBoundsException):
        w.matmul(short, np.zeros(8, np.float32), 8, 8)
    with pytest.raises(g4.IndexOutOfBoundsException):
        w.matmul(np.zeros(8, np.float32), short, 8, 8)
    with pytest.raises(g4.IndexOutOfBoundsException):
        w.matmul_argmax(short, 8, 8)
    with pytest.raises(g4.IndexOutOfBoundsException):
        w.matmul_argmax(np.zeros(8, np.float32), 8, 8, logits=short)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.ffn(ctx, w, w, w, short, 8, 16)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.ffn_gate_up(ctx, w, w, short, 8, 16)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.ffn_block(ctx, w, w, w, w, w, short, 8, 16, 1e-6)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.lm_head(ctx, w, w, short, 32, 8, 1e-6, 0.0)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.moe_route(ctx, np.zeros((2, 8), np.float32), 2, True, expert_scale=short)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.moe_routed(ctx, w, w, np.zeros((2, 8), np.float32), np.zeros((2, 8), np.float32), 2, True, 8, 4,
                      expert_scale=short)
    # ids and weights of different lengths, or not T*k entries
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.moe(ctx, w, w, np.zeros((2, 8), np.float32), np.zeros((2, 3), np.int32), np.zeros(5, np.float32), 8, 4)
    with pytest.raises(g4.IndexOutOfBoundsException):
        g4.moe(ctx, w, w, np.zeros((2, 8), np.float32), np.zeros(5, np.int32), np.zeros(5, np.float32), 8, 4)
    with pytest.raises(g4.IllegalArgumentException):
        g4.moe(ctx, w, w, np.zeros(17, np.float32), np.zeros((2, 3), np.int32), np.zeros((2, 3), np.float32), 8, 4)


def test_device_index_arguments_must_be_int32_device_tensors(g4):
    import torch
    ctx = type("C", (), {"handle": None})()
    w = _fake_tensor(g4)
    for bad in (np.zeros(1, np.int32), torch.zeros(1, dtype=torch.int64), torch.zeros(1, dtype=torch.int32)):
        # host memory (numpy, or a CPU tensor) would hand the kernel a host address
        with pytest.raises(g4.IllegalArgumentException):
            g4._dev_i32(bad, "index")
        with pytest.raises(g4.IllegalArgumentException):
            w.matmul_argmax_dev(None, None, bad, 8, 8)
        with pytest.raises(g4.IllegalArgumentException):
            g4.moe_route_dev(ctx, None, 1, 8, 2, True, bad, None)
        with pytest.raises(g4.IllegalArgumentException):
            g4.lm_head_dev(ctx, w, w, None, None, bad, 8, 8, 1e-6, 0.0)
    assert g4._dev_i32(1234, "raw address") == 1234

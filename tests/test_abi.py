"""CPU tests of the C ABI: the library loads, exports every function include/flyeval.h declares, and its
host-side argument checks answer without a GPU.  No compute call is made here."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from helpers import REPO, tiny_connectome

HEADER = os.path.join(REPO, "include", "flyeval.h")


def _declared() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(fly_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    from chessfly import _hip
    if not os.path.exists(_hip.LIB_PATH):
        subprocess.run(["make", "-C", os.path.join(REPO, "alpha-fly_amd", "csrc"), "-j8"], check=True)
    return _hip.load()


def test_header_declares_the_expected_entry_points():
    names = _declared()
    assert {"fly_cone_create", "fly_plan_create", "fly_forward_io", "fly_forward_literal", "fly_model_forward",
            "fly_encoder", "fly_head", "fly_last_error", "fly_abi_version"} <= names


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in sorted(_declared()) if not hasattr(lib, name)]
    assert not missing, missing


def test_binding_covers_the_header_exactly():
    from chessfly import _hip
    assert set(_hip.SIGNATURES) == _declared()


def test_version_and_error_reporting_on_host(lib):
    assert lib.fly_abi_version() == 2
    assert lib.fly_set_tuning(b"no-such-knob", 1) == 1          # FLY_ERR_INVALID
    assert b"no-such-knob" in lib.fly_last_error()
    out = ctypes.c_void_p()
    assert lib.fly_cone_create(0, 0, None, None, None, 0, None, 0, 1, 0, None, ctypes.byref(out)) == 1
    assert out.value is None
    assert lib.fly_forward_io_workspace(None, 64) == 0


def test_product_refuses_cpu_tensors():
    """No CPU fallback: the drop-in classes raise instead of computing on the host."""
    from chessfly.brain import ConnectomeRNN
    rnn = ConnectomeRNN(tiny_connectome(), global_scale=3.0)
    with torch.no_grad():
        with pytest.raises(RuntimeError, match="HIP device"):
            rnn(torch.zeros(30, 4), 3)
        with pytest.raises(RuntimeError, match="HIP device"):
            rnn.forward_io(torch.zeros(5, 4), torch.arange(5), torch.arange(25, 30), 3)
    with pytest.raises(RuntimeError, match="HIP device"):
        rnn(torch.zeros(30, 4), 3)                              # the training path refuses the host as well
    with pytest.raises(RuntimeError, match="HIP device"):
        rnn.forward_io(torch.zeros(5, 4), torch.arange(5), torch.arange(25, 30), 3)


def test_evaluator_outputs_checks_arguments_on_host(lib):
    """fly_evaluator_outputs refuses null or negative arguments before launching anything."""
    assert lib.fly_evaluator_outputs(None, None, 1, 5, None, None, 0, None, None, None, None, None) == 1
    assert b"flag" in lib.fly_last_error()
    flag = ctypes.c_int32(0)
    assert lib.fly_evaluator_outputs(None, None, -1, 5, None, None, 0, None, None, None, ctypes.addressof(flag),
                                     None) == 1
    assert b"negative" in lib.fly_last_error()
    assert lib.fly_evaluator_outputs(None, None, 2, 5, None, None, 0, None, None, None, ctypes.addressof(flag),
                                     None) == 1
    assert b"wdl" in lib.fly_last_error()


def test_probe_library_is_apart_and_checks_arguments_on_host():
    """The bench's measurement probes live in libflyprobe.so, not in the evaluator's ABI: libflyeval.so exports
    no probe, and the probe library refuses null pointers and out-of-range sizes before launching anything."""
    from chessfly import _hip
    lib = _hip.load()
    assert not hasattr(lib, "fly_gather_probe")
    path = os.path.join(REPO, "alpha-fly_amd", "csrc", "libflyprobe.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-C", os.path.join(REPO, "alpha-fly_amd", "csrc"), "-j8"], check=True)
    probe = ctypes.CDLL(path)
    probe.flyprobe_last_error.restype = ctypes.c_char_p
    i64, p_ = ctypes.c_int64, ctypes.c_void_p
    probe.flyprobe_random_gather.argtypes = [p_, i64, i64, i64, p_, i64, p_, p_]
    probe.flyprobe_hashed_gather.argtypes = [p_, i64, i64, i64, i64, i64, i64, p_, p_]
    i32 = ctypes.c_int32
    probe.flyprobe_replay_step.argtypes = [p_, p_, i64, i64, p_, i64, i64, i64, i32, p_, p_, p_]
    assert probe.flyprobe_random_gather(None, 1024, 128, 128, None, 10, None, None) == 1
    buf = ctypes.create_string_buffer(16)
    p = ctypes.addressof(buf)
    assert probe.flyprobe_random_gather(p, 1 << 31, 128, 128, p, 10, p, None) == 1
    assert probe.flyprobe_random_gather(p, 1024, 64, 128, p, 10, p, None) == 1
    assert b"row_bytes" in probe.flyprobe_last_error()
    assert probe.flyprobe_random_gather(p, 1024, 128, 96, p, 10, p, None) == 1
    assert b"read_bytes" in probe.flyprobe_last_error()
    assert probe.flyprobe_hashed_gather(None, 1024, 8, 128, 128, 10, 1, p, None) == 1
    assert b"null" in probe.flyprobe_last_error()
    assert probe.flyprobe_hashed_gather(p, 1024, 9, 128, 128, 10, 1, p, None) == 1
    assert b"fit" in probe.flyprobe_last_error()
    assert probe.flyprobe_hashed_gather(p, 1024, 8, 128, 96, 10, 1, p, None) == 1
    assert b"read_bytes" in probe.flyprobe_last_error()
    assert probe.flyprobe_replay_step(None, None, 10, 10, None, 10, 64, 64, 1, None, None, None) == 1
    assert b"null" in probe.flyprobe_last_error()
    assert probe.flyprobe_replay_step(p, p, 10, 10, p, 10, 32, 64, 1, None, p, None) == 1
    assert b"layout" in probe.flyprobe_last_error()
    probe.flyprobe_replay_step_io.argtypes = [p_, p_, p_, i64, i64, p_, i64, i64, p_, i64, i64, p_, i64, i32, p_,
                                              p_]
    assert probe.flyprobe_replay_step_io(p, p, None, 10, 10, p, 10, 64, None, 0, 0, p, 64, 1, None, None) == 1
    assert b"null" in probe.flyprobe_last_error()
    assert probe.flyprobe_replay_step_io(p, p, p, 10, 10, p, 10, 64, p, 5, 32, p, 64, 1, None, None) == 1
    assert b"input drive" in probe.flyprobe_last_error()
    probe.flyprobe_sweep_create.argtypes = [p_, p_, i64, i64, i64, p_, ctypes.POINTER(p_), p_]
    out = p_(12345)
    cfg = (ctypes.c_int32 * 7)(8, 0, 0, 0, 0, 1, 0)
    assert probe.flyprobe_sweep_create(p, p, 10, 100, 10, cfg, ctypes.byref(out), None) == 1
    assert b"bands" in probe.flyprobe_last_error() and out.value is None
    cfg[0] = 4
    assert probe.flyprobe_sweep_create(None, p, 10, 100, 10, cfg, ctypes.byref(out), None) == 1
    assert b"null" in probe.flyprobe_last_error()


def test_tuning_is_read_and_written_under_a_lock(lib):
    """fly_set_tuning from several threads at once while others read the values back (fly_get_tuning): every read
    sees a value some writer set, unknown keys are refused, and the defaults come back when set."""
    import threading
    keys = [b"sweep_grid", b"sweep_piece", b"unroll", b"gemm_tile"]
    errors = []

    def writer(k, base):
        for i in range(2000):
            if lib.fly_set_tuning(k, base + i % 7) != 0:
                errors.append(("set", k))

    def reader(k, base):
        v = ctypes.c_int64(-1)
        for _ in range(2000):
            if lib.fly_get_tuning(k, ctypes.byref(v)) != 0 or not (v.value == 0 or base <= v.value < base + 7):
                errors.append(("get", k, v.value))

    threads = [threading.Thread(target=f, args=(k, 10 * (j + 1))) for j, k in enumerate(keys) for f in (writer, reader)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:5]
    v = ctypes.c_int64(-1)
    assert lib.fly_get_tuning(b"no-such-knob", ctypes.byref(v)) == 1
    for k in keys:
        assert lib.fly_set_tuning(k, 0) == 0
        assert lib.fly_get_tuning(k, ctypes.byref(v)) == 0 and v.value == 0

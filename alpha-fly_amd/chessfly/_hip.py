"""ctypes binding of libflyeval.so, the gfx950 HIP library behind the evaluator (include/flyeval.h).

Loading fails loudly: there is no CPU or PyTorch fallback for anything the library computes.  Device
pointers are passed as integers (torch `data_ptr()`), the stream is torch's current HIP stream.
"""

from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libflyeval.so")

ABI_VERSION = 2
MODE_DEVIATION_F16 = 0
MODE_F32 = 1
CONE_UNPRUNED = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_pp = ctypes.POINTER(ctypes.c_void_p)


class HeadDesc(ctypes.Structure):
    """fly_head_desc: RunningNorm statistics and the four read-out maps (device pointers)."""
    _fields_ = [("n_out", _i64), ("n_moves", _i64), ("norm_mean", _p), ("norm_var", _p), ("norm_eps", _f32),
                ("norm_clip", _f32), ("policy_w", _p), ("policy_b", _p), ("from_w", _p), ("from_b", _p),
                ("to_w", _p), ("to_b", _p), ("value_w", _p), ("value_b", _p), ("move_from", _p), ("move_to", _p)]


# name -> (restype, argtypes); every function declared in include/flyeval.h
SIGNATURES = {
    "fly_abi_version": (_i32, []),
    "fly_last_error": (ctypes.c_char_p, []),
    "fly_cone_create": (_i32, [_i64, _i64, _p, _p, _p, _i64, _p, _i64, _i32, _i32, _p, _pp]),
    "fly_cone_destroy": (_i32, [_p]),
    "fly_cone_sizes": (_i32, [_p, _p, _p, _p]),
    "fly_cone_rows": (_i32, [_p, _i32, _p, _p]),
    "fly_cone_step": (_i32, [_p, _i32, _p, _p, _p, _p, _p, _p]),
    "fly_cone_outputs": (_i32, [_p, _p, _p]),
    "fly_edge_weights": (_i32, [_p, _p, _p, _i64, _p, _p]),
    "fly_plan_create": (_i32, [_p, _p, _p, _p, _p, _p, _f32, _i32, _p, _pp]),
    "fly_plan_create_full": (_i32, [_i64, _i64, _p, _p, _p, _p, _f32, _p, _p, _pp]),
    "fly_plan_sweep_info": (_i32, [_p, _i32, _p]),
    "fly_sweep_create": (_i32, [_p, _p, _i64, _i64, _i64, _p, _pp]),
    "fly_sweep_destroy": (_i32, [_p]),
    "fly_sweep_info": (_i32, [_p, _p]),
    "fly_plan_destroy": (_i32, [_p]),
    "fly_plan_resting": (_i32, [_p, _p, _p]),
    "fly_plan_matrix": (_i32, [_p, _i32, _p, _p, _p, _p]),
    "fly_forward_io_workspace": (_sz, [_p, _i64]),
    "fly_forward_io": (_i32, [_p, _p, _i64, _i64, _p, _i64, _p, _sz, _p]),
    "fly_forward_io_f64_workspace": (_sz, [_p, _i64]),
    "fly_forward_io_f64": (_i32, [_p, _p, _i64, _i64, _p, _i64, _p, _sz, _p]),
    "fly_forward_literal_workspace": (_sz, [_p, _i64]),
    "fly_forward_literal": (_i32, [_p, _p, _i64, _p, _i64, _i32, _p, _i64, _p, _sz, _p]),
    "fly_forward_literal_f16_workspace": (_sz, [_p, _i64]),
    "fly_forward_literal_f16": (_i32, [_p, _p, _i64, _p, _i64, _i32, _p, _i64, _p, _sz, _p]),
    "fly_forward_literal_f64_workspace": (_sz, [_p, _i64]),
    "fly_forward_literal_f64": (_i32, [_p, _p, _i64, _p, _i64, _i32, _p, _i64, _p, _sz, _p]),
    "fly_plan_step_workspace": (_sz, [_p, _i32, _i64]),
    "fly_plan_step": (_i32, [_p, _i32, _p, _i64, _p, _i64, _i64, _p, _i64, _p, _sz, _p]),
    "fly_dense_create": (_i32, [ctypes.POINTER(HeadDesc), _p, _i64, _i64, _p, _i64, _p, _pp]),
    "fly_dense_destroy": (_i32, [_p]),
    "fly_encoder_workspace": (_sz, [_p, _i64]),
    "fly_encoder": (_i32, [_p, _p, _i32, _i64, _i64, _f32, _p, _i64, _i32, _p, _sz, _p]),
    "fly_head_workspace": (_sz, [_p, _i64]),
    "fly_head": (_i32, [_p, _p, _i64, _i64, _p, _p, _p, _sz, _p]),
    "fly_model_workspace": (_sz, [_p, _p, _i64]),
    "fly_model_forward": (_i32, [_p, _p, _p, _i32, _i64, _i64, _f32, _p, _p, _p, _sz, _p]),
    "fly_model_forward_static": (_i32, [_p, _p, _p, _i32, _i64, _i64, _f32, _p, _p, _p]),
    "fly_evaluator_outputs": (_i32, [_p, _p, _i64, _i64, _p, _p, _i64, _p, _p, _p, _p, _p]),
    "fly_evaluator_download": (_i32, [_p, _p, _sz, _i32, _p]),
    "fly_spmm": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i32, _p]),
    "fly_spmm_swept_workspace": (_sz, [_p, _i64]),
    "fly_spmm_swept": (_i32, [_p, _p, _i64, _p, _i64, _i64, _p, _i64, _p, _sz, _p]),
    "fly_transposed_backward": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _i32, _p,
                                       _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p]),
    "fly_gather_records": (_i32, [_p, _p, _i64, _p, _i64, _p, _p]),
    "fly_spmm_f64": (_i32, [_p, _p, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i32, _p]),
    "fly_sddmm_f64": (_i32, [_p, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _p, _i32, _p]),
    "fly_transposed_backward_swept_workspace": (_sz, [_p, _i64]),
    "fly_transposed_backward_swept": (_i32, [_p, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _i64, _p,
                                             _sz, _p]),
    "fly_train_step_forward": (_i32, [_i64, _i64, _p, _i64, _i32, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _f32, _p,
                                      _i64, _p]),
    "fly_train_step_backward": (_i32, [_i64, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _i64, _f32, _p, _i64, _p,
                                       _p, _p, _p, _i64, _p, _i64, _p]),
    "fly_sddmm": (_i32, [_p, _p, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _p, _i32, _p]),
    "fly_spmv_work": (_i32, [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i32, _p, _i64, _p, _i64, _p, _i64, _p]),
    "fly_gather_values": (_i32, [_p, _i64, _p, _i64, _p, _p]),
    "fly_rest_forward": (_i32, [_p, _p, _p, _i64, _i64, _p, _p, _p, _p, _f32, _p, _p, _p, _p, _p, _p]),
    "fly_rest_backward": (_i32, [_p, _p, _p, _p, _p, _p, _p, _f32, _i64, _p, _p, _p, _p, _p]),
    "fly_rest_products_backward": (_i32, [_p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64,
                                          _p, _p]),
    "fly_profile_enable": (_i32, [_i32]),
    "fly_profile_read": (_i32, [_p, _p]),
    "fly_profile_launches": (_i64, [_p, _p, _i64]),
    "fly_set_tuning": (_i32, [ctypes.c_char_p, _i64]),
    "fly_get_tuning": (_i32, [ctypes.c_char_p, _p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library, with argument types set.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C alpha-fly_amd/csrc` "
                               "(or __graft_entry__.build()); the evaluator has no fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        if lib.fly_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {lib.fly_abi_version()}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed ({status}): {load().fly_last_error().decode(errors='replace')}")


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the evaluator runs on a HIP device (ROCm GPU); got a {t.device} tensor")


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch bytes from torch's caching allocator (256-byte aligned by construction)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


KERNEL_CLASSES = ("state_step", "encoder", "head", "other")


def profile_enable(on: bool) -> None:
    check(load().fly_profile_enable(1 if on else 0), "fly_profile_enable")


def profile_read() -> dict:
    """{kernel class: (milliseconds, launches)} recorded since profiling was enabled."""
    ms = (ctypes.c_double * 4)()
    n = (ctypes.c_int64 * 4)()
    check(load().fly_profile_read(ms, n), "fly_profile_read")
    return {name: (float(ms[i]), int(n[i])) for i, name in enumerate(KERNEL_CLASSES)}


def profile_launches() -> list[tuple[str, float]]:
    """(kernel class, milliseconds) of every launch recorded since profiling was enabled, in launch order."""
    lib = load()
    n = lib.fly_profile_launches(None, None, 0)
    if n < 0:
        raise RuntimeError(f"fly_profile_launches failed: {lib.fly_last_error().decode(errors='replace')}")
    cls = (ctypes.c_int32 * max(n, 1))()
    ms = (ctypes.c_double * max(n, 1))()
    if lib.fly_profile_launches(cls, ms, n) != n:
        raise RuntimeError(f"fly_profile_launches failed: {lib.fly_last_error().decode(errors='replace')}")
    return [(KERNEL_CLASSES[cls[i]], float(ms[i])) for i in range(n)]


class Handle:
    """Owner of a library object (cone, plan, dense plan or sweep tables): destroyed with the matching C call."""

    def __init__(self, handle: ctypes.c_void_p, destroy: str, key=None):
        self.handle, self._destroy, self.key = handle, destroy, key

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                getattr(load(), self._destroy)(h)
            except Exception:
                pass
            self.handle = None


def set_tuning(key: str, value: int) -> None:
    check(load().fly_set_tuning(key.encode(), int(value)), "fly_set_tuning")


SWEEP_INFO = ("positions", "pieces", "split_rows", "rows_per_wave", "bands", "workgroups", "tables")


def sweep_info(handle, t: int | None = None) -> dict:
    """How a swept structure runs: from a fly_sweep (t None) or step t of a plan (all zero when it does not sweep)."""
    info = (ctypes.c_int64 * 7)()
    if t is None:
        check(load().fly_sweep_info(handle, info), "fly_sweep_info")
    else:
        check(load().fly_plan_sweep_info(handle, int(t), info), "fly_plan_sweep_info")
    return dict(zip(SWEEP_INFO, (int(v) for v in info)))


def sweep_create(crow32: torch.Tensor, col32: torch.Tensor, n_rows: int, n_cols: int):
    """The banded-sweep tables of one CSR structure (fly_sweep_create) as a Handle, or None when it does not sweep."""
    h = ctypes.c_void_p()
    check(load().fly_sweep_create(crow32.data_ptr(), col32.data_ptr(), n_rows, col32.numel(), n_cols,
                                  stream(crow32.device), ctypes.byref(h)), "fly_sweep_create")
    return Handle(h, "fly_sweep_destroy") if h.value else None

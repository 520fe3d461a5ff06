"""ctypes binding of libgsplat_hip.so, the C ABI declared in include/gsplat_hip.h.

This is the only place Python touches the native library.  Every call passes
raw device pointers, sizes and the current HIP stream; return codes are turned
into ``RuntimeError`` carrying the library's message.  There is no fallback:
if the library is missing or a tensor is not on the GPU, the call fails.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libgsplat_hip.so"

_P = c_void_p
# The interface _SIGNATURES below was written against: abi.header_abi_hash()
# of include/gsplat_hip.h.  load() refuses a library built from any other
# header, and a CPU test keeps this digest and _SIGNATURES equal to the
# header's.  Change all three together.
_ABI_VERSION = "0ed8ce82e6221bc5"

# name -> argtypes (restype int unless listed in _RESTYPES)
_SIGNATURES = {
    "gsplat_last_error": [],
    "gsplat_version": [],
    "gsplat_abi_version": [],
    "gsplat_projection_simple_fwd": [
        c_int64, c_int64, c_int64, _P, _P, _P, c_int32, c_int32, c_int32, _P, _P, _P],
    "gsplat_projection_simple_bwd": [
        c_int64, c_int64, c_int64, _P, _P, _P, c_int32, c_int32, c_int32, _P, _P, _P,
        _P, _P],
    "gsplat_projection_fused_fwd": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_float, c_float, c_float, c_int32,
        _P, _P, _P, _P, _P, _P],
    "gsplat_projection_fused_bwd": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_int32,
        _P, _P, _P, _P, _P, _P, _P,
        _P, _P, _P, _P, _P, _P],
    "gsplat_projection_packed_workspace_size": [c_int64, c_int64, c_int64],
    "gsplat_projection_packed_fwd": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_float, c_float, c_float, c_int32,
        _P, c_size_t,
        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_projection_packed_fwd_noalloc": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_float, c_float, c_float, c_int32,
        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_projection_packed_fwd_noalloc_max_rows": [],
    "gsplat_projection_packed_bwd": [
        c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_int32,
        _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int32,
        _P, _P, _P, _P, _P, _P],
    "gsplat_projection_packed_bwd_rows": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_int32,
        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_projection_packed_bwd_rows_sh": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_int32,
        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
        c_float, c_float, _P, _P, c_int32, c_int32, _P, _P, _P, _P],
    "gsplat_projection_packed_bwd_rows_stats": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_float, c_int32,
        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
        _P, c_float, c_float, _P, _P, _P],
    "gsplat_sh_fwd": [c_int64, c_int32, c_int32, _P, _P, _P, _P, _P],
    "gsplat_sh_bwd": [c_int64, c_int32, c_int32, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_sh_rows_fwd": [c_int64, c_int64, c_int64, c_int32, c_int32,
                           _P, _P, _P, _P, _P, _P],
    "gsplat_sh_rows_bwd": [c_int64, c_int64, c_int64, c_int32, c_int32,
                           _P, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_rows_gather": [c_int64, c_int64, c_int64, c_int32, _P, _P, _P, _P],
    "gsplat_rows_scatter_sum": [c_int64, c_int64, c_int64, c_int32, _P, _P, _P, _P],
    "gsplat_isect_count_workspace_size": [c_int64],
    "gsplat_isect_count": [
        c_int64, c_int64, _P, _P, _P, _P, _P, c_int32, c_int32, c_int32,
        _P, c_size_t, _P, _P, _P],
    "gsplat_isect_emit": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_int32, _P, _P, _P, _P],
    "gsplat_isect_prepare_workspace_size": [c_int64],
    "gsplat_isect_prepare": [
        c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32, c_int32,
        _P, c_size_t, _P, _P, _P, _P, _P, _P],
    "gsplat_isect_emit_sorted_workspace_size": [c_int64],
    "gsplat_isect_emit_sorted": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32,
        c_int32, _P, _P, _P, c_int64, _P, c_size_t, _P, _P, _P],
    "gsplat_isect_emit_sorted_dev": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32,
        c_int32, _P, _P, _P, c_int64, _P, c_size_t, _P, _P, _P],
    "gsplat_isect_prepare_rows_workspace_size": [c_int64],
    "gsplat_isect_prepare_rows": [
        c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32, c_int32,
        _P, c_size_t, _P, _P, _P, _P, _P],
    "gsplat_sh_rows_fwd_isect_count": [
        c_int64, c_int64, c_int64, c_int32, c_int32, _P, _P, _P, _P, _P,
        c_int64, _P, _P, _P, _P, _P, _P, _P, c_int32, c_int32, c_int32,
        _P, c_size_t, _P, _P, _P, _P],
    "gsplat_isect_row_starts": [c_int64, _P, c_size_t, _P, _P, _P],
    "gsplat_isect_emit_tiles_workspace_size": [c_int64],
    "gsplat_isect_emit_tiles": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32,
        c_int32, _P, _P, c_int64, _P, c_size_t, _P, _P, _P, _P],
    "gsplat_isect_emit_tiles_dev": [
        c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int32, c_int32,
        c_int32, _P, _P, c_int64, _P, c_size_t, _P, _P, _P, _P],
    "gsplat_sort_pairs_workspace_size": [c_int64],
    "gsplat_sort_pairs_u64_u32": [
        c_int64, c_int32, _P, _P, _P, _P, _P, c_size_t, _P],
    "gsplat_isect_offsets": [c_int64, _P, c_int64, c_int32, c_int32, _P, _P],
    "gsplat_rasterize_fwd": [
        c_int64, c_int64, c_int64, c_int32, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_rasterize_bwd": [
        c_int64, c_int64, c_int64, c_int32, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P,
        _P, _P, _P, _P, _P, _P, _P, _P],
    "gsplat_rasterize_replay_size": [c_int64, c_int32, c_int32, c_int32, c_int64, c_int32],
    "gsplat_rasterize_fwd_replay": [
        c_int64, c_int64, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P, _P,
        c_size_t, c_int32, _P, _P, c_int64, _P],
    "gsplat_rasterize_bwd_replay": [
        c_int64, c_int64, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P,
        c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P,
        _P, _P, _P, _P, _P, _P, _P, _P, c_size_t, _P, c_int32, _P],
    "gsplat_quat_scale_to_covar_preci_fwd": [c_int64, _P, _P, c_int32, _P, _P, _P],
    "gsplat_quat_scale_to_covar_preci_bwd": [
        c_int64, _P, _P, c_int32, _P, _P, _P, _P, _P],
    "gsplat_rasterize_to_indices_workspace_size": [c_int64],
    "gsplat_rasterize_to_indices_count": [
        c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, c_int32,
        c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P, c_size_t, _P],
    "gsplat_rasterize_to_indices_write": [
        c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, c_int32,
        c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P],
    "gsplat_grad2d_stats": [
        c_int64, c_int64, _P, _P, _P, c_float, c_float, _P, _P, _P],
    "gsplat_adam_multi": [_P, c_int32, c_float, c_float, c_float, _P],
    "gsplat_adam": [
        _P, _P, _P, _P, _P, c_int64, c_int64, c_float, c_float, c_float,
        c_float, _P],
}
_RESTYPES = {
    "gsplat_last_error": ctypes.c_char_p,
    "gsplat_version": ctypes.c_char_p,
    "gsplat_abi_version": ctypes.c_char_p,
    "gsplat_projection_packed_workspace_size": c_size_t,
    "gsplat_rasterize_replay_size": c_size_t,
    "gsplat_projection_packed_fwd_noalloc_max_rows": c_int64,
    "gsplat_isect_count_workspace_size": c_size_t,
    "gsplat_sort_pairs_workspace_size": c_size_t,
    "gsplat_isect_prepare_workspace_size": c_size_t,
    "gsplat_isect_emit_sorted_workspace_size": c_size_t,
    "gsplat_isect_prepare_rows_workspace_size": c_size_t,
    "gsplat_isect_emit_tiles_workspace_size": c_size_t,
    "gsplat_rasterize_to_indices_workspace_size": c_size_t,
}


class AdamTensor(ctypes.Structure):
    """Mirror of ``gsplat_adam_tensor`` (include/gsplat_hip.h)."""

    _fields_ = [
        ("param", c_void_p),
        ("grad", c_void_p),
        ("exp_avg", c_void_p),
        ("exp_avg_sq", c_void_p),
        ("valid", c_void_p),
        ("n_rows", c_int64),
        ("row_size", c_int64),
        ("lr", c_float),
    ]


_lib: Optional[ctypes.CDLL] = None


_REBUILD = "build it with `python gsplat_amd/build.py`"


def load() -> ctypes.CDLL:
    """Load libgsplat_hip.so (once), check that it was built from the
    interface this binding was written against, and declare its signatures.
    A library of another interface is refused before any entry point is
    bound or called."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: {_REBUILD} "
            "(the HIP kernels are the only implementation; there is no fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    try:
        abi_fn = lib.gsplat_abi_version
    except AttributeError:
        raise RuntimeError(
            f"{LIB_PATH} reports no interface version (gsplat_abi_version is "
            f"missing); this binding expects ABI {_ABI_VERSION}: {_REBUILD}") from None
    abi_fn.argtypes = []
    abi_fn.restype = ctypes.c_char_p
    got = (abi_fn() or b"").decode(errors="replace")
    if got != _ABI_VERSION:
        raise RuntimeError(
            f"{LIB_PATH} was built from interface ABI {got}, but this binding "
            f"(gsplat_amd/_lib.py) was written for ABI {_ABI_VERSION}; calling it "
            f"could pass arguments of the wrong type: {_REBUILD}")
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


class EntryTimer:
    """Records HIP events on the current stream around chosen entry points.

    ``EntryTimer({"gsplat_rasterize_bwd"})`` installed with ``timing(...)``
    brackets every call of those entry points; ``results()`` (after a device
    synchronize) gives the per-entry list of durations in ms.  An empty set
    times every entry point.
    """

    def __init__(self, names=None):
        self.names = set(names or ())
        self.events = {}

    def wants(self, name: str) -> bool:
        return not self.names or name in self.names

    def record(self, name: str):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return e

    def add(self, name: str, start, end) -> None:
        self.events.setdefault(name, []).append((start, end))

    def results(self):
        return {k: [s.elapsed_time(e) for s, e in v] for k, v in self.events.items()}


_timer: Optional[EntryTimer] = None


class timing:
    """Context manager installing an EntryTimer."""

    def __init__(self, timer: EntryTimer):
        self.timer = timer

    def __enter__(self):
        global _timer
        self.prev, _timer = _timer, self.timer
        return self.timer

    def __exit__(self, *exc):
        global _timer
        _timer = self.prev
        return False


def call(name: str, *args) -> None:
    """Invoke an int-returning entry point and raise on failure."""
    lib = load()
    t = _timer
    if t is not None and t.wants(name):
        start = t.record(name)
        rc = getattr(lib, name)(*args)
        t.add(name, start, t.record(name))
    else:
        rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.gsplat_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def query(name: str, *args) -> int:
    """Invoke a size-returning entry point."""
    return int(getattr(load(), name)(*args))


def version() -> str:
    return load().gsplat_version().decode()


def stream() -> int:
    """Handle of the current HIP stream of the current device."""
    return torch.cuda.current_stream().cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    """Device address of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def check_input(t: Optional[torch.Tensor], name: str, dtype: Optional[torch.dtype] = None):
    """Device + contiguity (+ dtype) check, mirroring CHECK_INPUT
    (gsplat/cuda/include/Common.h:31-36)."""
    if t is None:
        return
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must have dtype {dtype}, got {t.dtype}")

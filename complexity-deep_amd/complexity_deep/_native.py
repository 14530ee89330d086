"""ctypes binding of libcdx.so, the gfx950 kernel library declared in include/cdx.h.

This is the only place the package touches native code.  There is no CPU or
PyTorch fallback: if the library is missing, or a tensor is not a bf16 tensor on a
ROCm device, the call raises.  Every launch goes onto the caller's current torch
stream and nothing synchronises the host.
"""

from __future__ import annotations

import contextlib
import ctypes
from pathlib import Path
from typing import Callable, Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libcdx.so"

_lib = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> (restype, argtypes), mirroring include/cdx.h
_SIGNATURES = {
    "cdx_version": (ctypes.c_int, []),
    "cdx_last_error": (ctypes.c_char_p, []),
    "cdx_add_rmsnorm_fwd": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_float, _i64, _i32, _vp, _vp, _vp]),
    "cdx_rmsnorm_ld_fwd": (ctypes.c_int, [_vp, _vp, ctypes.c_float, _i64, _i32, _vp, _i64, _vp]),
    "cdx_route_workspace_bytes": (ctypes.c_size_t, [_i64, _i32]),
    "cdx_route_plan": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                      ctypes.c_size_t, _vp]),
    "cdx_route_plans_workspace_bytes": (ctypes.c_size_t, [_i64, _i32, _i32]),
    "cdx_route_plans": (ctypes.c_int, [_vp, _i64, _vp, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                       ctypes.c_size_t, _vp]),
    "cdx_route_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "cdx_route_plan_noalloc": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "cdx_permute_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "cdx_unpermute_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "cdx_moe_swiglu_fwd": (ctypes.c_int, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                          _vp, _vp]),
    "cdx_moe_swiglu_residual_fwd": (ctypes.c_int, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                                   _vp, _vp, _vp]),
    "cdx_grouped_gemm_fwd": (ctypes.c_int, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "cdx_swiglu_fwd": (ctypes.c_int, [_vp, _vp, _i64, _i32, _i32, _vp, _vp]),
    "cdx_mu_qkv_fwd": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _i64,
                                      _vp]),
    "cdx_mu_qkv_rope_fwd": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i32, _i32,
                                           _i32, _i32, _vp, _vp, ctypes.c_float, _vp, _i64, _i64, _vp, _vp,
                                           _vp, _i64, _vp]),
    "cdx_mu_qkv_rope_bcast_fwd": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32,
                                                 _i32, _i32, _vp, _vp, ctypes.c_float, _vp, _i64, _i64, _vp,
                                                 _vp, _vp, _i64, _vp, _vp]),
    "cdx_attention_fwd": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i64, ctypes.c_float,
                                         _vp, _vp]),
    "cdx_mu_guidance_fwd": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, ctypes.c_float, ctypes.c_float,
                                           ctypes.c_float, ctypes.c_float, _vp, _i64, _vp]),
    "cdx_binpack_map": (ctypes.c_int, [_vp, _i64, _i32, _vp]),
    "cdx_embedding_fwd": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i32, _vp, _vp]),
    "cdx_linear_fwd": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]),
    "cdx_linear_residual_fwd": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]),
    "cdx_hbm_probe": (ctypes.c_int, [_i32, _vp, _vp, _i64, _vp]),
}


class NativeLibraryMissing(RuntimeError):
    pass


def lib():
    """Load libcdx.so once (raises NativeLibraryMissing if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing: build it with `python complexity-deep_amd/build_native.py` "
                "(or __graft_entry__.build()); there is no fallback path")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


# Optional per-call timing hook: when set, every C-ABI launch site records a pair of
# timing events on the stream the kernels go to and hands them to the hook as
# hook(name, start_event, end_event, shape_dict).  None (the default) costs one test.
_launch_hook: Optional[Callable] = None


def set_launch_hook(hook: Optional[Callable]) -> None:
    global _launch_hook
    _launch_hook = hook


class _NoRegion:
    """The region of an unhooked launch: nothing to record."""
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_REGION = _NoRegion()


@contextlib.contextmanager
def _timed_region(hook, name: str, device: torch.device, shape: dict):
    s = torch.cuda.current_stream(device)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(s)
    yield
    e1.record(s)
    hook(name, e0, e1, shape)


def launch_region(name: str, device: torch.device, **shape):
    """Bracket the launches of one C-ABI call with timing events (when hooked).

    The events go on the device's current torch stream, which is the stream every
    entry point is given (stream_of).  Unhooked (the default) it is a shared no-op
    context, so that a launch pays no generator set-up."""
    hook = _launch_hook
    if hook is None:
        return _NO_REGION
    return _timed_region(hook, name, device, shape)


def exported_symbols():
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().cdx_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def stream_of(t: torch.Tensor) -> int:
    """The raw hipStream_t of the current torch stream on t's device (what
    torch.cuda.current_stream(t.device).cuda_stream returns, without building a Stream
    object on every launch)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def row_stride(t: torch.Tensor, H: int, what: str) -> int:
    """Row stride (elements) of a [..., H] tensor whose rows are base + r * ld with unit
    stride inside a row, e.g. a column slice of a wider buffer.  Raises if the rows are
    not evenly spaced: an output is written in place and cannot be made contiguous."""
    if t.shape[-1] != H or t.stride(-1) != 1:
        raise ValueError(f"{what}: rows of {H} elements with unit stride expected, got shape {tuple(t.shape)} "
                         f"strides {t.stride()}")
    rows = t.numel() // H if H else 0
    if t.dim() == 1 or rows <= 1:
        return H
    dims = [(n, st) for n, st in zip(t.shape[:-1], t.stride()[:-1]) if n != 1]
    ld = dims[-1][1]
    for (n_outer, st_outer), (n_inner, st_inner) in zip(dims, dims[1:]):
        if st_outer != st_inner * n_inner:
            raise ValueError(f"{what}: rows are not evenly spaced (strides {t.stride()})")
    if ld < H:
        raise ValueError(f"{what}: row stride {ld} is smaller than the row ({H})")
    return ld


def require_device(*tensors: Optional[torch.Tensor], dtype: Optional[torch.dtype] = torch.bfloat16,
                   what: str = "op") -> None:
    """All tensors on one ROCm device (and of `dtype` if given)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{what}: tensors must be on a ROCm GPU (got {t.device}); "
                               "the MI355X kernels have no CPU path")
        if dtype is not None and t.dtype != dtype:
            raise RuntimeError(f"{what}: expected {dtype}, got {t.dtype}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} vs {t.device})")

"""Loader of liblocals_amd.so (the C ABI declared in include/locals_amd.h) and argument plumbing.

The product path has no fallback: if the library is not built, or no GPU is present when a kernel is called, this
module raises.  Tensors cross the boundary as raw device pointers; every call is enqueued on torch's current stream
of the tensor's device and nothing here synchronises.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblocals_amd.so")

F16, BF16, F32 = 0, 1, 2
_DT = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}
_STATUS = {-1: "invalid argument", -2: "unsupported shape", -3: "workspace too small",
           -4: "needs more than the allocation-free entry point's fixed scratch"}

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
Z = ctypes.c_size_t
LL = ctypes.c_longlong

# name -> (restype, argtypes); must match include/locals_amd.h
SIGNATURES = {
    "lcl_decode_workspace_bytes": (Z, [I, I, I, I]),
    "lcl_qkv_attend": (I, [P, I, P, P, P, P, P, P, I, P, P, F, I, I, I, I, I, I, I, P, P, Z, P]),
    "lcl_qkv_attend_ex": (I, [P, I, P, P, P, P, P, P, I, P, P, F, I, I, I, I, I, I, I, P, P, Z, P, P, P]),
    "lcl_qkv_attend_noalloc": (I, [P, I, P, P, P, P, P, P, I, P, P, F, I, I, I, I, I, I, I, P, P]),
    "lcl_ragged_attention": (I, [P, I, P, P, I, P, P, F, P, I, I, I, I, I, I, I, P, P, Z, P]),
    "lcl_ragged_attention_ex": (I, [P, I, P, P, I, P, P, F, P, I, I, I, I, I, I, I, P, P, Z, P, P, P]),
    "lcl_quantize_append": (I, [P, P, I, P, P, P, P, P, P, I, I, I, I, I, I, I, P]),
    "lcl_dequantize": (I, [P, P, P, I, ctypes.c_longlong, I, P, I, P]),
    "lcl_kv_gather": (I, [P, P, P, I, I, I, I, P, P, P, P, P, P, P, P]),
    "lcl_sdpa_workspace_bytes": (Z, [I, I, I, I, I]),
    "lcl_sdpa_workspace_bytes_kv": (Z, [I, I, I, I, I, I, I, I, I]),
    "lcl_sdpa": (I, [P, I, I, P, P, P, P, P, P, P, P, I, P, I, I, P, LL, P, LL, LL, LL, LL, P, F, I, I, I, I, I, I, I, I,
                     P, P, Z, P]),
    "lcl_sdpa_ex": (I, [P, I, I, P, P, P, P, P, P, P, P, I, P, I, I, P, LL, P, LL, LL, LL, LL, P, F, I, I, I, I, I, I, I,
                        I, P, P, Z, P, P, P]),
    "lcl_qk_norm_rope": (I, [P, I, P, P, P, I, F, F, I, I, I, I, I, I, P, P, P, P]),
    "lcl_qk_norm_rope_append": (I, [P, I, P, P, P, I, F, F, I, I, I, I, I, I, P, P, P, P, P, P, P, I, I, I, P]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """The C ABI library (loaded once).  Raises RuntimeError if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `python -m locals_amd.build` (no CPU fallback exists)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise ValueError(f"unsupported dtype {t}") from None


def ptr(t) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    if rc < 0:
        raise ValueError(f"{what}: {_STATUS.get(rc, 'error')} (status {rc})")
    raise RuntimeError(f"{what}: HIP error {rc}")


def require_gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("locals_amd kernels take GPU tensors (there is no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same GPU")
    return dev

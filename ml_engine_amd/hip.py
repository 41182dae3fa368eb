"""ctypes binding of include/mle_hip.h (libmle_hip.so).

The HIP library is the product path: there is no fallback.  If the shared
library is missing, loading raises instead of computing anything elsewhere.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent / "lib"

P = C.c_void_p
I = C.c_int
SZ = C.c_size_t
F = C.c_float
D = C.c_double
I64 = C.c_int64

# name -> (restype, argtypes); mirrors include/mle_hip.h
SIGNATURES: dict[str, tuple] = {
    "mle_last_error": (C.c_char_p, []),
    "mle_version": (C.c_char_p, []),
    "mle_init": (I, [I]),
    "mle_device_alloc": (I, [C.POINTER(P), SZ]),
    "mle_device_free": (I, [P]),
    "mle_memcpy_h2d": (I, [P, P, SZ, P]),
    "mle_memcpy_d2h": (I, [P, P, SZ, P]),
    "mle_memcpy_d2d": (I, [P, P, SZ, P]),
    "mle_read_scalar": (I, [P, P, P]),
    "mle_scalar_last": (I, [P]),
    "mle_scalar_state": (I, [P, P, P]),
    "mle_scalar_clear": (I, []),
    "mle_scalar_expect": (I, [P, C.c_uint, P]),
    "mle_graph_capture_begin": (I, [P]),
    "mle_graph_capture_end": (I, [P, P]),
    "mle_graph_launch": (I, [P, P]),
    "mle_graph_destroy": (I, [P]),
    "mle_stream_create": (I, [C.POINTER(P)]),
    "mle_stream_destroy": (I, [P]),
    "mle_stream_sync": (I, [P]),
    "mle_arena_create": (I, [SZ, C.POINTER(P)]),
    "mle_arena_alloc": (I, [P, SZ, C.POINTER(P)]),
    "mle_arena_reset": (I, [P]),
    "mle_arena_destroy": (I, [P]),
    "mle_arena_used": (SZ, [P]),
    "mle_arena_capacity": (SZ, [P]),
    "mle_fill": (I, [P, P, F, SZ]),
    "mle_scale_add": (I, [P, P, P, P, F, SZ]),
    "mle_accumulate": (I, [P, P, P, D, SZ]),
    "mle_scale_write": (I, [P, P, P, F, SZ]),
    "mle_scale_assign": (I, [P, P, P, D, SZ]),
    "mle_accumulate2": (I, [P, P, P, I, P, I, SZ]),
    "mle_add_act_fwd": (I, [P, P, P, P, P, I, SZ]),
    "mle_act_bwd_add": (I, [P, P, P, I, P, I, P, I, P, I, SZ]),
    "mle_scale_inplace": (I, [P, P, F, I, SZ]),
    "mle_scale_by_device": (I, [P, P, P, I, SZ]),
    "mle_bias_add_rows": (I, [P, P, P, SZ, I]),
    "mle_broadcast_channel_add": (I, [P, P, P, P, I, I, SZ]),
    "mle_headify": (I, [P, P, P, I, I, I, I, I]),
    "mle_matpe": (I, [P, P, P, I, I, I, I]),
    "mle_timestep_pe": (I, [P, P, I, I]),
    "mle_matpe_table": (I, [P, P, I, I, I]),
    "mle_add_broadcast": (I, [P, P, P, P, I, SZ]),
    "mle_act_fwd": (I, [P, I, P, P, SZ]),
    "mle_act_bwd": (I, [P, I, P, P, P, SZ, I]),
    "mle_gemm": (I, [P, I, I, I, I, I, F, P, I64, I64, P, I64, I64, F, P, I64, I64, I, P]),
    "mle_gemm_ws_bytes": (SZ, [I, I, I, I]),
    "mle_gemm_ex": (I, [P, I, I, I, I, I, F, P, I64, I64, P, I64, I64, F, P, I64, I64, I, P, P, P, SZ]),
    "mle_gemm_batched_ex": (I, [P, I, I, I, I, I, F, P, I64, I64, P, I64, I64, F, P, I64, I64, I, P, I64, P, I64, P, SZ]),
    "mle_gemm_sum_ws_bytes": (SZ, [I, I, I]),
    "mle_gemm_sum": (I, [P, I, I, I, I, I, F, P, I64, I64, P, I64, I64, F, P, I64, I, P, SZ]),
    "mle_gemm_grid": (I, [P, I, I, I, I, I, F, P, I64, I64, I64, P, I64, I64, I64, F, P, I64, I64, I64, I, I, P, SZ]),
    "mle_gemm_rowstats": (I, [P, I, I, I, I, I, F, P, I64, P, I64, F, P, I64, P, P, I64, P, SZ]),
    "mle_softmax_xent_keys_fwd_rowstats": (I, [P, P, P, I64, P, I, I, P, I, I, P, P, SZ]),
    "mle_softmax_xent_keys_fwd_rowstats_read": (I, [P, P, P, I64, P, I, I, P, I, I, P, P, SZ, P]),
    "mle_gemm_act_fwd": (I, [P, I, I, I, I, I, F, P, I64, P, I64, F, P, P, I, P, P, SZ]),
    "mle_gemm_act_bwd": (I, [P, I, I, I, I, I, F, P, I64, P, I64, F, P, I, P, P, I, P, SZ]),
    "mle_linear_bwd_ws_bytes": (SZ, [I, I, I, I]),
    "mle_linear_bwd": (I, [P, I, I, I, I, P, P, I64, P, I64, P, I, P, P, I64, P, SZ]),
    "mle_linear_bwd_ex": (I, [P, I, I, I, I, P, P, I64, P, I64, P, I, P, P, I64, I, P, SZ]),
    "mle_linear_bwd_act": (I, [P, I, I, I, P, P, P, P, I, P, P, I, I, P, P, I, P, SZ]),
    "mle_colsum": (I, [P, P, SZ, I, P, F]),
    "mle_channel_sum": (I, [P, P, I, I, SZ, I, P]),
    "mle_channel_sum_ex": (I, [P, P, I, I, SZ, I, P, SZ, I]),
    "mle_softmax_fwd": (I, [P, P, P, I, I, I, I, I]),
    "mle_softmax_bwd": (I, [P, P, P, P, I, I, I, I, I]),
    "mle_attention_ws_bytes": (SZ, [I, I, I]),
    "mle_attention_fwd": (I, [P, P, P, P, P, I, I, I, I, I, F, I, P, SZ]),
    "mle_attention_bwd": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, F, I, I, I, I, I, P, SZ]),
    "mle_loss_ws_bytes": (SZ, [SZ]),
    "mle_mse_fwd": (I, [P, P, P, SZ, P, P, SZ]),
    "mle_mse_fwd_read": (I, [P, P, P, SZ, P, P, SZ, P]),
    "mle_mse_fwd_bwd_read": (I, [P, P, P, SZ, P, P, P, SZ, P]),
    "mle_mse_act_fwd_bwd_read": (I, [P, P, P, SZ, I, P, P, P, P, SZ, P]),
    "mle_add_mse_act_fwd_bwd_read": (I, [P, P, P, P, P, SZ, I, P, P, P, P, SZ, P]),
    "mle_mse_bwd": (I, [P, P, P, P, P, SZ, I]),
    "mle_softmax_xent_keys_fwd": (I, [P, P, P, I, I, P, I, I, P, P, SZ]),
    "mle_softmax_xent_keys_small_read": (I, [P, P, P, I, I, P, I, I, I, P, P, P]),
    "mle_linear_xent_keys_small_read": (I, [P, I, I, I, P, P, P, P, P, I, I, P, I, P, P, P]),
    "mle_softmax_xent_keys_bwd": (I, [P, P, P, P, I, I, P, P, I, I, I]),
    "mle_softmax_xent_fwd": (I, [P, P, P, P, I, I, P, P, SZ]),
    "mle_softmax_xent_bwd": (I, [P, P, P, P, P, SZ, I]),
    "mle_norm_ws_bytes": (SZ, [I, I, SZ, I]),
    "mle_norm_fwd": (I, [P, P, P, P, I, I, SZ, I, F, P, SZ]),
    "mle_norm_fwd_ex": (I, [P, P, P, P, I, I, SZ, I, F, P, SZ, I]),
    "mle_add_norm_partials": (I, [P, P, P, SZ, P, I, I, SZ, I, P, SZ]),
    "mle_norm_fwd_act": (I, [P, P, P, P, I, P, I, I, SZ, I, F, P, SZ, I]),
    "mle_norm_fwd_act_bias": (I, [P, P, P, P, I, P, P, I, I, SZ, I, F, P, SZ, I]),
    "mle_norm_bwd_act": (I, [P, P, P, I, P, I, P, P, I, I, SZ, I, F, I, P, SZ, I]),
    "mle_norm_bwd": (I, [P, P, P, P, P, I, I, SZ, I, F, I, P, SZ, I]),
    "mle_norm_bwd_partials": (I, [P, P, P, P, I, I, I, I, SZ, I, I, P, SZ]),
    "mle_norm_bwd_apply_add": (I, [P, P, P, P, I, P, P, I, P, I, P, I, I, SZ, I, F, I, P, SZ]),
    "mle_batchnorm_ws_bytes": (SZ, [I, I, SZ]),
    "mle_batchnorm_fwd": (I, [P, P, P, P, I, I, SZ, F, P, SZ]),
    "mle_batchnorm_bwd": (I, [P, P, P, P, P, I, I, SZ, F, P, SZ, I]),
    "mle_rmsnorm_fwd": (I, [P, P, P, P, I, I, I, I]),
    "mle_rmsnorm_bwd": (I, [P, P, P, P, P, I, I, I, I, I]),
    "mle_copy_crop_fwd": (I, [P, P, P, P, I, I, I, I, I, I, I]),
    "mle_copy_crop_bwd": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I]),
    "mle_weight_swap": (I, [P, P, P, I, I, I, I]),
    "mle_conv2d_fwd": (I, [P, P, P, P, P, I, I, I, I, I, I, I, I, I]),
    "mle_conv2d_dgrad": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, I]),
    "mle_conv2d_wgrad_ws_bytes": (SZ, [I, I, I, I, I, I, I, I, I]),
    "mle_conv2d_wgrad": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, P, SZ]),
    "mle_conv2d_wgrad_bias": (I, [P, P, P, P, P, I, I, I, I, I, I, I, I, I, I, P, SZ]),
    "mle_conv2d_pair_supported": (I, [I, I, I, I, I, I]),
    "mle_conv2d_pair_fwd": (I, [P, P, I, I, I, I, P, P, P, I, P, P, P, I]),
    "mle_conv2d_pair_dgrad": (I, [P, P, I, I, I, I, I, P, P, I, P, P, I]),
    "mle_sqnorm_ws_bytes": (SZ, [SZ]),
    "mle_grad_sqnorm": (I, [P, P, SZ, P, P, P, SZ]),
    "mle_sqrt_scale": (I, [P, P, D]),
    "mle_grad_sqnorm_ex": (I, [P, P, SZ, P, P, I, D, P, SZ]),
    "mle_adam_update": (I, [P, P, P, P, P, SZ, I, F, F, F, F, F, I, P]),
    "mle_adamw_clip_ws_bytes": (SZ, [SZ]),
    "mle_adamw_clip_fused": (I, [P, P, P, P, P, SZ, I, F, F, F, F, F, I, D, P, P, SZ]),
    "mle_adamw_clip_fused_noalloc": (I, [P, P, P, P, P, SZ, I, F, F, F, F, F, I, D, P]),
    "mle_embed_gather": (I, [P, P, P, P, I, I, I, I]),
    "mle_embed_scatter_ws_bytes": (SZ, [I, I]),
    "mle_embed_scatter_add": (I, [P, P, P, P, I, I, I, I, I, F, P, SZ]),
    "mle_embed_grad": (I, [P, P, P, P, I, I, I, I, I, I, P, SZ]),
    "mle_embed_index_bytes": (SZ, [I, I, I]),
    "mle_embed_gather_indexed": (I, [P, P, P, P, I, I, I, I, I, P, SZ]),
    "mle_embed_grad_indexed": (I, [P, P, P, P, I, I, I, I, I]),
    "mle_onehot": (I, [P, P, P, I, I, I, I]),
    "mle_onehot_update": (I, [P, P, P, P, I, I, I, I]),
    "mle_argmax": (I, [P, P, I, I, P]),
    "mle_probe_arm": (I, [C.c_char_p]),
    "mle_probe_read": (I, [C.POINTER(I), C.POINTER(D), C.POINTER(D), C.POINTER(D)]),
    "mle_event_create": (I, [C.POINTER(P)]),
    "mle_event_record": (I, [P, P]),
    "mle_event_elapsed_ms": (I, [P, P, C.POINTER(F)]),
    "mle_event_destroy": (I, [P]),
}

ACT = {"relu": 0, "gelu": 1, "silu": 2, "tanh": 3, "sigmoid": 4, "leaky_relu": 5}


class MLEError(RuntimeError):
    pass


_lib = None


def lib() -> C.CDLL:
    """Load libmle_hip.so (built in-tree by ml_engine_amd.build)."""
    global _lib
    if _lib is None:
        path = LIB_DIR / "libmle_hip.so"
        if not path.exists():
            raise MLEError(f"{path} is missing: run `python -m ml_engine_amd.build` (or __graft_entry__.build())")
        _lib = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise MLEError(f"mle status {rc}: {lib().mle_last_error().decode()}")


def call(name: str, *args):
    """Call an int-returning C ABI function and raise on failure."""
    check(getattr(lib(), name)(*args))


_inited = False


def init(device: int = 0) -> None:
    global _inited
    if not _inited:
        call("mle_init", device)
        _inited = True


class Buffer:
    """A device allocation owned from Python (test / bench plumbing)."""

    def __init__(self, nbytes: int):
        init()
        self.nbytes = max(int(nbytes), 1)
        p = P()
        call("mle_device_alloc", C.byref(p), self.nbytes)
        self.ptr = p.value
        self.dtype = None
        self.shape = None

    @classmethod
    def from_array(cls, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.dtype, b.shape = a.dtype, a.shape
        if a.nbytes:
            call("mle_memcpy_h2d", b.ptr, a.ctypes.data, a.nbytes, None)
        return b

    @classmethod
    def zeros(cls, shape, dtype=np.float32) -> "Buffer":
        return cls.from_array(np.zeros(shape, dtype=dtype))

    @classmethod
    def empty(cls, shape, dtype=np.float32) -> "Buffer":
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        b = cls(n)
        b.dtype, b.shape = np.dtype(dtype), tuple(shape) if np.ndim(shape) else (int(shape),)
        return b

    def numpy(self, shape=None, dtype=None) -> np.ndarray:
        dtype = np.dtype(dtype or self.dtype or np.float32)
        shape = shape if shape is not None else (self.shape if self.shape is not None else (self.nbytes // dtype.itemsize,))
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            call("mle_stream_sync", None)
            call("mle_memcpy_d2h", out.ctypes.data, self.ptr, out.nbytes, None)
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        call("mle_memcpy_h2d", self.ptr, a.ctypes.data, a.nbytes, None)

    def free(self) -> None:
        if getattr(self, "ptr", None):
            lib().mle_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync(stream=None) -> None:
    call("mle_stream_sync", stream)


class Event:
    """A device event (mle_event_*): record on a stream, read the time between two."""

    def __init__(self):
        init()
        p = P()
        call("mle_event_create", C.byref(p))
        self.ptr = p.value

    def record(self, stream=None) -> None:
        call("mle_event_record", self.ptr, stream)

    def ms_since(self, start: "Event") -> float:
        ms = F()
        call("mle_event_elapsed_ms", start.ptr, self.ptr, C.byref(ms))
        return ms.value

    def __del__(self):
        try:
            if getattr(self, "ptr", None):
                lib().mle_event_destroy(self.ptr)
                self.ptr = None
        except Exception:
            pass


def version() -> str:
    return lib().mle_version().decode()

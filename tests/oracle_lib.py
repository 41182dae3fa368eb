"""ctypes loader for the CPU oracle (oracle/liboracle.so) -- test infrastructure."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
P = C.c_void_p
I = C.c_int
LL = C.c_longlong
F = C.c_float
D = C.c_double
PP = C.POINTER(C.c_void_p)

SIGS = {
    "orc_num_threads": (I, []),
    "orc_set_threads": (None, [I]),
    "orc_bcmm": (None, [I, P, P, P, I, I, I, I, I, I, I, I, I, F]),
    "orc_bcmm_naive": (None, [I, P, P, P, I, I, I, I, I, I, I, I, I, F]),
    "orc_bcompress": (None, [P, P, LL, I, F]),
    "orc_bcumadd": (None, [P, P, LL, I]),
    "orc_channel_squeeze": (None, [P, P, I, I, LL, I]),
    "orc_broadcast_add": (None, [P, P, P, I, I, LL]),
    "orc_scale_add": (None, [P, P, P, F, LL]),
    "orc_accumulate": (None, [P, P, D, LL]),
    "orc_scale_write": (None, [P, P, F, LL]),
    "orc_act_fwd": (None, [I, P, P, LL]),
    "orc_act_bwd": (None, [I, P, P, P, LL]),
    "orc_headify": (None, [P, P, I, I, I, I, I]),
    "orc_matpe": (None, [P, P, I, I, I, I]),
    "orc_pe": (None, [P, I, I]),
    "orc_softmax": (None, [P, P, I, I, I, I, I]),
    "orc_softmax_bwd": (None, [P, P, P, I, I, I, I]),
    "orc_norm_fwd": (None, [P, P, P, I, I, LL, I, F]),
    "orc_norm_bwd": (None, [P, P, P, P, I, I, LL, I, F, I]),
    "orc_conv_fwd": (None, [P, P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_conv_dgrad": (None, [P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_conv_wgrad": (None, [P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_conv_fwd_naive": (None, [P, P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_conv_dgrad_naive": (None, [P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_conv_wgrad_naive": (None, [P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_mse_loss": (F, [P, P, LL]),
    "orc_mse_bwd": (None, [P, P, P, P, LL]),
    "orc_softmax_xent_fwd": (F, [P, P, P, I, I]),
    "orc_softmax_xent_bwd": (None, [P, P, P, P, LL, I]),
    "orc_sumsq": (None, [P, LL, P]),
    "orc_sqrt_scale": (None, [P, D]),
    "orc_clip": (None, [P, LL, P]),
    "orc_adam": (None, [P, P, LL, I, P, P, F, F, F, F, F, I]),
    "orc_gather": (None, [P, P, P, I, I, I, I]),
    "orc_scatter_add": (None, [P, P, P, I, I, I, I, I, F]),
    "orc_onehot": (None, [P, P, I, I, I, I]),
    "orc_argmax": (None, [P, I, I, P]),
    "orc_rmsnorm_fwd": (None, [P, P, P, I, I, I, I]),
    "orc_rmsnorm_bwd": (None, [P, P, P, P, I, I, I, I]),
    "orc_batchnorm_fwd": (None, [P, P, P, I, I, LL, F]),
    "orc_batchnorm_bwd": (None, [P, P, P, P, I, I, LL, F]),
    "orc_copy_crop_fwd": (None, [P, P, P, I, I, I, I, I, I, I]),
    "orc_copy_crop_bwd": (None, [P, P, P, I, I, I, I, I, I, I]),
    "orc_convT_fwd": (None, [P, P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_convT_dgrad": (None, [P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_convT_wgrad": (None, [P, P, P, I, I, I, I, I, I, I, I, I]),
    "orc_c1_step": (F, [I, I, I, I, P, P, PP, PP, PP, PP, F, I, I, P]),
    "orc_c4_step": (F, [I, I, I, I, I, I, P, P, PP, PP, PP, PP, F, I, I]),
    "orc_c5_step": (F, [I, I, I, I, I, I, I, I, P, P, PP, PP, PP, PP, F, I, I]),
}

_lib = None
_V4_FLAGS = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}


def host_has_v4() -> bool:
    """True when this CPU has the x86-64-v4 (AVX-512) extensions liboracle_v4.so is built for."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("flags"):
                return _V4_FLAGS <= set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return False


def lib_path() -> Path:
    v4 = ROOT / "oracle" / "liboracle_v4.so"
    return v4 if v4.exists() and host_has_v4() else ROOT / "oracle" / "liboracle.so"


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        path = lib_path()
        if not path.exists():
            raise RuntimeError(f"{path} missing: run `make -C oracle` or __graft_entry__.build()")
        _lib = C.CDLL(str(path))
        for name, (res, args) in SIGS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


def ptr_table(arrs: list[np.ndarray]):
    t = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    return t


def call(name: str, *args):
    return getattr(lib(), name)(*args)

"""ctypes driver for the engine's model harness (libmle_engine.so).

Builds the benchmark configurations with the C++ GraphOperations API and steps
them; used by the tests and bench.py.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip

KIND = {"mlp": 1, "flat": 2, "block": 4, "resblock": 5, "unet_up": 6, "conv_layernorm": 7}
STEP_ZERO, STEP_FORWARD, STEP_BACKWARD, STEP_UPDATE, STEP_ALL = 1, 2, 4, 8, 15
STEP_CLOBBER_SCALE = 16
P, I, LL, F, SZ = C.c_void_p, C.c_int, C.c_longlong, C.c_float, C.c_size_t

_SIGS = {
    "mle_model_create": (P, [I, C.POINTER(LL), I]),
    "mle_model_destroy": (None, [P]),
    "mle_model_set_quirks": (None, [I, I, I]),
    "mle_model_set_seed": (None, [C.c_ulonglong]),
    "mle_model_set_lazy_zero": (None, [I]),
    "mle_model_set_fusion": (None, [I]),
    "mle_model_num_params": (I, [P]),
    "mle_model_param_name": (C.c_char_p, [P, I]),
    "mle_model_param_numel": (LL, [P, I]),
    "mle_model_param_t": (I, [P, I]),
    "mle_model_param_io": (I, [P, I, I, P, I]),
    "mle_model_grads_save": (I, [P]),
    "mle_model_grads_restore": (I, [P]),
    "mle_model_input": (I, [P, I, P, SZ]),
    "mle_model_step": (I, [P, F, I, F]),
    "mle_model_step_graph": (I, [P, F, I]),
    "mle_model_loss": (F, [P]),
    "mle_model_clip_pending": (LL, []),
    "mle_model_target_read": (I, [P, P, SZ]),
    "mle_model_sync": (I, [P]),
    "mle_model_stream": (P, [P]),
    "mle_model_num_nodes": (I, [P]),
    "mle_model_node_numel": (LL, [P, I]),
    "mle_model_node_read": (I, [P, I, I, P, SZ]),
    "mle_model_save": (I, [P, C.c_char_p]),
    "mle_model_load": (I, [P, C.c_char_p]),
    "mle_model_temb_save": (I, [P, C.c_char_p, C.POINTER(C.c_char_p), I]),
    "mle_model_temb_load": (I, [P, C.c_char_p, I, C.POINTER(C.c_char_p), I]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        hip.lib()  # libmle_hip.so first: the engine links against it
        path = hip.LIB_DIR / "libmle_engine.so"
        if not path.exists():
            raise hip.MLEError(f"{path} is missing: run `python -m ml_engine_amd.build`")
        _lib = C.CDLL(str(path))
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


class Model:
    """One configuration built with the engine (parameters in the flat arena)."""

    def __init__(self, kind: str, dims, seed: int = 0, reference_quirks: bool = True, lazy_zero: bool = True,
                 fuse: bool = True, layernorm_reference_layout: bool | None = None):
        L = lib()
        hip.init(0)
        ln = reference_quirks if layernorm_reference_layout is None else layernorm_reference_layout
        L.mle_model_set_quirks(int(reference_quirks), int(reference_quirks), int(ln))
        L.mle_model_set_lazy_zero(int(lazy_zero))
        L.mle_model_set_fusion(int(fuse))
        L.mle_model_set_seed(seed)
        arr = (LL * len(dims))(*[int(d) for d in dims])
        self.h = L.mle_model_create(KIND[kind], arr, len(dims))
        if not self.h:
            raise hip.MLEError(f"model {kind} {dims} not created")
        self.kind = kind
        self.dims = list(dims)
        n = L.mle_model_num_params(self.h)
        self.names = [L.mle_model_param_name(self.h, i).decode() for i in range(n)]
        self.numel = [int(L.mle_model_param_numel(self.h, i)) for i in range(n)]

    # which: 0 params, 1 grads, 2 m, 3 v
    def get(self, i: int, which: int = 0) -> np.ndarray:
        out = np.empty(self.numel[i], np.float32)
        hip.check(lib().mle_model_param_io(self.h, i, which, out.ctypes.data, 0))
        return out

    def set(self, i: int, arr: np.ndarray, which: int = 0) -> None:
        a = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
        assert a.size == self.numel[i], (self.names[i], a.size, self.numel[i])
        hip.check(lib().mle_model_param_io(self.h, i, which, a.ctypes.data, 1))

    def input(self, slot: int, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        hip.check(lib().mle_model_input(self.h, slot, a.ctypes.data, a.nbytes))

    def step(self, lr: float, mode: int = STEP_ALL, clip: float = 0.0) -> None:
        hip.check(lib().mle_model_step(self.h, lr, mode, clip))

    def step_graph(self, lr: float, mode: int = STEP_ALL) -> None:
        """The same step with zero_grad / forward / backward replayed as one recorded graph."""
        hip.check(lib().mle_model_step_graph(self.h, lr, mode))

    def grads_save(self) -> None:
        hip.check(lib().mle_model_grads_save(self.h))

    def grads_restore(self) -> None:
        hip.check(lib().mle_model_grads_restore(self.h))

    def sync(self) -> None:
        hip.check(lib().mle_model_sync(self.h))

    @property
    def loss(self) -> float:
        return float(lib().mle_model_loss(self.h))

    def target(self, count: int) -> np.ndarray:
        """The first `count` floats of the one-hot target matrix (C1 / C4)."""
        out = np.empty(count, np.float32)
        rc = lib().mle_model_target_read(self.h, out.ctypes.data, count)
        if rc != 0:
            raise RuntimeError(f"mle_model_target_read failed ({rc})")
        return out

    @property
    def stream(self):
        return lib().mle_model_stream(self.h)

    def t(self, i: int) -> int:
        return int(lib().mle_model_param_t(self.h, i))

    def nodes(self) -> int:
        return int(lib().mle_model_num_nodes(self.h))

    def node(self, i: int, which: int = 0) -> np.ndarray | None:
        """Node i's output (0) or gradient (1), as ReadValueAt reads it; None
        when the node has no such buffer."""
        n = int(lib().mle_model_node_numel(self.h, i))
        out = np.empty(max(n, 0), np.float32)
        if lib().mle_model_node_read(self.h, i, which, out.ctypes.data, out.size) != 0:
            return None
        return out

    def save(self, path: str) -> None:
        hip.check(lib().mle_model_save(self.h, str(path).encode()))

    def load(self, path: str) -> None:
        hip.check(lib().mle_model_load(self.h, str(path).encode()))

    @staticmethod
    def _words(words):
        arr = (C.c_char_p * len(words))(*[None if w is None else w.encode() for w in words])
        return arr, len(words)

    def temb_save(self, path: str, words) -> None:
        arr, n = self._words(words)
        hip.check(lib().mle_model_temb_save(self.h, str(path).encode(), arr, n))

    def temb_load(self, path: str, replace: bool = False, words=()) -> int:
        arr, n = self._words(list(words))
        return int(lib().mle_model_temb_load(self.h, str(path).encode(), int(replace), arr, n))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().mle_model_destroy(self.h)
            self.h = None

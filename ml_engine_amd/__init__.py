"""MI355X-native (gfx950) backward / optimizer hot path of ML_Engine.

Native parts (built in-tree by ml_engine_amd.build):
  lib/libmle_hip.so     hand-written HIP kernels behind the C ABI in include/mle_hip.h
  lib/libmle_engine.so  the GraphOperations / NodeBackProp / AdamParameter C++ layer

Python here is plumbing for tests and the benchmark (ctypes over the C ABI).
"""
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
__all__ = ["ROOT"]

"""CPU checks of the drop-in boundary: the C ABI library loads and exports every
function declared in include/*.h, and the Python binding covers them all.
No compute is launched (there is no GPU here)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(mle_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    assert len(names) > 40
    for required in ["mle_gemm", "mle_adamw_clip_fused", "mle_norm_bwd", "mle_softmax_bwd", "mle_conv2d_wgrad",
                     "mle_embed_scatter_add", "mle_arena_create", "mle_grad_sqnorm"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    path = ROOT / "ml_engine_amd" / "lib" / "libmle_hip.so"
    if not path.exists():
        pytest.fail(f"{path} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_matches_header():
    from ml_engine_amd import hip

    declared = set(declared_functions())
    bound = set(hip.SIGNATURES)
    assert declared == bound, f"header-only: {sorted(declared - bound)}, binding-only: {sorted(bound - declared)}"


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from ml_engine_amd import hip

    monkeypatch.setattr(hip, "LIB_DIR", tmp_path)
    monkeypatch.setattr(hip, "_lib", None)
    with pytest.raises(hip.MLEError):
        hip.lib()

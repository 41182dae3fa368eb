"""The allocation-free optimizer entry point (mle_adamw_clip_fused_noalloc)
against mle_adamw_clip_fused with a caller workspace: the same kernels, so the
parameters, both moments and the clip scale must agree bit for bit.  Two calls
in a row on the device's shared scratch, the second over a smaller span, so a
value left in the scratch by the first call would show in the second."""
import ctypes as C

import numpy as np
import pytest

from ml_engine_amd import hip as H

pytestmark = pytest.mark.gpu


def _state(n, seed):
    r = np.random.default_rng(seed)
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    g[r.random(n) < 0.01] *= 100.0  # the global norm exceeds 1, so the clip divides
    m = (r.standard_normal(n) * 1e-4).astype(np.float32)
    v = (r.random(n) * 1e-7).astype(np.float32)
    return p, g, m, v


def _run(n, seed, t, adamw, clip, noalloc):
    p, g, m, v = _state(n, seed)
    bp, bg, bm, bv = (H.Buffer.from_array(a) for a in (p, g, m, v))
    norm = H.Buffer.zeros(1, np.float64)
    args = (None, bp.ptr, bg.ptr, bm.ptr, bv.ptr, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01, adamw, clip, norm.ptr)
    if noalloc:
        H.call("mle_adamw_clip_fused_noalloc", *args)
    else:
        ws_bytes = H.lib().mle_adamw_clip_ws_bytes(n)
        ws = H.Buffer(ws_bytes)
        H.call("mle_adamw_clip_fused", *args, ws.ptr, ws_bytes)
    H.sync()
    out = [b.numpy() for b in (bp, bm, bv)] + [norm.numpy()]
    for b in (bp, bg, bm, bv, norm):
        b.free()
    return out


@pytest.mark.parametrize("adamw", [1, 0])
def test_noalloc_matches_workspace_entry_point(hip, adamw):
    # first a large span (the norm uses the full 8192 partials), then a much
    # smaller one with an odd length (scalar tail), at a later step t
    for n, seed, t in ((50_000_003, 1, 1), (12_347, 2, 7)):
        ref = _run(n, seed, t, adamw, 1.0, noalloc=False)
        got = _run(n, seed, t, adamw, 1.0, noalloc=True)
        assert ref[3][0] > 1.0, ref[3]
        for what, a, b in zip(("p", "m", "v", "norm"), got, ref):
            np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8), err_msg=f"n={n} {what}")


def test_noalloc_without_clip_and_empty_span(hip):
    ref = _run(4099, 3, 2, 1, 0.0, noalloc=False)
    got = _run(4099, 3, 2, 1, 0.0, noalloc=True)
    for a, b in zip(got[:3], ref[:3]):
        np.testing.assert_array_equal(a, b)
    # n == 0 returns without launching anything (the pointers are never read)
    rc =H.lib().mle_adamw_clip_fused_noalloc(None, C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), 0,
                                              1, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1, 1.0, None)
    assert rc == 0
    # a null operand is rejected before any launch
    rc = H.lib().mle_adamw_clip_fused_noalloc(None, None, None, None, None, 16, 1, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1, 1.0,
                                              None)
    assert rc == -1 and b"null pointer" in H.lib().mle_last_error()

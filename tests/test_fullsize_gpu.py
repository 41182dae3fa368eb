"""Parity against the oracle at the benchmark configurations' real sizes.

The kernel and engine tests elsewhere run reduced shapes; these run the exact
shapes bench.py times, so the kernel dispatch they exercise is the measured
one (persistent and pair GEMM kernels, LM-head row-statistics epilogue, fused
attention at seq 256 x 8 heads, the register-direct convolutions at 64 -> 128
channels, the 100 M-parameter arena):
  C4  transformer block step, batch 32, seq 256, d 512, 8 x 64 heads, FFN 2048,
      vocab 8000, AdamW                         vs orc_c4_step
  C5  U-Net residual block step, 64 -> 128 channels at 64 x 64, GN(32), time
      dim 256, batch 2 and 16 (the timed one), AdamW   vs orc_c5_step
  C3  Linear backward 8192 x 1024 x 4096 through the two mle_gemm calls bench.py
      makes: 256 sampled dX rows, 256 sampled dW columns, the whole db
  C2  accumulate + clipNorm + AdamW over 100 M parameters in 64 tensors, 10
      steps                                     vs orc_sumsq / orc_sqrt_scale /
                                                   orc_clip / orc_adam
Tolerances (written per test): 1e-4 relative for GEMM / conv results, 1e-5
relative for the optimizer, with an absolute floor relative to the largest
reference magnitude for sums that cancel.
"""
import numpy as np
import pytest

from conftest import assert_close
from ml_engine_amd import hip as H
from ml_engine_amd.configs import (BlockConfig, FlatConfig, GemmConfig, ResBlockConfig, block_data, flat_data,
                                   gemm_data, resblock_data)
from ml_engine_amd.models import STEP_ALL, Model
from test_engine_gpu import check_update, oracle_tables

pytestmark = pytest.mark.gpu

GRAD = dict(rtol=1e-4, atol_scale=1e-5)   # composed GEMM / conv gradients
EW = dict(rtol=1e-5, atol_scale=1e-6)     # optimizer state


def _report(what, got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    s = np.abs(ref).max()
    print(f"[fullsize] {what}: max|err| / max|ref| = {np.abs(got - ref).max() / max(s, 1e-300):.3g}", flush=True)


def test_c4_full_size_vs_oracle(hip, orc):
    cfg = BlockConfig()
    print(f"[fullsize] C4 {cfg}", flush=True)
    ids, tgt, params = block_data(cfg, seed=3)
    m = Model("block", cfg.dims(), reference_quirks=True)
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, ids)
    m.input(1, tgt)
    m.step(cfg.lr, STEP_ALL)
    m.sync()
    op, og, om, ov = oracle_tables(params)
    T = orc.ptr_table
    loss = orc.call("orc_c4_step", cfg.batch, cfg.seq, cfg.d_model, cfg.heads, cfg.ffn, cfg.vocab, orc.ptr(ids),
                    orc.ptr(tgt), T(op), T(og), T(om), T(ov), 0.0, 1, 0)
    print(f"[fullsize] C4 loss {m.loss!r} oracle {loss!r}", flush=True)
    assert abs(m.loss - loss) <= 1e-5 * abs(loss), (m.loss, loss)
    for i in range(len(params)):
        got = m.get(i, 1)
        _report(f"C4 grad {m.names[i]}", got, og[i])
        # the query bias gradient is zero by symmetry (a per-column shift of the
        # scores leaves a column-normalised softmax unchanged): biases are judged
        # on the scale of their layer's weight gradient, which sums the same dY
        s = max(np.abs(og[i]).max(), np.abs(og[i - 1]).max()) if i >= 2 and i % 2 == 0 else None
        assert_close(got, og[i], what=f"C4 grad {m.names[i]}", scale=s, **GRAD)
    check_update(orc, m, params, cfg.lr, 1, True, "C4")
    m.close()


@pytest.mark.parametrize("batch", [2, 16])
def test_c5_full_size_vs_oracle(hip, orc, batch):
    """Batch 16 is the timed workload: the weight-gradient kernels split
    K = batch x 4096 pixels, so each split there walks 8x more pixels and
    crosses 8x more image boundaries than at batch 2."""
    cfg = ResBlockConfig(batch=batch)
    print(f"[fullsize] C5 {cfg}", flush=True)
    x, noise, t, params = resblock_data(cfg, seed=4)
    m = Model("resblock", cfg.dims(t), reference_quirks=True)
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, x)
    m.input(1, noise)
    m.step(cfg.lr, STEP_ALL)
    m.sync()
    op, og, om, ov = oracle_tables(params)
    T = orc.ptr_table
    loss = orc.call("orc_c5_step", cfg.batch, cfg.cin, cfg.cout, cfg.h, cfg.w, cfg.groups, cfg.tdim, t, orc.ptr(x),
                    orc.ptr(noise), T(op), T(og), T(om), T(ov), 0.0, 1, 0)
    print(f"[fullsize] C5 loss {m.loss!r} oracle {loss!r}", flush=True)
    assert abs(m.loss - loss) <= 1e-5 * abs(loss), (m.loss, loss)
    for i in range(len(params)):
        got = m.get(i, 1)
        _report(f"C5 grad {m.names[i]}", got, og[i])
        assert_close(got, og[i], what=f"C5 grad {m.names[i]}", **GRAD)
    # the reference's Broadcast_Channel reduces only the first `width` channels
    # of the time-embedding gradient (64 of 128 here)
    assert np.all(m.get(7, 1)[cfg.w:] == 0)
    check_update(orc, m, params, cfg.lr, 1, True, "C5")
    m.close()


def test_c3_exact_shape_vs_oracle(hip, orc):
    """dX = dY W^T and dW = X^T dY with db fused, accumulating (beta 1) into
    nonzero destinations, through the same call as bench.py's C3 leg (the
    Linear backward entry point, whose weight gradient here runs as two K
    splits and a reduce), and through two plain GEMM calls."""
    cfg = GemmConfig()
    M, K, N = cfg.m, cfg.k, cfg.n
    print(f"[fullsize] C3 {M}x{K}x{N}", flush=True)
    X, W, dY = gemm_data(cfg, seed=1)
    r = np.random.default_rng(11)
    dX0 = r.standard_normal((M, K), dtype=np.float32)
    dW0 = r.standard_normal((K, N), dtype=np.float32)
    db0 = r.standard_normal(N, dtype=np.float32)
    gX, gW, gdY = H.Buffer.from_array(X), H.Buffer.from_array(W), H.Buffer.from_array(dY)
    gdX, gdW, gdb = H.Buffer.from_array(dX0), H.Buffer.from_array(dW0), H.Buffer.from_array(db0)
    need = H.lib().mle_linear_bwd_ws_bytes(M, K, N, 1)
    gws = H.Buffer(max(need, 256))
    H.call("mle_linear_bwd", None, M, K, N, 1, gX.ptr, gdY.ptr, 0, gW.ptr, 0, gdX.ptr, 1, gdW.ptr, gdb.ptr, 0, gws.ptr,
           need)
    dX, dW, db = gdX.numpy(), gdW.numpy(), gdb.numpy()
    # the two plain GEMM calls: the same dX bits (the same kernel), dW and db
    # from one unsplit pass
    gdX2, gdW2, gdb2 = H.Buffer.from_array(dX0), H.Buffer.from_array(dW0), H.Buffer.from_array(db0)
    H.call("mle_gemm", None, 0, 1, M, K, N, 1.0, gdY.ptr, N, 0, gW.ptr, N, 0, 1.0, gdX2.ptr, K, 0, 1, None)
    H.call("mle_gemm", None, 1, 0, K, N, M, 1.0, gX.ptr, K, 0, gdY.ptr, N, 0, 1.0, gdW2.ptr, N, 0, 1, gdb2.ptr)
    np.testing.assert_array_equal(gdX2.numpy(), dX)
    assert_close(gdW2.numpy(), dW, what="C3 dW, one pass against two splits", **GRAD)
    assert_close(gdb2.numpy(), db, what="C3 db, one pass against two splits", **GRAD)
    for b in (gdX2, gdW2, gdb2, gws):
        b.free()

    rows = np.sort(r.choice(M, 256, replace=False))
    cols = np.sort(r.choice(N, 256, replace=False))
    # dX rows: dX0[rows] + dY[rows] W^T  (bcmmABT, kind 1)
    want_dx = np.ascontiguousarray(dX0[rows])
    dYr = np.ascontiguousarray(dY[rows])
    orc.call("orc_bcmm", 1, orc.ptr(dYr), orc.ptr(W), orc.ptr(want_dx), 1, 1, 256, N, K, 1, 3, 0, 3, 1.0)
    # dW columns: dW0[:, cols] + X^T dY[:, cols]  (bcmmATB, kind 2)
    want_dw = np.ascontiguousarray(dW0[:, cols])
    dYc = np.ascontiguousarray(dY[:, cols])
    orc.call("orc_bcmm", 2, orc.ptr(X), orc.ptr(dYc), orc.ptr(want_dw), 1, 1, K, M, 256, 1, 3, 3, 0, 1.0)
    # db: db0 + column sums of dY  (BCompress)
    want_db = db0.copy()
    orc.call("orc_bcompress", orc.ptr(dY), orc.ptr(want_db), M, N, 1.0)
    for what, got, ref in (("dX rows", dX[rows], want_dx), ("dW cols", dW[:, cols], want_dw), ("db", db, want_db)):
        _report(f"C3 {what}", got, ref)
        assert_close(got, ref, what=f"C3 {what}", **GRAD)
    # rows and columns outside the sample moved too (the whole output was written)
    assert np.abs(dX - dX0).max(axis=1).min() > 0 and np.abs(dW - dW0).max(axis=0).min() > 0
    for b in (gX, gW, gdY, gdX, gdW, gdb):
        b.free()


def test_c2_full_size_vs_oracle(hip, orc):
    """10 steps of accumulate -> clipNorm -> AdamW over the 100 M-parameter
    arena.  The pristine gradient is restored before each step (the reference
    clips in place), on both sides."""
    cfg = FlatConfig()
    sizes, p, g = flat_data(cfg, seed=2)
    print(f"[fullsize] C2 {len(sizes)} tensors, {sum(sizes)} params, {cfg.steps} steps", flush=True)
    m = Model("flat", [len(sizes)] + sizes)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    for i in range(len(sizes)):
        m.set(i, p[offs[i]:offs[i + 1]], 0)
    ref_p = [p[offs[i]:offs[i + 1]].copy() for i in range(len(sizes))]
    ref_m = [np.zeros(s, np.float32) for s in sizes]
    ref_v = [np.zeros(s, np.float32) for s in sizes]
    chunks_g = [g[offs[i]:offs[i + 1]] for i in range(len(sizes))]
    norms = []
    for step in range(1, cfg.steps + 1):
        for i, c in enumerate(chunks_g):
            m.set(i, c, 1)
        m.step(cfg.lr, 8, cfg.max_norm)  # accumulate + clipNorm + ParameterUpdate
        acc = np.zeros(1, np.float64)
        for c in chunks_g:
            orc.call("orc_sumsq", orc.ptr(c), c.size, orc.ptr(acc))
        orc.call("orc_sqrt_scale", orc.ptr(acc), 1.0)
        norms.append(float(acc[0]))
        for i, c in enumerate(chunks_g):
            gc = c.copy()
            orc.call("orc_clip", orc.ptr(gc), gc.size, orc.ptr(acc))
            orc.call("orc_adam", orc.ptr(ref_p[i]), orc.ptr(gc), gc.size, step, orc.ptr(ref_m[i]), orc.ptr(ref_v[i]),
                     0.9, 0.999, 1e-8, 0.01, cfg.lr, 1)
    m.sync()
    assert norms[0] > 1.0, norms  # the clip triggers (||g|| is about 100)
    worst = 0.0
    for i in range(len(sizes)):
        got_p = m.get(i, 0)
        worst = max(worst, float(np.abs(got_p - ref_p[i]).max() / np.abs(ref_p[i]).max()))
        assert_close(m.get(i, 2), ref_m[i], what=f"C2 m {i}", **EW)
        assert_close(m.get(i, 3), ref_v[i], what=f"C2 v {i}", **EW)
        assert_close(got_p, ref_p[i], what=f"C2 p {i}", **EW)
        assert m.t(i) == cfg.steps + 1
    print(f"[fullsize] C2 norm {norms[0]:.6g}; p max|err| / max|ref| = {worst:.3g}", flush=True)
    m.close()

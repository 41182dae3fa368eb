"""End-to-end parity of the C++ engine (GraphOperations API over the HIP C ABI)
against the oracle's restatement of the same training step.

Per step: loss, every parameter gradient, and the AdamW/Adam update.  The
update is checked by applying the oracle's optimizer to the engine's own
gradients: at t = 1 the step is lr * g/(|g| + eps), so a gradient element whose
sign sits inside fp32 noise would flip a whole lr-sized step and hide what is
being tested (the fused update over the parameter arena).
"""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close
from ml_engine_amd.configs import (BlockConfig, FlatConfig, MLPConfig, ResBlockConfig, block_data, flat_data,
                                   mlp_data, resblock_data)
from ml_engine_amd.models import STEP_ALL, STEP_CLOBBER_SCALE, Model
from ml_engine_amd.models import lib as models_lib

pytestmark = pytest.mark.gpu

GRAD = dict(rtol=1e-4, atol_scale=1e-5)   # composed GEMM / conv gradients (as at full size)
EW = dict(rtol=1e-5, atol_scale=1e-6)


def check_update(orc, m, params0, lr, t, adamw, what):
    for i, p0 in enumerate(params0):
        g = m.get(i, 1)
        p = p0.reshape(-1).copy()
        mm = np.zeros_like(p)
        vv = np.zeros_like(p)
        orc.call("orc_adam", orc.ptr(p), orc.ptr(g), p.size, t, orc.ptr(mm), orc.ptr(vv), 0.9, 0.999, 1e-8, 0.01, lr,
                 int(adamw))
        assert_close(m.get(i, 2), mm, what=f"{what} m[{m.names[i]}]", **EW)
        assert_close(m.get(i, 3), vv, what=f"{what} v[{m.names[i]}]", **EW)
        assert_close(m.get(i, 0), p, what=f"{what} p[{m.names[i]}]", **EW)


def oracle_tables(params):
    op = [np.ascontiguousarray(p.reshape(-1)).copy() for p in params]
    og = [np.zeros_like(p) for p in op]
    om = [np.zeros_like(p) for p in op]
    ov = [np.zeros_like(p) for p in op]
    return op, og, om, ov


def test_mlp_step(hip, orc):
    cfg = MLPConfig()
    x, labels, params = mlp_data(cfg, seed=0)
    m = Model("mlp", cfg.dims())
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, x)
    m.input(1, labels)
    m.step(cfg.lr, STEP_ALL)
    m.sync()
    op, og, om, ov = oracle_tables(params)
    T = orc.ptr_table
    loss = orc.call("orc_c1_step", cfg.batch, cfg.inp, cfg.hidden, cfg.classes, orc.ptr(x), orc.ptr(labels), T(op),
                    T(og), T(om), T(ov), 0.0, 1, 0, None)
    assert abs(m.loss - loss) <= 1e-5 * abs(loss)
    for i in range(4):
        assert_close(m.get(i, 1), og[i], what=f"grad {m.names[i]}", **GRAD)
    check_update(orc, m, params, cfg.lr, 1, False, "mlp")
    assert all(m.t(i) == 2 for i in range(4))
    m.close()


@pytest.mark.parametrize("quirks", [True, False])
@pytest.mark.parametrize("dims", [(2, 32, 64, 4), (2, 128, 128, 2)], ids=["heads16", "heads64_fused_attention"])
def test_block_step(hip, orc, quirks, dims):
    """One step of the block against the oracle's composition.  With 64-wide
    heads and seq a multiple of 64 MultiHeadAttention runs the fused attention
    node; with 16-wide heads the stored-score chain."""
    batch, seq, d_model, heads = dims
    cfg = BlockConfig(batch=batch, seq=seq, d_model=d_model, heads=heads, ffn=128, vocab=97)
    ids, tgt, params = block_data(cfg, seed=3)
    m = Model("block", cfg.dims(), reference_quirks=quirks)
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, ids)
    m.input(1, tgt)
    m.step(cfg.lr, STEP_ALL)
    m.sync()
    op, og, om, ov = oracle_tables(params)
    T = orc.ptr_table
    loss = orc.call("orc_c4_step", cfg.batch, cfg.seq, cfg.d_model, cfg.heads, cfg.ffn, cfg.vocab, orc.ptr(ids),
                    orc.ptr(tgt), T(op), T(og), T(om), T(ov), 0.0, 1, int(not quirks))
    assert abs(m.loss - loss) <= 1e-5 * abs(loss), (m.loss, loss)
    for i in range(len(params)):
        # Parameters 1..14 are (W, b) pairs.  The query bias gradient is zero by
        # symmetry (a per-column shift of the scores does not change a
        # column-normalised softmax), so biases are judged on the scale of
        # their layer's weight gradient, which sums the same dY terms.
        s = max(np.abs(og[i]).max(), np.abs(og[i - 1]).max()) if i >= 2 and i % 2 == 0 else None
        assert_close(m.get(i, 1), og[i], what=f"grad {m.names[i]}", scale=s, **GRAD)
    check_update(orc, m, params, cfg.lr, 1, True, "block")
    m.close()


@pytest.mark.parametrize("quirks", [True, False])
def test_resblock_step(hip, orc, quirks):
    cfg = ResBlockConfig(batch=2, cin=8, cout=16, h=12, w=12, groups=4, tdim=32)
    x, noise, t, params = resblock_data(cfg, seed=4)
    m = Model("resblock", cfg.dims(t), reference_quirks=quirks)
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, x)
    m.input(1, noise)
    m.step(cfg.lr, STEP_ALL)
    m.sync()
    op, og, om, ov = oracle_tables(params)
    T = orc.ptr_table
    loss = orc.call("orc_c5_step", cfg.batch, cfg.cin, cfg.cout, cfg.h, cfg.w, cfg.groups, cfg.tdim, t, orc.ptr(x),
                    orc.ptr(noise), T(op), T(og), T(om), T(ov), 0.0, 1, int(not quirks))
    assert abs(m.loss - loss) <= 1e-5 * abs(loss), (m.loss, loss)
    for i in range(len(params)):
        assert_close(m.get(i, 1), og[i], what=f"grad {m.names[i]}", **GRAD)
    if quirks:  # only the first `width` channels of the time-embedding gradient are reduced
        assert np.all(m.get(7, 1)[cfg.w:] == 0)
    check_update(orc, m, params, cfg.lr, 1, True, "resblock")
    m.close()


def _flat_model(cfg, seed=2):
    sizes, p, g = flat_data(cfg, seed=seed)
    m = Model("flat", [len(sizes)] + sizes)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    chunks_p = [p[offs[i]:offs[i + 1]].copy() for i in range(len(sizes))]
    chunks_g = [g[offs[i]:offs[i + 1]].copy() for i in range(len(sizes))]
    for i in range(len(sizes)):
        m.set(i, chunks_p[i], 0)
        m.set(i, chunks_g[i], 1)
    return m, sizes, chunks_p, chunks_g


def _oracle_norm(orc, grads):
    acc = np.zeros(1, np.float64)
    for c in grads:
        orc.call("orc_sumsq", orc.ptr(c), c.size, orc.ptr(acc))
    orc.call("orc_sqrt_scale", orc.ptr(acc), 1.0)
    return acc


def test_flat_clip_adamw(hip, orc):
    """accumulate + clipNorm + ParameterUpdate, each step from the pristine
    gradients (restored on both sides: the reference clips them in place)."""
    cfg = FlatConfig(total=300_000, tensors=8, lo=4096, hi=80_000, steps=3)
    m, sizes, chunks_p, chunks_g = _flat_model(cfg)
    ref_p = [c.copy() for c in chunks_p]
    ref_m = [np.zeros_like(c) for c in chunks_p]
    ref_v = [np.zeros_like(c) for c in chunks_p]
    for step in range(1, cfg.steps + 1):
        for i, c in enumerate(chunks_g):
            m.set(i, c, 1)
        m.step(cfg.lr, 8, cfg.max_norm)  # accumulate + clipNorm + ParameterUpdate
        acc = _oracle_norm(orc, chunks_g)
        for i, c in enumerate(chunks_g):
            gc = c.copy()
            orc.call("orc_clip", orc.ptr(gc), gc.size, orc.ptr(acc))
            orc.call("orc_adam", orc.ptr(ref_p[i]), orc.ptr(gc), gc.size, step, orc.ptr(ref_m[i]), orc.ptr(ref_v[i]),
                     0.9, 0.999, 1e-8, 0.01, cfg.lr, 1)
    m.sync()
    for i in range(len(sizes)):
        assert_close(m.get(i, 2), ref_m[i], what=f"m {i}", **EW)
        assert_close(m.get(i, 3), ref_v[i], what=f"v {i}", **EW)
        assert_close(m.get(i, 0), ref_p[i], what=f"p {i}", **EW)
        assert m.t(i) == cfg.steps + 1
    m.close()


def test_clip_reads_as_reference(hip, orc):
    """The reference divides the parameter gradients in place at clipNorm
    (Engine/engine.cu:3362, 302).  Here the division is deferred into the
    update, yet every read sees the reference's values: after clipNorm alone,
    after the update, and through a second step that starts from the clipped
    gradients (its norm is taken over them).  The scale is the one clipNorm saw
    even if the caller overwrites its buffer before the update."""
    cfg = FlatConfig(total=200_000, tensors=5, lo=4096, hi=80_000)
    pending = models_lib().mle_model_clip_pending
    # between clipNorm and the update
    m, sizes, _, chunks_g = _flat_model(cfg)
    m.step(cfg.lr, 0, cfg.max_norm)  # accumulate + clipNorm, no update
    assert pending() == len(sizes)
    acc = _oracle_norm(orc, chunks_g)
    assert acc[0] > 1.0
    clipped = [c.copy() for c in chunks_g]
    for c in clipped:
        orc.call("orc_clip", orc.ptr(c), c.size, orc.ptr(acc))
    for i in range(len(sizes)):
        assert_close(m.get(i, 1), clipped[i], what=f"grad after clipNorm {i}", **EW)
    # Regression: the pending-clip set holds parameters by address.  A model
    # closed with its parameters still marked (as after every clipped update)
    # once left dangling entries there, and the next model's accumulate walked
    # them (a host abort).  A destroyed parameter now leaves the set.
    m.step(cfg.lr, 0, cfg.max_norm)
    assert pending() == len(sizes)
    m.close()
    assert pending() == 0
    # two full steps without restoring the gradients, and the same with the
    # scale buffer overwritten between clipNorm and the update
    results = []
    for mode in (8, 8 | STEP_CLOBBER_SCALE):
        m, sizes, chunks_p, chunks_g = _flat_model(cfg)
        ref_p = [c.copy() for c in chunks_p]
        ref_m = [np.zeros_like(c) for c in chunks_p]
        ref_v = [np.zeros_like(c) for c in chunks_p]
        ref_g = [c.copy() for c in chunks_g]
        for step in (1, 2):
            m.step(cfg.lr, mode, cfg.max_norm)
            acc = _oracle_norm(orc, ref_g)  # over the gradients as the reference left them
            for i, gr in enumerate(ref_g):
                orc.call("orc_clip", orc.ptr(gr), gr.size, orc.ptr(acc))  # in place, as ScalePtr
                orc.call("orc_adam", orc.ptr(ref_p[i]), orc.ptr(gr), gr.size, step, orc.ptr(ref_m[i]),
                         orc.ptr(ref_v[i]), 0.9, 0.999, 1e-8, 0.01, cfg.lr, 1)
            # reading applies the pending division in place; without the read
            # (first mode, first step) the next accumulate applies it
            if step == 2 or mode & STEP_CLOBBER_SCALE:
                for i in range(len(sizes)):
                    assert_close(m.get(i, 1), ref_g[i], what=f"mode {mode} step {step} grad {i}", **EW)
        got = [(m.get(i, 0), m.get(i, 2), m.get(i, 3)) for i in range(len(sizes))]
        for i, (p, mm, vv) in enumerate(got):
            assert_close(mm, ref_m[i], what=f"mode {mode} m {i}", **EW)
            assert_close(vv, ref_v[i], what=f"mode {mode} v {i}", **EW)
            assert_close(p, ref_p[i], what=f"mode {mode} p {i}", **EW)
        results.append(got)
        m.close()
        assert pending() == 0
    for a, b in zip(results[0], results[1]):
        for u, v in zip(a, b):
            np.testing.assert_array_equal(u, v)


@pytest.mark.parametrize("reference_layout", [True, False])
def test_layernorm_multichannel_quirk(hip, orc, reference_layout):
    """LayerNorm over a [C > 1, H, W] sample: the reference's LayerBackward
    gives a gradient to the first batch*H*W elements only (its C == 1 guard,
    Engine/kernels.cu:849-862); mle::Quirks::layernorm_reference_layout keeps
    that (default) or applies the per-sample formula everywhere.  Checked
    through a 1x1 convolution's weight and bias gradients against the oracle."""
    N, Cin, Cc, Hh, Ww = 2, 3, 4, 5, 6
    r = np.random.default_rng(77)
    x = r.standard_normal((N, Cin, Hh, Ww), dtype=np.float32)
    target = r.standard_normal((N, Cc, Hh, Ww), dtype=np.float32)
    W = (r.standard_normal((Cc, Cin, 1, 1)) * 0.5).astype(np.float32)
    b = (r.standard_normal(Cc) * 0.1).astype(np.float32)
    m = Model("conv_layernorm", [N, Cin, Cc, Hh, Ww], layernorm_reference_layout=reference_layout)
    m.set(0, W)
    m.set(1, b)
    m.input(0, x)
    m.input(1, target)
    m.step(0.0, 7)  # zero_grad + forward + backward
    m.sync()
    P = orc.ptr
    y = np.zeros((N, Cc, Hh, Ww), np.float32)
    orc.call("orc_conv_fwd", P(x), P(W), P(b), P(y), N, Cin, Hh, Ww, Cc, 1, 1, 0, 1)
    yn, st = np.zeros_like(y), np.zeros(2 * N, np.float32)
    orc.call("orc_norm_fwd", P(y), P(yn), P(st), N, Cc, Hh * Ww, 1, 1e-5)
    loss = orc.call("orc_mse_loss", P(yn), P(target), yn.size)
    dyn, dy = np.zeros_like(y), np.zeros_like(y)
    orc.call("orc_mse_bwd", P(yn), P(target), None, P(dyn), yn.size)
    orc.call("orc_norm_bwd", P(yn), P(dyn), P(dy), P(st), N, Cc, Hh * Ww, 1, 1e-5, int(reference_layout))
    dW = np.zeros_like(W)
    orc.call("orc_conv_wgrad", P(x), P(dy), P(dW), N, Cin, Hh, Ww, Cc, 1, 1, 0, 1)
    db = dy.astype(np.float64).sum(axis=(0, 2, 3))
    assert abs(m.loss - loss) <= 1e-5 * abs(loss)
    assert_close(m.get(0, 1), dW.reshape(-1), what="conv weight grad", **GRAD)
    assert_close(m.get(1, 1), db, what="conv bias grad", rtol=1e-4, atol_scale=1e-4,
                 scale=float(np.abs(dy).max() * N * Hh * Ww))
    if reference_layout:  # the guard leaves everything past the first N*H*W elements without gradient
        assert np.all(dy.reshape(-1)[N * Hh * Ww:] == 0)
    m.close()


def _probe_step(hip, m, lr, fam):
    """One full step with the launch probe armed for one GEMM family; returns
    the number of launches of that family."""
    n, ms, fl, by = C.c_int(0), C.c_double(0), C.c_double(0), C.c_double(0)
    hip.call("mle_probe_arm", fam.encode())
    m.step(lr, STEP_ALL)
    m.sync()
    hip.call("mle_probe_read", C.byref(n), C.byref(ms), C.byref(fl), C.byref(by))
    hip.call("mle_probe_arm", None)
    return n.value


@pytest.mark.parametrize("quirks", [True, False])
def test_block_qkv_fusion(hip, quirks):
    """Fused Q/K/V projections (one batched forward, one batched dW + db, one
    grouped sum-of-products dX) agree with one GEMM per projection and remove
    exactly two NN launches and four backward products (NT and TN launches,
    and the Linear pairs that hold one of each: at this size every unfused
    projection's dX and dW share a launch)."""
    cfg = BlockConfig(batch=4, seq=64, d_model=128, heads=4, ffn=256, vocab=300)
    ids, tgt, params = block_data(cfg, seed=5)
    runs = {}
    for fuse in (True, False):
        m = Model("block", cfg.dims(), reference_quirks=quirks, fuse=fuse)
        for i, p in enumerate(params):
            m.set(i, p)
        m.input(0, ids)
        m.input(1, tgt)
        counts = {}
        for fam in ("gemm_nn", "gemm_nt", "gemm_tn", "gemm_pair"):
            for i, p in enumerate(params):  # same starting point for every probed step
                m.set(i, p)
                m.set(i, np.zeros_like(p), 2)
                m.set(i, np.zeros_like(p), 3)
            counts[fam] = _probe_step(hip, m, cfg.lr, fam)
        runs[fuse] = (counts, m.loss, [m.get(i, 1) for i in range(len(params))])
        m.close()
    (cf, lf, gf), (cu, lu, gu) = runs[True], runs[False]
    assert cu["gemm_nn"] - cf["gemm_nn"] == 2, (cu, cf)
    products = {k: c["gemm_nt"] + c["gemm_tn"] + 2 * c["gemm_pair"] for k, c in (("u", cu), ("f", cf))}
    assert products["u"] - products["f"] == 4, (cu, cf)
    assert abs(lf - lu) <= 1e-5 * abs(lu)
    for i in range(len(params)):
        # Biases are judged on the scale of their layer's weight gradient (the
        # query bias gradient is zero up to rounding by symmetry).
        scale = float(np.abs(gu[i]).max())
        if i >= 2 and i % 2 == 0:
            scale = max(scale, float(np.abs(gu[i - 1]).max()))
        assert np.abs(gf[i] - gu[i]).max() <= 1e-4 * scale, (i, np.abs(gf[i] - gu[i]).max(), scale)


def _state(m, n):
    return [[m.get(i, w) for i in range(n)] for w in range(4)]  # params, grads, m, v


@pytest.mark.parametrize("kind", ["mlp", "block", "resblock"])
def test_step_graph_matches_eager(hip, kind):
    """Replays of the recorded zero_grad / forward / backward pass (the update
    launched from the host) give, step after step, the bits of eager steps:
    loss, parameters, gradients and Adam moments -- with the program's own
    work and synchronisations between the replays (host reads of every
    tensor), and again after a mode change (forward + backward without
    zero_grad, recorded anew)."""
    from ml_engine_amd.models import STEP_BACKWARD, STEP_FORWARD
    if kind == "mlp":
        cfg = MLPConfig()
        x, labels, params = mlp_data(cfg, seed=7)
        dims, inputs = cfg.dims(), [x, labels]
    elif kind == "block":
        cfg = BlockConfig(batch=2, seq=64, d_model=64, heads=1, ffn=128, vocab=97)
        ids, tgt, params = block_data(cfg, seed=7)
        dims, inputs = cfg.dims(), [ids, tgt]
    else:
        cfg = ResBlockConfig(batch=2, cin=8, cout=16, h=12, w=12, groups=4, tdim=32)
        x, noise, t, params = resblock_data(cfg, seed=7)
        dims, inputs = cfg.dims(t), [x, noise]
    models = []
    for _ in range(2):
        m = Model(kind, dims)
        for i, p in enumerate(params):
            m.set(i, p)
        for slot, a in enumerate(inputs):
            m.input(slot, a)
        models.append(m)
    eager, graph = models
    n = len(params)
    for step, mode in enumerate([STEP_ALL] * 4 + [STEP_FORWARD | STEP_BACKWARD] * 2 + [STEP_ALL]):
        eager.step(cfg.lr, mode)
        eager.sync()
        le = eager.loss
        graph.step_graph(cfg.lr, mode)
        lg = graph.loss
        assert lg == le, (step, lg, le)
        for w, (a, b) in enumerate(zip(_state(eager, n), _state(graph, n))):
            for i in range(n):
                np.testing.assert_array_equal(b[i].view(np.uint32), a[i].view(np.uint32),
                                              err_msg=f"step {step} tensor {w}/{i}")
    for m in models:
        m.close()


def test_graph_loss_is_the_models_own(hip):
    """A replayed pass publishes its loss into the device's shared read-back
    slot; another model's step (or any scalar read) publishes there too.  The
    replayed model's loss is still its own: read from the slot only while the
    slot holds this graph's sequence number, else from the loss node."""
    cfg = MLPConfig()
    x, labels, params = mlp_data(cfg, seed=7)
    x2, labels2, params2 = mlp_data(cfg, seed=8)

    def make(p, xx, ll):
        m = Model("mlp", cfg.dims())
        for i, a in enumerate(p):
            m.set(i, a)
        m.input(0, xx)
        m.input(1, ll)
        return m

    a, a_eager, b = make(params, x, labels), make(params, x, labels), make(params2, x2, labels2)
    for step in range(3):
        a_eager.step(cfg.lr, STEP_ALL)
        la = a_eager.loss
        a.step_graph(cfg.lr, STEP_ALL)
        if step == 0:
            assert a.loss == la  # nothing published after the replay: the slot's value
            continue
        b.step(cfg.lr, STEP_ALL)  # publishes b's loss after a's
        lb = b.loss
        assert lb != la
        assert a.loss == la, (step, a.loss, la, lb)
        assert b.loss == lb
    # two replayed models, read in the opposite order
    b.step_graph(cfg.lr, STEP_ALL)
    a.step_graph(cfg.lr, STEP_ALL)
    a_eager.step(cfg.lr, STEP_ALL)
    la = a_eager.loss
    lb = b.loss
    assert a.loss == la
    assert lb != la
    for m in (a, a_eager, b):
        m.close()


def test_resblock_fusion_matches_unfused(hip):
    """C5 residual block with the graph fusions (GroupNorm -> SiLU in one pass
    each way) against one kernel per op: the same loss, parameter gradients
    and, through the backward hand-off, the same bits, over a step with an
    update and a backward without zero_grad."""
    from ml_engine_amd.models import STEP_BACKWARD, STEP_FORWARD
    cfg = ResBlockConfig(batch=2, cin=8, cout=16, h=12, w=12, groups=4, tdim=32)
    x, noise, t, params = resblock_data(cfg, seed=9)
    runs = {}
    for fuse in (True, False):
        m = Model("resblock", cfg.dims(t), fuse=fuse)
        for i, p in enumerate(params):
            m.set(i, p)
        m.input(0, x)
        m.input(1, noise)
        m.step(cfg.lr, STEP_ALL)
        m.sync()
        # every node's output and gradient after the first step: the fused
        # run defers or skips some writes (the activation before the loss is
        # recomputed when read) and must read back the same values
        nodes = [(m.node(i, 0), m.node(i, 1)) for i in range(m.nodes())]
        first_loss = m.loss
        m.step(cfg.lr, STEP_FORWARD | STEP_BACKWARD)  # adds into the gradients
        m.sync()
        runs[fuse] = (m.loss, [m.get(i, 1) for i in range(len(params))], [m.get(i, 0) for i in range(len(params))],
                      nodes, first_loss)
        m.close()
    (lf, gf, pf, nf, f1), (lu, gu, pu, nu, u1) = runs[True], runs[False]
    assert lf == lu and f1 == u1
    assert len(nf) == len(nu)
    # Node buffers within 1e-6 of their scale, not bit for bit: the block
    # input's gradient is summed over conv1's and the 1x1 skip's products in
    # one paired launch when fused, in two passes when not (1-ulp apart).
    for i, ((of, df), (ou, du)) in enumerate(zip(nf, nu)):
        for got, want, what in ((of, ou, "output"), (df, du, "gradient")):
            assert (got is None) == (want is None), (i, what)
            if got is not None:
                scale = float(np.abs(want).max()) if want.size else 0.0
                np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * scale, err_msg=f"node {i} {what}")
    for i in range(len(params)):
        np.testing.assert_array_equal(gf[i].view(np.uint32), gu[i].view(np.uint32), err_msg=f"grad {i}")
        np.testing.assert_array_equal(pf[i].view(np.uint32), pu[i].view(np.uint32), err_msg=f"param {i}")


def test_mlp_fusion_matches_unfused(hip):
    """C1 MLP with the graph fusions (the classifier head's Linear and
    cross-entropy in one launch, the ReLU backward in the classifier's
    backward launch) against one kernel per op: the first step's gradients,
    and the losses of three steps, to rounding (the fused head adds the
    logits' products in its own order)."""
    cfg = MLPConfig()
    x, labels, params = mlp_data(cfg, seed=21)
    runs = {}
    for fuse in (True, False):
        m = Model("mlp", cfg.dims(), fuse=fuse)
        for i, p in enumerate(params):
            m.set(i, p)
        m.input(0, x)
        m.input(1, labels)
        m.step(cfg.lr, STEP_ALL)
        m.sync()
        grads = [m.get(i, 1) for i in range(len(params))]
        losses = [m.loss]
        for _ in range(2):
            m.step(cfg.lr, STEP_ALL)
            losses.append(m.loss)
        m.sync()
        runs[fuse] = (losses, grads)
        m.close()
    (lf, gf), (lu, gu) = runs[True], runs[False]
    for a, b in zip(lf, lu):
        assert abs(a - b) <= 1e-6 * abs(b), (lf, lu)
    for i in range(len(params)):
        assert_close(gf[i], gu[i], what=f"C1 grad {i}, fused against unfused", **GRAD)


@pytest.mark.parametrize("kind", ["mlp", "block"])
@pytest.mark.parametrize("graphed", [False, True])
def test_onehot_target_lazy(hip, kind, graphed):
    """The one-hot target, whose only consumer (cross-entropy against key
    targets) reads the ids, is not updated by the forward; a read brings it up
    to date: after several steps, targets changed between steps, eager and
    graph-replayed, the matrix read is the one-hot of the current targets."""
    if kind == "mlp":
        cfg = MLPConfig()
        x, labels, params = mlp_data(cfg, seed=11)
        dims, inputs, rows, cols = cfg.dims(), [x, labels], cfg.batch, cfg.classes
    else:
        cfg = BlockConfig(batch=2, seq=64, d_model=64, heads=1, ffn=128, vocab=97)
        x, labels, params = block_data(cfg, seed=11)
        dims, inputs, rows, cols = cfg.dims(), [x, labels], cfg.batch * cfg.seq, cfg.vocab
    m = Model(kind, dims)
    for i, p in enumerate(params):
        m.set(i, p)
    for slot, a in enumerate(inputs):
        m.input(slot, a)
    r = np.random.default_rng(3)
    tgt = np.asarray(labels).astype(np.int32)
    for step in range(4):
        if step == 2:  # new targets, then two more steps before the read
            tgt = r.integers(0, cols, tgt.shape).astype(np.int32)
            m.input(1, tgt)
        if graphed:
            m.step_graph(cfg.lr, STEP_ALL)
        else:
            m.step(cfg.lr, STEP_ALL)
        m.sync()
        if step in (0, 3):
            want = np.zeros((rows, cols), np.float32)
            want[np.arange(rows), tgt.reshape(-1)] = 1.0
            got = m.target(rows * cols).reshape(rows, cols)
            np.testing.assert_array_equal(got, want, err_msg=f"step {step}")
    m.close()


def test_block_fusion_full_size(hip):
    """Full C4 shape, where the graph fusions run on the persistent GEMM kernel
    (LM-head row statistics for the loss, batched Q/K/V): one step agrees with
    the unfused graph (one GEMM per layer, a loss that reads the logits) --
    loss within 1e-5, every parameter gradient within 1e-4 of its scale."""
    cfg = BlockConfig()
    ids, tgt, params = block_data(cfg, seed=3)
    runs = {}
    for fuse in (True, False):
        m = Model("block", cfg.dims(), fuse=fuse)
        for i, p in enumerate(params):
            m.set(i, p)
        m.input(0, ids)
        m.input(1, tgt)
        m.step(0.0, 7)  # zero_grad + forward + backward
        m.sync()
        runs[fuse] = (m.loss, [m.get(i, 1) for i in range(len(params))])
        m.close()
    (lf, gf), (lu, gu) = runs[True], runs[False]
    assert abs(lf - lu) <= 1e-5 * abs(lu), (lf, lu)
    for i in range(len(params)):
        scale = float(np.abs(gu[i]).max())
        if i >= 2 and i % 2 == 0:
            scale = max(scale, float(np.abs(gu[i - 1]).max()))
        assert np.abs(gf[i] - gu[i]).max() <= 1e-4 * scale, (i, np.abs(gf[i] - gu[i]).max(), scale)


def test_block_full_size_properties(hip):
    """Full C4 shape: one step runs, the loss is near ln(V) for random init, every
    gradient is finite, and a second step reproduces the first bit for bit when
    the parameters are restored (deterministic reductions, no atomics)."""
    cfg = BlockConfig()
    ids, tgt, params = block_data(cfg, seed=3)
    m = Model("block", cfg.dims())
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, ids)
    m.input(1, tgt)
    m.step(0.0, 7)  # zero_grad + forward + backward
    m.sync()
    loss1 = m.loss
    g1 = [m.get(i, 1) for i in range(len(params))]
    assert abs(loss1 * cfg.vocab - np.log(cfg.vocab)) < 0.5  # loss is sum(-t log p) / (rows * V)
    for g in g1:
        assert np.all(np.isfinite(g))
    m.step(0.0, 7)
    m.sync()
    assert m.loss == loss1
    for i in range(len(params)):
        np.testing.assert_array_equal(m.get(i, 1), g1[i])
    m.close()


# --------------------------------------------- engine against golden fixtures
def _engine_grads(kind, dims, params, inputs, lr):
    m = Model(kind, dims, reference_quirks=False)
    for i, p in enumerate(params):
        m.set(i, p)
    for slot, x in enumerate(inputs):
        m.input(slot, x)
    m.step(lr, STEP_ALL)
    m.sync()
    out = [m.get(i, 1) for i in range(len(params))], m.loss
    m.close()
    return out


def test_golden_c1_engine(hip):
    from golden import make_golden as G
    from test_golden import grads, load

    (x, labels, params), d = G.inputs_c1()
    fx = load("c1_mlp_step.npz", d)
    got, loss = _engine_grads("mlp", G.C1.dims(), params, [x, labels], G.C1.lr)
    assert abs(loss - float(fx["loss"])) <= 1e-5 * abs(float(fx["loss"]))
    for i, (a, b) in enumerate(zip(got, grads(fx))):
        assert_close(a, b, what=f"golden c1 grad {i}", **GRAD)


def test_golden_c4_engine(hip):
    from golden import make_golden as G
    from test_golden import bias_scale, grads, load

    (ids, tgt, params), d = G.inputs_c4()
    fx = load("c4_block_step.npz", d)
    got, loss = _engine_grads("block", G.C4.dims(), params, [ids, tgt], G.C4.lr)
    assert abs(loss - float(fx["loss"])) <= 1e-5 * abs(float(fx["loss"]))
    ref = grads(fx)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert_close(a, b, what=f"golden c4 grad {i}", scale=bias_scale(ref, i), **GRAD)


def test_golden_c5_engine(hip):
    from golden import make_golden as G
    from test_golden import grads, load

    (x, noise, t, params), d = G.inputs_c5()
    fx = load("c5_resblock_step.npz", d)
    got, loss = _engine_grads("resblock", G.C5.dims(t), params, [x, noise], G.C5.lr)
    assert abs(loss - float(fx["loss"])) <= 1e-5 * abs(float(fx["loss"]))
    for i, (a, b) in enumerate(zip(got, grads(fx))):
        assert_close(a, b, what=f"golden c5 grad {i}", **GRAD)


# ------------------------------------ lazy gradient clearing is invisible
def _run_sequence(kind, dims, params, inputs, lr, lazy):
    """zero+fwd+bwd, then fwd+bwd again without zero_grad (the reference keeps
    adding into node and parameter gradients), then a full step with update."""
    from ml_engine_amd.models import STEP_BACKWARD, STEP_FORWARD, STEP_ZERO
    m = Model(kind, dims, reference_quirks=True, lazy_zero=lazy)
    for i, p in enumerate(params):
        m.set(i, p)
    for slot, x in enumerate(inputs):
        m.input(slot, x)
    out = []
    m.step(lr, STEP_ZERO | STEP_FORWARD | STEP_BACKWARD)
    m.sync()
    out.append([m.get(i, 1) for i in range(len(params))])
    m.step(lr, STEP_FORWARD | STEP_BACKWARD)
    m.sync()
    out.append([m.get(i, 1) for i in range(len(params))])
    m.step(lr, STEP_ALL)
    m.step(lr, STEP_ALL)
    m.sync()
    out.append([m.get(i, 0) for i in range(len(params))])
    m.close()
    return out


@pytest.mark.parametrize("kind", ["block", "resblock", "mlp"])
def test_lazy_zero_matches_eager(hip, kind):
    """Lazy clearing of node and parameter gradients (the first writer assigns:
    GEMM dW / column sums, conv bias sums, the embedding scatter) gives the bits
    of filling and adding, through accumulation without zero_grad and updates."""
    if kind == "mlp":
        cfg = MLPConfig()
        x, labels, params = mlp_data(cfg, seed=5)
        dims, inputs = cfg.dims(), [x, labels]
    elif kind == "block":
        cfg = BlockConfig(batch=2, seq=32, d_model=64, heads=4, ffn=128, vocab=97)
        ids, tgt, params = block_data(cfg, seed=3)
        dims, inputs = cfg.dims(), [ids, tgt]
    else:
        cfg = ResBlockConfig(batch=2, cin=8, cout=16, h=12, w=12, groups=4, tdim=32)
        x, noise, t, params = resblock_data(cfg, seed=4)
        dims, inputs = cfg.dims(t), [x, noise]
    lazy = _run_sequence(kind, dims, params, inputs, cfg.lr, True)
    eager = _run_sequence(kind, dims, params, inputs, cfg.lr, False)
    for phase, (a, b) in enumerate(zip(lazy, eager)):
        for i, (u, v) in enumerate(zip(a, b)):
            assert np.array_equal(u, v), f"{kind}: phase {phase} tensor {i} differs between lazy and eager clearing"
    # the second backward without zero_grad really accumulated
    assert not np.array_equal(lazy[0][-1], lazy[1][-1])


@pytest.mark.parametrize("kind", ["block", "resblock"])
def test_node_grads_match_eager(hip, kind):
    """Every node's gradient and output, read the way ReadValueAt reads them,
    equals the eager-clearing run's bits after a step and after a second
    backward without zero_grad.  With lazy clearing a pass-through backward
    (Add, Broadcast_Channel) leaves its input's gradient as an alias of its
    own, and the shared pair backward of the residual block's two
    convolutions writes the input gradient once: the reads here copy the
    aliases over and must see the reference's values."""
    from ml_engine_amd.models import STEP_BACKWARD, STEP_FORWARD, STEP_ZERO
    if kind == "block":
        cfg = BlockConfig(batch=2, seq=32, d_model=64, heads=4, ffn=128, vocab=97)
        ids, tgt, params = block_data(cfg, seed=3)
        dims, inputs = cfg.dims(), [ids, tgt]
    else:
        cfg = ResBlockConfig(batch=2, cin=8, cout=16, h=12, w=12, groups=4, tdim=32)
        x, noise, t, params = resblock_data(cfg, seed=4)
        dims, inputs = cfg.dims(t), [x, noise]
    runs = []
    for lazy in (True, False):
        m = Model(kind, dims, reference_quirks=True, lazy_zero=lazy)
        for i, p in enumerate(params):
            m.set(i, p)
        for slot, a in enumerate(inputs):
            m.input(slot, a)
        snaps = []
        for mode in (STEP_ZERO | STEP_FORWARD | STEP_BACKWARD, STEP_FORWARD | STEP_BACKWARD):
            m.step(cfg.lr, mode)
            m.sync()
            snaps.append([(m.node(i, 0), m.node(i, 1)) for i in range(m.nodes())])
        runs.append(snaps)
        m.close()
    (lazy_run, eager_run) = runs
    for phase, (a, b) in enumerate(zip(lazy_run, eager_run)):
        assert len(a) == len(b)
        for i, ((ao, ag), (bo, bg)) in enumerate(zip(a, b)):
            for what, u, v in (("output", ao, bo), ("grad", ag, bg)):
                assert (u is None) == (v is None), (kind, phase, i, what)
                if u is not None:  # equal values (an assigned -0 reads as 0 + -0 = 0 when added)
                    np.testing.assert_array_equal(u, v, err_msg=f"{kind}: phase {phase} node {i} {what}")


def test_early_loss_gradient_reads_as_reference(hip):
    """The last MSE node's forward writes its prediction's gradient in the
    same pass as the loss, held until its backward commits it.  Between
    forward and backward every node gradient still reads 0, as after the
    reference's zero_grad + forward; a read there drops the early gradient
    and the backward computes it as usual.  Both orders, and eager clearing,
    end with the same node gradients."""
    from ml_engine_amd.models import STEP_BACKWARD, STEP_FORWARD, STEP_ZERO
    cfg = ResBlockConfig(batch=2, cin=8, cout=16, h=12, w=12, groups=4, tdim=32)
    x, noise, t, params = resblock_data(cfg, seed=4)

    def make(lazy):
        m = Model("resblock", cfg.dims(t), reference_quirks=True, lazy_zero=lazy)
        for i, p in enumerate(params):
            m.set(i, p)
        m.input(0, x)
        m.input(1, noise)
        return m

    runs = []
    for lazy, read_between in ((True, True), (True, False), (False, False)):
        m = make(lazy)
        m.step(cfg.lr, STEP_ZERO | STEP_FORWARD)
        if read_between:
            for i in range(m.nodes()):
                g = m.node(i, 1)
                if g is not None:
                    assert not np.any(g), f"node {i} gradient before backward"
        m.step(cfg.lr, STEP_BACKWARD)
        m.sync()
        runs.append(([m.node(i, 1) for i in range(m.nodes())], [m.get(i, 1) for i in range(len(params))], m.loss))
        m.close()
    base = runs[2]
    for grads, pgrads, loss in runs[:2]:
        assert loss == base[2]
        for i, (u, v) in enumerate(zip(grads, base[0])):
            if u is not None:
                np.testing.assert_array_equal(u, v, err_msg=f"node {i}")
        for i, (u, v) in enumerate(zip(pgrads, base[1])):
            np.testing.assert_array_equal(u, v, err_msg=f"param {i}")


def unet_up_oracle(orc, x, skip, target, W, b, k, stride, pad):
    """Oracle composition of the harness's U-Net decoder step: forward chain,
    MSE loss, backward chain; returns (loss, dW, db)."""
    N, Cin, H, Wd = x.shape
    Cout = W.shape[0]
    Cs, Hs, Ws = skip.shape[1:]
    Ho, Wo = (H - 1) * stride - 2 * pad + k, (Wd - 1) * stride - 2 * pad + k
    C = Cs + Cout
    P = orc.ptr
    up = np.zeros((N, Cout, Ho, Wo), np.float32)
    orc.call("orc_convT_fwd", P(x), P(W), P(b), P(up), N, Cin, H, Wd, Cout, k, k, pad, stride)
    cat = np.zeros((N, C, Ho, Wo), np.float32)
    orc.call("orc_copy_crop_fwd", P(skip), P(up), P(cat), N, Cs, Hs, Ws, Cout, Ho, Wo)
    bn, st_bn = np.zeros_like(cat), np.zeros(2 * C, np.float32)
    orc.call("orc_batchnorm_fwd", P(cat), P(bn), P(st_bn), N, C, Ho * Wo, 1e-5)
    r0, n0 = np.zeros_like(cat), np.zeros(N * C * Ho, np.float32)
    orc.call("orc_rmsnorm_fwd", P(bn), P(r0), P(n0), N * C, Ho, Wo, 0)
    inn, st_in = np.zeros_like(cat), np.zeros(2 * N * C, np.float32)
    orc.call("orc_norm_fwd", P(r0), P(inn), P(st_in), N, C, Ho * Wo, C, 1e-5)
    r1, n1 = np.zeros_like(cat), np.zeros(N * C * Wo, np.float32)
    orc.call("orc_rmsnorm_fwd", P(inn), P(r1), P(n1), N * C, Ho, Wo, 1)
    loss = orc.call("orc_mse_loss", P(r1), P(target), r1.size)
    d = np.zeros_like(cat)
    orc.call("orc_mse_bwd", P(r1), P(target), None, P(d), d.size)
    d_inn = np.zeros_like(cat)
    orc.call("orc_rmsnorm_bwd", P(r1), P(d), P(n1), P(d_inn), N * C, Ho, Wo, 1)
    d_r0 = np.zeros_like(cat)
    orc.call("orc_norm_bwd", P(inn), P(d_inn), P(d_r0), P(st_in), N, C, Ho * Wo, C, 1e-5, 1)
    d_bn = np.zeros_like(cat)
    orc.call("orc_rmsnorm_bwd", P(r0), P(d_r0), P(n0), P(d_bn), N * C, Ho, Wo, 0)
    d_cat = np.zeros_like(cat)
    orc.call("orc_batchnorm_bwd", P(bn), P(d_bn), P(d_cat), P(st_bn), N, C, Ho * Wo, 1e-5)
    d_skip, d_up = np.zeros_like(skip), np.zeros_like(up)
    orc.call("orc_copy_crop_bwd", P(d_cat), P(d_skip), P(d_up), N, Cs, Hs, Ws, Cout, Ho, Wo)
    dW = np.zeros_like(W)
    orc.call("orc_convT_wgrad", P(x), P(d_up), P(dW), N, Cin, H, Wd, Cout, k, k, pad, stride)
    db = d_up.astype(np.float64).sum(axis=(0, 2, 3))
    return loss, dW, db, np.abs(d_up).max() * d_up[:, 0].size


@pytest.mark.parametrize("N,Cin,Cout,H,Cs,Hs,k,stride,pad", [(2, 8, 6, 8, 4, 20, 2, 2, 0), (2, 5, 3, 9, 2, 9, 3, 1, 1),
                                                            (4, 32, 16, 16, 16, 36, 4, 2, 1)])
def test_unet_up_step(hip, orc, N, Cin, Cout, H, Cs, Hs, k, stride, pad):
    """Convolute2DT, CopyCrop, BatchNorm, RMSNorm (both axes) and InstanceNorm
    composed through the C++ API: loss, weight and bias gradients against the
    oracle composition, then the AdamW update."""
    r = np.random.default_rng(N * 100 + Cin + k)
    Ho = (H - 1) * stride - 2 * pad + k
    x = r.standard_normal((N, Cin, H, H), dtype=np.float32)
    skip = r.standard_normal((N, Cs, Hs, Hs), dtype=np.float32)
    target = r.standard_normal((N, Cs + Cout, Ho, Ho), dtype=np.float32)
    W = (r.standard_normal((Cout, Cin, k, k)) * 0.2).astype(np.float32)
    b = (r.standard_normal(Cout) * 0.1).astype(np.float32)
    m = Model("unet_up", [N, Cin, Cout, H, H, Cs, Hs, Hs, k, stride, pad])
    m.set(0, W)
    m.set(1, b)
    m.input(0, x)
    m.input(1, skip)
    m.input(2, target)
    lr = 1e-3
    m.step(lr, STEP_ALL)
    m.sync()
    loss, dW, db, db_scale = unet_up_oracle(orc, x, skip, target, W, b, k, stride, pad)
    assert abs(m.loss - loss) <= 1e-5 * abs(loss), (m.loss, loss)
    assert_close(m.get(0, 1), dW.reshape(-1), what="convT weight grad", **GRAD)
    # the bias gradient is a sum of terms that nearly cancel (BatchNorm removes
    # the channel mean): scale its floor by the size of the summed terms
    assert_close(m.get(1, 1), db, what="convT bias grad", rtol=1e-4, atol_scale=1e-4, scale=db_scale)
    check_update(orc, m, [W, b], lr, 1, True, "unet_up")
    m.close()

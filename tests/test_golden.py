"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from float64 torch autograd models) against the CPU
oracle in its exact modes.  Runs without torch: the fixtures carry the
expected loss and gradients, and a SHA-256 of the regenerated inputs."""
import numpy as np
import pytest

from conftest import assert_close
from golden import make_golden as G

GRAD = dict(rtol=1e-4, atol_scale=1e-4)


def load(name: str, digest: str) -> dict:
    with np.load(G.HERE / name, allow_pickle=False) as z:
        fx = {k: z[k] for k in z.files}
    assert str(fx["inputs_sha256"]) == digest, f"{name}: the seeded input generator changed; rerun make_golden.py"
    return fx


def grads(fx: dict) -> list:
    return [fx[f"grad{i}"] for i in range(sum(k.startswith("grad") for k in fx))]


def tables(params):
    op = [np.ascontiguousarray(q.reshape(-1)).copy() for q in params]
    return op, [np.zeros_like(q) for q in op], [np.zeros_like(q) for q in op], [np.zeros_like(q) for q in op]


def bias_scale(ref: list, i: int):
    """Biases (even index >= 2 in the block) are judged on their layer's weight-gradient scale."""
    return max(np.abs(ref[i]).max(), np.abs(ref[i - 1]).max()) if i >= 2 and i % 2 == 0 else None


def test_golden_c1_oracle(orc):
    (x, labels, params), d = G.inputs_c1()
    fx = load("c1_mlp_step.npz", d)
    c = G.C1
    op, og, om, ov = tables(params)
    loss = orc.call("orc_c1_step", c.batch, c.inp, c.hidden, c.classes, orc.ptr(x), orc.ptr(labels),
                    orc.ptr_table(op), orc.ptr_table(og), orc.ptr_table(om), orc.ptr_table(ov), 0.0, 1, 0, None)
    assert loss == pytest.approx(float(fx["loss"]), rel=1e-5)
    for i, (a, b) in enumerate(zip(og, grads(fx))):
        assert_close(a, b, what=f"c1 grad {i}", **GRAD)


def test_golden_c4_oracle(orc):
    (ids, tgt, params), d = G.inputs_c4()
    fx = load("c4_block_step.npz", d)
    c = G.C4
    op, og, om, ov = tables(params)
    loss = orc.call("orc_c4_step", c.batch, c.seq, c.d_model, c.heads, c.ffn, c.vocab, orc.ptr(ids), orc.ptr(tgt),
                    orc.ptr_table(op), orc.ptr_table(og), orc.ptr_table(om), orc.ptr_table(ov), 0.0, 1, 1)
    assert loss == pytest.approx(float(fx["loss"]), rel=1e-5)
    ref = grads(fx)
    for i, (a, b) in enumerate(zip(og, ref)):
        assert_close(a, b, what=f"c4 grad {i}", scale=bias_scale(ref, i), **GRAD)


def test_golden_c5_oracle(orc):
    (x, noise, t, params), d = G.inputs_c5()
    fx = load("c5_resblock_step.npz", d)
    c = G.C5
    op, og, om, ov = tables(params)
    loss = orc.call("orc_c5_step", c.batch, c.cin, c.cout, c.h, c.w, c.groups, c.tdim, t, orc.ptr(x),
                    orc.ptr(noise), orc.ptr_table(op), orc.ptr_table(og), orc.ptr_table(om), orc.ptr_table(ov),
                    0.0, 1, 1)
    assert loss == pytest.approx(float(fx["loss"]), rel=1e-5)
    for i, (a, b) in enumerate(zip(og, grads(fx))):
        assert_close(a, b, what=f"c5 grad {i}", **GRAD)


def test_golden_detects_a_planted_error(orc):
    """A dropped term in the oracle's result must fail the fixture check: the
    LM-head bias gradient with one token's contribution removed."""
    (ids, tgt, params), d = G.inputs_c4()
    fx = load("c4_block_step.npz", d)
    c = G.C4
    op, og, om, ov = tables(params)
    orc.call("orc_c4_step", c.batch, c.seq, c.d_model, c.heads, c.ffn, c.vocab, orc.ptr(ids), orc.ptr(tgt),
             orc.ptr_table(op), orc.ptr_table(og), orc.ptr_table(om), orc.ptr_table(ov), 0.0, 1, 1)
    ref = grads(fx)
    bad = og[14].copy()
    bad[tgt[0, 0]] += 1.0 / c.batch  # undo the -t/B term of one token
    with pytest.raises(AssertionError):
        assert_close(bad, ref[14], what="planted", scale=bias_scale(ref, 14), **GRAD)

"""Fused attention (mle_attention_fwd / mle_attention_bwd) against the oracle's
composition of MultiHeadAttention's node chain: headify, BMMABT, Scale,
SOFTMASK / SOFTMAX type 1, BMM, DeHeadify and their backwards
(Engine/transformer.cu:647-661; the oracle's orc_bcmm, orc_softmax,
orc_softmax_bwd and orc_headify, as orc_c4_step composes them).

Tolerance: the GEMM class (1e-4 relative, 1e-5 of the largest magnitude):
every output is a sum of products of fp32 operands, with exp() of the
shifted scores in between (the kernels use the hardware exp2, the oracle
libm expf)."""
import numpy as np
import pytest

from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

MM = dict(rtol=1e-4, atol_scale=1e-5)
HD = 64


def B(h, a):
    return h.Buffer.from_array(np.ascontiguousarray(a))


def oracle_attention(orc, q, k, v, dout, b, h, s, scale, causal, kref):
    """q, k, v, dout: [b, s, h*64] float32.  Returns out, dq, dk, dv ([b, s, h*64])."""
    E = h * HD
    nsd, nss = b * s * E, b * h * s * s

    def headify(x):
        xc = np.ascontiguousarray(x)  # held: the oracle reads it through a raw pointer
        y = np.zeros(nsd, np.float32)
        orc.call("orc_headify", orc.ptr(xc), orc.ptr(y), b, h, s, HD, 0)
        return y

    def dehead(x):
        y = np.zeros(nsd, np.float32)
        orc.call("orc_headify", orc.ptr(x), orc.ptr(y), b, h, s, HD, 1)
        return y.reshape(b, s, E)

    Q, K, V, dO = headify(q), headify(k), headify(v), headify(dout)
    sc, scs, A = (np.zeros(nss, np.float32) for _ in range(3))
    orc.call("orc_bcmm", 1, orc.ptr(Q), orc.ptr(K), orc.ptr(sc), b, h, s, HD, s, 0, 3, 3, 3, 1.0)
    orc.call("orc_scale_write", orc.ptr(sc), orc.ptr(scs), scale, nss)
    orc.call("orc_softmax", orc.ptr(scs), orc.ptr(A), b * h, s, s, 1, int(causal))
    O = np.zeros(nsd, np.float32)
    orc.call("orc_bcmm", 0, orc.ptr(A), orc.ptr(V), orc.ptr(O), b, h, s, s, HD, 0, 3, 3, 3, 1.0)
    dA, dV = np.zeros(nss, np.float32), np.zeros(nsd, np.float32)
    orc.call("orc_bcmm", 1, orc.ptr(dO), orc.ptr(V), orc.ptr(dA), b, h, s, HD, s, 1, 3, 3, 3, 1.0)
    orc.call("orc_bcmm", 2, orc.ptr(A), orc.ptr(dO), orc.ptr(dV), b, h, s, s, HD, 1, 3, 3, 3, 1.0)
    dscs, dsc = np.zeros(nss, np.float32), np.zeros(nss, np.float32)
    orc.call("orc_softmax_bwd", orc.ptr(A), orc.ptr(dA), orc.ptr(dscs), b * h, s, s, 1)
    orc.call("orc_accumulate", orc.ptr(dscs), orc.ptr(dsc), float(scale), nss)
    dQ, dK = np.zeros(nsd, np.float32), np.zeros(nsd, np.float32)
    orc.call("orc_bcmm", 0, orc.ptr(dsc), orc.ptr(K), orc.ptr(dQ), b, h, s, s, HD, 1, 3, 3, 3, 1.0)
    if kref:
        orc.call("orc_bcmm", 3, orc.ptr(Q), orc.ptr(dsc), orc.ptr(dK), b, h, HD, s, s, 1, 3, 3, 3, 1.0)
    else:
        orc.call("orc_bcmm", 2, orc.ptr(dsc), orc.ptr(Q), orc.ptr(dK), b, h, s, s, HD, 1, 3, 3, 3, 1.0)
    o = np.zeros(nsd, np.float32)
    orc.call("orc_headify", orc.ptr(O), orc.ptr(o), b, h, s, HD, 2)
    return o.reshape(b, s, E), dehead(dQ), dehead(dK), dehead(dV)


CASES = [
    # (batch, heads, seq, extra columns of ld, causal, reference K gradient)
    (2, 2, 64, 0, 1, 1), (2, 2, 64, 0, 0, 0), (1, 3, 192, 0, 1, 0), (1, 3, 192, 0, 0, 1),
    (2, 1, 128, 64, 1, 1), (1, 2, 256, 0, 1, 1), (1, 2, 256, 0, 1, 0),
    # past 256 the slice kernels hand over to the four-kernel path
    (1, 2, 320, 0, 1, 1), (1, 1, 384, 64, 0, 0),
]


@pytest.mark.parametrize("b,h,s,extra,causal,kref", CASES)
def test_attention_fused(hip, orc, b, h, s, extra, causal, kref):
    r = rng(1000 + 97 * b + 13 * h + s + extra + 5 * causal + kref)
    E = h * HD
    ld = E + extra
    scale = 1.0 / 8.0
    full = lambda: r.standard_normal((b, s, ld), dtype=np.float32)  # noqa: E731
    q, k, v, dout = full(), full(), full(), full()
    ref_o, ref_dq, ref_dk, ref_dv = oracle_attention(orc, q[:, :, :E], k[:, :, :E], v[:, :, :E], dout[:, :, :E],
                                                     b, h, s, scale, causal, kref)
    L = hip.lib()
    ws = hip.Buffer(L.mle_attention_ws_bytes(b, h, s))
    gq, gk, gv, gdo = B(hip, q), B(hip, k), B(hip, v), B(hip, dout)
    gout = B(hip, np.full((b, s, ld), np.nan, np.float32))
    hip.call("mle_attention_fwd", None, gq.ptr, gk.ptr, gv.ptr, gout.ptr, b, h, s, HD, ld, scale, causal, ws.ptr,
             ws.nbytes)
    out = gout.numpy().reshape(b, s, ld)
    assert_close(out[:, :, :E], ref_o, what="attention out", **MM)
    assert np.isnan(out[:, :, E:]).all(), "columns past heads*64 must stay untouched"

    # assign (destinations start as NaN), then accumulate onto random values
    for acc in (0, 1):
        init = [r.standard_normal((b, s, ld), dtype=np.float32) for _ in range(3)]
        bufs = [B(hip, x if acc else np.full_like(x, np.nan)) for x in init]
        hip.call("mle_attention_bwd", None, gq.ptr, gk.ptr, gv.ptr, gdo.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr,
                 b, h, s, HD, ld, scale, causal, acc, acc, acc, kref, ws.ptr, ws.nbytes)
        for name, buf, x, ref in zip(("dq", "dk", "dv"), bufs, init, (ref_dq, ref_dk, ref_dv)):
            got = buf.numpy().reshape(b, s, ld)
            want = ref + (x[:, :, :E] if acc else 0)
            assert_close(got[:, :, :E], want, what=f"attention {name} acc={acc}", scale=float(np.abs(ref).max()), **MM)


def test_attention_rejects_unsupported(hip):
    L = hip.lib()
    g = hip.Buffer.zeros(64 * 64 * 4)
    ws = hip.Buffer(L.mle_attention_ws_bytes(1, 1, 64))
    with pytest.raises(hip.MLEError):  # head_dim 32
        hip.call("mle_attention_fwd", None, g.ptr, g.ptr, g.ptr, g.ptr, 1, 1, 64, 32, 64, 1.0, 1, ws.ptr, ws.nbytes)
    with pytest.raises(hip.MLEError):  # seq not a multiple of 64
        hip.call("mle_attention_fwd", None, g.ptr, g.ptr, g.ptr, g.ptr, 1, 1, 48, 64, 64, 1.0, 1, ws.ptr, ws.nbytes)
    # tensors of 2 GiB (2^29 floats: 1024 x 1024 x 512) and more are refused by
    # their byte size before anything is launched; the buffers are never read
    for call in ("mle_attention_fwd", "mle_attention_bwd"):
        args = (None, g.ptr, g.ptr, g.ptr, g.ptr) if call == "mle_attention_fwd" else \
            (None, g.ptr, g.ptr, g.ptr, g.ptr, g.ptr, g.ptr, g.ptr)
        shape = (1024, 8, 1024, 64, 512, 1.0, 1)
        tail = (ws.ptr, ws.nbytes) if call == "mle_attention_fwd" else (1, 1, 1, 1, ws.ptr, ws.nbytes)
        with pytest.raises(hip.MLEError, match="2 GiB|head_dim"):
            hip.call(call, *args, *shape, *tail)

"""Kernel-level parity: every C ABI entry point against the CPU oracle.

Bars: integer/index paths bit-exact; elementwise,
reduction and optimizer results within 1e-5 relative; GEMM and convolution
within 1e-4 relative (absolute floor scaled by the output's largest value,
which is where fp32 accumulation error lives for a K-long dot product).
"""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_close, rng

pytestmark = pytest.mark.gpu

EW = dict(rtol=1e-5, atol_scale=1e-6)      # elementwise / reductions / optimizer
MM = dict(rtol=1e-4, atol_scale=1e-5)      # GEMM / conv


def B(h, a):
    return h.Buffer.from_array(np.ascontiguousarray(a))


# --------------------------------------------------------------------------- GEMM
GEMM_CASES = [
    # (ta, tb, M, N, K, batch)
    (0, 0, 64, 64, 32, 1),
    (0, 1, 130, 70, 37, 1),
    (1, 0, 129, 257, 45, 1),
    (1, 1, 33, 100, 64, 1),
    (0, 0, 256, 384, 512, 1),
    (0, 1, 200, 136, 256, 3),
    (1, 0, 64, 96, 300, 2),
    (1, 1, 256, 256, 64, 2),
    # grids large enough for the 128 x 128 tile, with ragged edges and batches
    (0, 0, 2048, 4096, 40, 1),
    (1, 0, 2050, 4100, 36, 1),
    (0, 1, 1024, 1024, 20, 8),
    (1, 1, 2064, 2056, 24, 2),
    # register-direct kernel (K % 16 == 0, >= 192 tiles): one workgroup per CU
    # (<= 256 workgroups, deep prefetch) and two per CU, every layout, ragged
    # M and N, K shorter and longer than the prefetch depth
    (0, 0, 2000, 1700, 48, 1),
    (0, 1, 2000, 1700, 16, 1),
    (1, 0, 1990, 1708, 112, 1),
    (1, 1, 2010, 1696, 80, 1),
    (0, 0, 2100, 2052, 32, 1),
    (0, 1, 2100, 2052, 208, 1),
    (1, 0, 2098, 2060, 48, 1),
    (1, 1, 2060, 2100, 16, 1),
    (0, 1, 1000, 1000, 96, 2),
    # K a multiple of 64 (deepest stage shapes), ragged M and N
    (0, 0, 2100, 2052, 128, 1),
    (0, 1, 1990, 2100, 192, 1),
    (1, 0, 2098, 2060, 256, 1),
    (1, 1, 2060, 2004, 64, 1),
    # N not a multiple of 4 with float4-able operands: not the direct kernel
    (0, 1, 2000, 1702, 48, 1),
    # persistent kernel (more 128 x 128 tiles than two per CU, K % 64 == 0): each
    # workgroup walks several tiles, the loads of the next tile overlapping
    # the last stages of the current one; ragged edges and batches
    (0, 0, 4100, 4000, 64, 1),
    (0, 1, 3000, 2900, 192, 1),
    (1, 0, 2500, 4096, 128, 1),
    (1, 1, 2100, 2052, 64, 2),
    (0, 0, 1000, 1000, 256, 9),
    # one-thread-per-element kernel (M or K of at most 4): a Linear on one
    # row (time embedding), its input and weight gradients, odd sizes, batches
    (0, 0, 1, 128, 256, 1), (0, 1, 1, 256, 128, 1), (1, 0, 256, 128, 1, 1),
    (1, 1, 3, 37, 53, 2), (0, 0, 70, 33, 3, 3), (0, 1, 4, 1000, 999, 1),
]


@pytest.mark.parametrize("ta,tb,M,N,K,batch", GEMM_CASES)
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gemm(hip, orc, ta, tb, M, N, K, batch, beta):
    r = rng(1000 + M + N + K + batch + ta * 7 + tb * 11)
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    A = r.standard_normal(a_shape, dtype=np.float32)
    Bm = r.standard_normal(b_shape, dtype=np.float32)
    C0 = r.standard_normal((batch, M, N), dtype=np.float32)
    alpha = 0.5
    ref = C0.copy()
    kind = ta * 2 + tb
    # orc_bcmm dims: kind 0 (m,n,p)=(M,K,N), 1 (M,K,N), 2 (M,K,N), 3 (M,K,N)
    orc.call("orc_bcmm", kind, orc.ptr(A), orc.ptr(Bm), orc.ptr(ref), batch, 1, M, K, N, int(beta != 0), 3, 3, 3, alpha)
    dA, dB, dC = B(hip, A), B(hip, Bm), B(hip, C0)
    lda = M if ta else K
    ldb = K if tb else N
    hip.call("mle_gemm", None, ta, tb, M, N, K, alpha, dA.ptr, lda, A[0].size, dB.ptr, ldb, Bm[0].size, beta,
             dC.ptr, N, M * N, batch, None)
    assert_close(dC.numpy(), ref, what=f"gemm ta={ta} tb={tb}", **MM)


@pytest.mark.parametrize("case", ["scores_nt", "xty_tn", "mix_nn", "tt"])
@pytest.mark.parametrize("b,heads,seq,hd", [(2, 3, 40, 16), (4, 8, 256, 64)])
def test_gemm_grid_heads_in_place(hip, orc, case, b, heads, seq, hd):
    """Per-head products addressed in the [b, seq, heads*hd] layout (two-level
    batch: batch stride seq*E, head stride hd) against the oracle's bcmm on
    explicitly headified copies, for every layout."""
    r = rng(b * 13 + heads + seq + len(case))
    E = heads * hd
    X = r.standard_normal((b, seq, E), dtype=np.float32)
    Y = r.standard_normal((b, seq, E), dtype=np.float32)
    P = r.standard_normal((b, heads, seq, seq), dtype=np.float32)
    hf = lambda T: np.ascontiguousarray(T.reshape(b, seq, heads, hd).transpose(0, 2, 1, 3))  # [b, heads, seq, hd]
    proj = (E, seq * E, hd)            # (ld, outer stride, inner stride) of a head slice of X / Y
    sq = (seq, heads * seq * seq, seq * seq)
    # (ta, tb, M, N, K, A device/explicit/addr, B ..., C shape, C addr or None for contiguous [b, heads, M, N])
    if case == "scores_nt":
        ta, tb, M, N, K = 0, 1, seq, seq, hd
        Ad, Ae, Aa, Bd, Be, Ba = X, hf(X), proj, Y, hf(Y), proj
    elif case == "xty_tn":
        ta, tb, M, N, K = 1, 0, hd, hd, seq
        Ad, Ae, Aa, Bd, Be, Ba = X, hf(X), proj, Y, hf(Y), proj
    elif case == "mix_nn":
        ta, tb, M, N, K = 0, 0, seq, hd, seq
        Ad, Ae, Aa, Bd, Be, Ba = P, P, sq, Y, hf(Y), proj
    else:
        ta, tb, M, N, K = 1, 1, hd, seq, seq
        Ad, Ae, Aa, Bd, Be, Ba = X, hf(X), proj, P, P, sq
    alpha = 0.25
    ref = r.standard_normal((b, heads, M, N), dtype=np.float32)
    C0 = ref.copy()
    Ae, Be = np.ascontiguousarray(Ae), np.ascontiguousarray(Be)  # held while the oracle reads them
    orc.call("orc_bcmm", ta * 2 + tb, orc.ptr(Ae), orc.ptr(Be), orc.ptr(ref), b, heads, M, K, N, 1, 3, 3, 3, alpha)
    if case == "mix_nn":  # result written in the projection layout [b, seq, heads * hd]
        C0p = np.ascontiguousarray(C0.transpose(0, 2, 1, 3).reshape(b, seq, E))
        gC = B(hip, C0p)
        cl, cs, ci = E, seq * E, hd
    else:
        gC = B(hip, C0)
        cl, cs, ci = N, heads * M * N, M * N
    gA, gB = B(hip, Ad), B(hip, Bd)
    hip.call("mle_gemm_grid", None, ta, tb, M, N, K, alpha, gA.ptr, *Aa, gB.ptr, *Ba, 1.0, gC.ptr, cl, cs, ci, b, heads,
             None, 0)
    got = gC.numpy()
    if case == "mix_nn":
        got = got.reshape(b, seq, heads, hd).transpose(0, 2, 1, 3)
    assert_close(got, ref, what=f"gemm_grid {case}", **MM)


@pytest.mark.parametrize("ta,tb,M,N,K,batch,cs", [
    (1, 0, 256, 256, 8192, 1, True),    # dW of a small Linear: split over K
    (1, 0, 512, 1000, 4100, 1, True),   # ragged N and K
    (0, 1, 300, 200, 3000, 1, False),
    (0, 0, 128, 130, 2048, 3, False),   # batched split
])
def test_gemm_split_k(hip, orc, ta, tb, M, N, K, batch, cs):
    r = rng(M + N + K)
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    A = r.standard_normal(a_shape, dtype=np.float32)
    Bm = r.standard_normal(b_shape, dtype=np.float32)
    C0 = r.standard_normal((batch, M, N), dtype=np.float32)
    ref = C0.copy()
    orc.call("orc_bcmm", ta * 2 + tb, orc.ptr(A), orc.ptr(Bm), orc.ptr(ref), batch, 1, M, K, N, 1, 3, 3, 3, 0.75)
    L = hip.lib()
    need = L.mle_gemm_ws_bytes(M, N, K, batch)
    assert need > 0, "shape expected to split"
    ws = hip.Buffer(need)
    dA, dB, dC = B(hip, A), B(hip, Bm), B(hip, C0)
    cs0 = r.standard_normal(N, dtype=np.float32)
    dcs = B(hip, cs0) if cs else None
    bias = r.standard_normal(N, dtype=np.float32)
    dbias = B(hip, bias)
    hip.call("mle_gemm_ex", None, ta, tb, M, N, K, 0.75, dA.ptr, M if ta else K, A[0].size, dB.ptr, K if tb else N,
             Bm[0].size, 1.0, dC.ptr, N, M * N, batch, dcs.ptr if cs else None, dbias.ptr, ws.ptr, ws.nbytes)
    assert_close(dC.numpy(), ref + bias, what="split-K gemm + bias", **MM)
    if cs:
        bsum = Bm[0].astype(np.float64).sum(1 if tb else 0)
        assert_close(dcs.numpy(), cs0 + bsum, what="split-K colsum", **EW)


@pytest.mark.parametrize("ta,tb,M,N,K,batch,with_ws", [
    (0, 0, 1000, 512, 512, 3, False),   # sibling projections: X broadcast, W_i, b_i strided
    (0, 0, 4000, 1536, 128, 3, False),  # persistent kernel with per-item bias
    (0, 0, 257, 132, 100, 2, True),
    (1, 0, 512, 512, 8192, 3, True),    # sibling dW_i = X^T dY_i, db_i: split over K
    (1, 0, 128, 200, 3000, 3, True),
    (1, 0, 96, 64, 300, 3, False),
])
def test_gemm_batched_ex(hip, orc, ta, tb, M, N, K, batch, with_ws):
    """Batched GEMM whose items carry their own bias and column-sum vectors
    (stride_bias / stride_colsum), with item strides that leave gaps between
    items as the parameter arena does."""
    r = rng(M + 3 * N + K + batch)
    gap = 8                                            # floats between consecutive items
    a_shape = (K, M) if ta else (M, K)                 # A broadcast over the batch (stride 0)
    A = r.standard_normal(a_shape, dtype=np.float32)
    b_item = (N, K) if tb else (K, N)
    sb = int(np.prod(b_item)) + gap
    Bflat = r.standard_normal(batch * sb, dtype=np.float32)
    Bi = [Bflat[i * sb:i * sb + int(np.prod(b_item))].reshape(b_item) for i in range(batch)]
    sc = M * N + gap
    Cflat = r.standard_normal(batch * sc, dtype=np.float32)
    beta = 1.0 if ta else 0.0
    ref = []
    for i in range(batch):
        c = Cflat[i * sc:i * sc + M * N].reshape(M, N).copy()
        Ac, Bc = np.ascontiguousarray(A), np.ascontiguousarray(Bi[i])  # held while the oracle reads them
        orc.call("orc_bcmm", ta * 2 + tb, orc.ptr(Ac), orc.ptr(Bc), orc.ptr(c), 1, 1, M, K, N, int(beta != 0), 3, 3, 3,
                 0.5)
        ref.append(c)
    svec = N + 4
    gA, gB, gC = B(hip, A), B(hip, Bflat), B(hip, Cflat)
    L = hip.lib()
    need = L.mle_gemm_ws_bytes(M, N, K, batch) if with_ws else 0
    ws = hip.Buffer(max(need, 4)) if with_ws else None
    if ta:  # dW-style: fused column sums of each B_i into its own vector
        cs0 = r.standard_normal(batch * svec, dtype=np.float32)
        gcs = B(hip, cs0)
        hip.call("mle_gemm_batched_ex", None, ta, tb, M, N, K, 0.5, gA.ptr, M, 0, gB.ptr, K if tb else N, sb, beta,
                 gC.ptr, N, sc, batch, gcs.ptr, svec, None, 0, ws.ptr if ws else None, need)
        cs = gcs.numpy()
        for i in range(batch):
            want = cs0[i * svec:i * svec + N] + Bi[i].astype(np.float64).sum(1 if tb else 0)
            assert_close(cs[i * svec:i * svec + N], want, what=f"colsum item {i}", **EW)
            assert np.array_equal(cs[i * svec + N:(i + 1) * svec], cs0[i * svec + N:(i + 1) * svec]), "gap written"
    else:   # forward-style: per-item bias
        bias = r.standard_normal(batch * svec, dtype=np.float32)
        gbias = B(hip, bias)
        hip.call("mle_gemm_batched_ex", None, ta, tb, M, N, K, 0.5, gA.ptr, M if ta else K, 0, gB.ptr,
                 K if tb else N, sb, beta, gC.ptr, N, sc, batch, None, 0, gbias.ptr, svec, ws.ptr if ws else None, need)
        for i in range(batch):
            ref[i] += bias[i * svec:i * svec + N]
    got = gC.numpy()
    for i in range(batch):
        assert_close(got[i * sc:i * sc + M * N].reshape(M, N), ref[i], what=f"batched_ex item {i}", **MM)
        assert np.array_equal(got[i * sc + M * N:(i + 1) * sc], Cflat[i * sc + M * N:(i + 1) * sc]), "gap written"


@pytest.mark.parametrize("ta,tb,M,N,K,terms", [
    (0, 1, 8192, 512, 512, 3),   # dX = sum_i dY_i W_i^T of sibling projections
    # register-direct kernel: the terms extend its K loop (every layout,
    # ragged M and N)
    (0, 1, 2000, 1700, 64, 3),
    (1, 0, 1990, 1708, 48, 2),
    (0, 0, 2100, 2052, 32, 4),
    (1, 1, 2060, 2004, 80, 3),
    # one split per term, reduced in term order
    (0, 1, 1000, 132, 260, 3),
    (0, 0, 300, 200, 100, 2),
    (1, 0, 64, 96, 500, 4),
    (0, 1, 200, 64, 64, 1),
])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gemm_sum(hip, orc, ta, tb, M, N, K, terms, beta):
    """C = alpha * sum_t A_t B_t + beta C over term-strided operands."""
    r = rng(M + N + 5 * K + terms)
    gap = 4
    a_item = (K, M) if ta else (M, K)
    b_item = (N, K) if tb else (K, N)
    sa, sb = int(np.prod(a_item)) + gap, int(np.prod(b_item)) + 2 * gap
    Af = r.standard_normal(terms * sa, dtype=np.float32)
    Bf = r.standard_normal(terms * sb, dtype=np.float32)
    C0 = r.standard_normal((M, N), dtype=np.float32)
    ref = C0.copy() if beta else np.zeros((M, N), np.float32)
    for t in range(terms):
        At = np.ascontiguousarray(Af[t * sa:t * sa + int(np.prod(a_item))].reshape(a_item))
        Bt = np.ascontiguousarray(Bf[t * sb:t * sb + int(np.prod(b_item))].reshape(b_item))
        orc.call("orc_bcmm", ta * 2 + tb, orc.ptr(At), orc.ptr(Bt), orc.ptr(ref), 1, 1, M, K, N, 1, 3, 3, 3, 0.75)
    L = hip.lib()
    need = L.mle_gemm_sum_ws_bytes(M, N, terms)
    ws = hip.Buffer(max(need, 4))
    gA, gB, gC = B(hip, Af), B(hip, Bf), B(hip, C0)
    hip.call("mle_gemm_sum", None, ta, tb, M, N, K, 0.75, gA.ptr, M if ta else K, sa, gB.ptr, K if tb else N, sb, beta,
             gC.ptr, N, terms, ws.ptr, need)
    assert_close(gC.numpy(), ref, what=f"gemm_sum terms={terms}", **MM)
    if terms > 1:
        with pytest.raises(hip.MLEError):
            hip.call("mle_gemm_sum", None, ta, tb, M, N, K, 0.75, gA.ptr, M if ta else K, sa, gB.ptr,
                     K if tb else N, sb, beta, gC.ptr, N, terms, ws.ptr, need - 4)


@pytest.mark.parametrize("rows,inp,out,layers,bias,acc", [
    (8192, 384, 128, 1, True, 0),     # dX and dW share one launch
    (8192, 384, 256, 3, True, 1),     # three layers: dX terms folded into K, dW batched
    (8192, 512, 512, 1, False, 1),    # the attention output projection's shape
    (8192, 2048, 128, 1, True, 0),    # dX on the persistent kernel: two launches
    (300, 130, 70, 2, True, 1),       # small: LDS kernels, split partials
    (64, 256, 10, 1, True, 0),        # both products small: one one-thread-per-output launch
    (64, 256, 10, 1, True, 1),
    (64, 100, 7, 2, True, 1),         # small, two layers: one launch per product
    (64, 784, 256, 1, True, 0),       # K split over a workgroup's waves, both products in one launch
    (64, 784, 256, 1, True, 1),
    (100, 60, 333, 1, True, 1),       # the same with ragged tiles and K tails
    (512, 512, 512, 1, False, 0),     # 32-wide K-split tiles
])
def test_linear_bwd(hip, orc, rows, inp, out, layers, bias, acc):
    """mle_linear_bwd against the oracle's bcmm products and column sums, with
    gaps between the layers' dY, W/dW and db (the parameter arena's padding),
    which must stay untouched."""
    r = rng(rows + inp + 7 * out + layers)
    gap = 8
    sdy, sw, sb = rows * out + gap, inp * out + gap, out + gap
    X = r.standard_normal((rows, inp), dtype=np.float32)
    dYf = r.standard_normal(layers * sdy, dtype=np.float32)
    Wf = r.standard_normal(layers * sw, dtype=np.float32)
    dX0 = r.standard_normal((rows, inp), dtype=np.float32)
    dWf = r.standard_normal(layers * sw, dtype=np.float32)
    dbf = r.standard_normal(layers * sb, dtype=np.float32)
    dY = [np.ascontiguousarray(dYf[l * sdy:l * sdy + rows * out].reshape(rows, out)) for l in range(layers)]
    W = [np.ascontiguousarray(Wf[l * sw:l * sw + inp * out].reshape(inp, out)) for l in range(layers)]
    want_dx = dX0.copy() if acc else np.zeros_like(dX0)
    for l in range(layers):
        orc.call("orc_bcmm", 1, orc.ptr(dY[l]), orc.ptr(W[l]), orc.ptr(want_dx), 1, 1, rows, out, inp, 1, 3, 3, 3, 1.0)
    want_dw, want_db = [], []
    for l in range(layers):
        w = np.ascontiguousarray(dWf[l * sw:l * sw + inp * out].reshape(inp, out)).copy()
        orc.call("orc_bcmm", 2, orc.ptr(X), orc.ptr(dY[l]), orc.ptr(w), 1, 1, inp, rows, out, 1, 3, 3, 3, 1.0)
        want_dw.append(w)
        want_db.append(dbf[l * sb:l * sb + out] + dY[l].astype(np.float64).sum(0))
    L = hip.lib()
    need = L.mle_linear_bwd_ws_bytes(rows, inp, out, layers)
    ws = hip.Buffer(max(need, 4))
    gX, gdY, gW, gdX, gdW, gdb = (B(hip, a) for a in (X, dYf, Wf, dX0, dWf, dbf))
    hip.call("mle_linear_bwd", None, rows, inp, out, layers, gX.ptr, gdY.ptr, sdy, gW.ptr, sw, gdX.ptr, acc, gdW.ptr,
             gdb.ptr if bias else None, sb, ws.ptr, need)
    assert_close(gdX.numpy(), want_dx, what="linear_bwd dX", **MM)
    got_w, got_b = gdW.numpy(), gdb.numpy()
    for l in range(layers):
        assert_close(got_w[l * sw:l * sw + inp * out].reshape(inp, out), want_dw[l], what=f"linear_bwd dW {l}", **MM)
        assert np.array_equal(got_w[l * sw + inp * out:(l + 1) * sw], dWf[l * sw + inp * out:(l + 1) * sw]), "dW gap"
        if bias:
            assert_close(got_b[l * sb:l * sb + out], want_db[l], what=f"linear_bwd db {l}", **EW)
        else:
            assert np.array_equal(got_b, dbf), "db written without bias"
    # mle_linear_bwd_ex with accumulate_dw 0: dW and db assigned (NaN before),
    # the bits of adding into zeros; the gaps stay untouched
    zw = [np.zeros((inp, out), np.float32) for _ in range(layers)]
    for l in range(layers):
        orc.call("orc_bcmm", 2, orc.ptr(X), orc.ptr(dY[l]), orc.ptr(zw[l]), 1, 1, inp, rows, out, 1, 3, 3, 3, 1.0)
    nan_w, nan_b = dWf.copy(), dbf.copy()
    for l in range(layers):
        nan_w[l * sw:l * sw + inp * out] = np.nan
        nan_b[l * sb:l * sb + out] = np.nan
    gdW2, gdb2, gdX2 = B(hip, nan_w), B(hip, nan_b), B(hip, dX0)
    hip.call("mle_linear_bwd_ex", None, rows, inp, out, layers, gX.ptr, gdY.ptr, sdy, gW.ptr, sw, gdX2.ptr, acc,
             gdW2.ptr, gdb2.ptr if bias else None, sb, 0, ws.ptr, need)
    got_w2, got_b2 = gdW2.numpy(), gdb2.numpy()
    zero_w, zero_b = B(hip, np.where(np.isnan(nan_w), 0.0, nan_w).astype(np.float32)), \
        B(hip, np.where(np.isnan(nan_b), 0.0, nan_b).astype(np.float32))
    gdX3 = B(hip, dX0)
    hip.call("mle_linear_bwd", None, rows, inp, out, layers, gX.ptr, gdY.ptr, sdy, gW.ptr, sw, gdX3.ptr, acc,
             zero_w.ptr, zero_b.ptr if bias else None, sb, ws.ptr, need)
    np.testing.assert_array_equal(got_w2, zero_w.numpy())
    if bias:
        np.testing.assert_array_equal(got_b2, zero_b.numpy())
    for l in range(layers):
        assert_close(got_w2[l * sw:l * sw + inp * out].reshape(inp, out), zw[l], what=f"linear_bwd_ex dW {l}", **MM)
    # errors: a short workspace (when one is needed) and zero layers
    if need:
        with pytest.raises(hip.MLEError):
            hip.call("mle_linear_bwd", None, rows, inp, out, layers, gX.ptr, gdY.ptr, sdy, gW.ptr, sw, gdX.ptr, acc,
                     gdW.ptr, None, sb, ws.ptr, need - 4)
    with pytest.raises(hip.MLEError):
        hip.call("mle_linear_bwd", None, rows, inp, out, 0, gX.ptr, gdY.ptr, sdy, gW.ptr, sw, gdX.ptr, acc, gdW.ptr,
                 None, sb, ws.ptr, need)


@pytest.mark.parametrize("M,N,K", [(100, 40, 300), (40, 40, 500), (300, 90, 77), (2048, 4096, 40), (64, 130, 300),
                                   (2048, 4096, 48), (2000, 1700, 48), (1000, 2052, 4112)])
def test_gemm_colsum_tiles(hip, orc, M, N, K):
    """dW = X^T dY with the fused column sum, on every workgroup tile shape."""
    r = rng(M * 3 + N + K)
    X = r.standard_normal((K, M), dtype=np.float32)
    dY = r.standard_normal((K, N), dtype=np.float32)
    dWr = np.ones((M, N), np.float32)
    dbr = np.full(N, 0.25, np.float32)
    orc.call("orc_bcmm", 2, orc.ptr(X), orc.ptr(dY), orc.ptr(dWr), 1, 1, M, K, N, 1, 3, 3, 0, 1.0)
    orc.call("orc_bcompress", orc.ptr(dY), orc.ptr(dbr), K, N, 1.0)
    gX, gY = B(hip, X), B(hip, dY)
    gW, gb = B(hip, np.ones((M, N), np.float32)), B(hip, np.full(N, 0.25, np.float32))
    hip.call("mle_gemm", None, 1, 0, M, N, K, 1.0, gX.ptr, M, 0, gY.ptr, N, 0, 1.0, gW.ptr, N, 0, 1, gb.ptr)
    assert_close(gW.numpy(), dWr, what="dW", **MM)
    assert_close(gb.numpy(), dbr, what="db", **EW)


def test_gemm_broadcast_and_colsum(hip, orc):
    r = rng(7)
    M, N, K, batch = 96, 80, 72, 3
    A = r.standard_normal((batch, M, K), dtype=np.float32)
    W = r.standard_normal((K, N), dtype=np.float32)  # broadcast operand (stride 0)
    ref = np.zeros((batch, M, N), np.float32)
    orc.call("orc_bcmm", 0, orc.ptr(A), orc.ptr(W), orc.ptr(ref), batch, 1, M, K, N, 0, 3, 0, 3, 1.0)
    dA, dW, dC = B(hip, A), B(hip, W), hip.Buffer.zeros((batch, M, N))
    hip.call("mle_gemm", None, 0, 0, M, N, K, 1.0, dA.ptr, K, M * K, dW.ptr, N, 0, 0.0, dC.ptr, N, M * N, batch, None)
    assert_close(dC.numpy(), ref, what="gemm broadcast B", **MM)
    bias = r.standard_normal(N, dtype=np.float32)
    dbias, dC2 = B(hip, bias), hip.Buffer.zeros((batch, M, N))
    hip.call("mle_gemm_ex", None, 0, 0, M, N, K, 1.0, dA.ptr, K, M * K, dW.ptr, N, 0, 0.0, dC2.ptr, N, M * N, batch,
             None, dbias.ptr, None, 0)
    assert_close(dC2.numpy(), ref + bias, what="gemm + bias epilogue", **MM)
    # dW = X^T dY with fused db = colsum(dY) (Linear backward)
    X = r.standard_normal((300, 64), dtype=np.float32)
    dY = r.standard_normal((300, 130), dtype=np.float32)
    dWr = np.ones((64, 130), np.float32)
    dbr = np.full(130, 0.25, np.float32)
    orc.call("orc_bcmm", 2, orc.ptr(X), orc.ptr(dY), orc.ptr(dWr), 1, 1, 64, 300, 130, 1, 3, 3, 0, 1.0)
    orc.call("orc_bcompress", orc.ptr(dY), orc.ptr(dbr), 300, 130, 1.0)
    gX, gY = B(hip, X), B(hip, dY)
    gW, gb = B(hip, np.ones((64, 130), np.float32)), B(hip, np.full(130, 0.25, np.float32))
    hip.call("mle_gemm", None, 1, 0, 64, 130, 300, 1.0, gX.ptr, 64, 0, gY.ptr, 130, 0, 1.0, gW.ptr, 130, 0, 1, gb.ptr)
    assert_close(gW.numpy(), dWr, what="dW", **MM)
    assert_close(gb.numpy(), dbr, what="db (fused colsum)", **EW)


# ------------------------------------------------------------------- activations
@pytest.mark.parametrize("kind", ["relu", "gelu", "silu", "tanh", "sigmoid", "leaky_relu"])
def test_activation(hip, orc, kind):
    r = rng(11)
    n = 10007
    x = (r.standard_normal(n, dtype=np.float32) * 4).astype(np.float32)
    x[:8] = [0.0, -0.0, 1e-30, -1e-30, 90.0, -90.0, 20.0, -20.0]
    dy = r.standard_normal(n, dtype=np.float32)
    dx0 = r.standard_normal(n, dtype=np.float32)
    k = hip.ACT[kind]
    yr = np.zeros_like(x)
    orc.call("orc_act_fwd", k, orc.ptr(x), orc.ptr(yr), n)
    dxr = dx0.copy()
    orc.call("orc_act_bwd", k, orc.ptr(x), orc.ptr(dy), orc.ptr(dxr), n)
    gx, gy, gdy, gdx = B(hip, x), hip.Buffer.zeros(n), B(hip, dy), B(hip, dx0)
    hip.call("mle_act_fwd", None, k, gx.ptr, gy.ptr, n)
    hip.call("mle_act_bwd", None, k, gx.ptr, gdy.ptr, gdx.ptr, n, 1)
    assert_close(gy.numpy(), yr, what=f"{kind} fwd", **EW)
    assert_close(gdx.numpy(), dxr, what=f"{kind} bwd", **EW)
    # assign: the destination is not read (NaN stays out), value = the sum into zeros
    dxz = np.zeros_like(x)
    orc.call("orc_act_bwd", k, orc.ptr(x), orc.ptr(dy), orc.ptr(dxz), n)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), n)
    hip.call("mle_act_bwd", None, k, gx.ptr, gdy.ptr, gdx.ptr, n, 0)
    assert_close(gdx.numpy(), dxz, what=f"{kind} bwd assign", **EW)


# ----------------------------------------------------------------------- softmax
@pytest.mark.parametrize("bc,rows,cols", [(3, 37, 45), (2, 256, 256), (1, 300, 20), (2, 5, 9000)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("causal", [0, 1])
def test_softmax(hip, orc, bc, rows, cols, axis, causal):
    r = rng(bc * 131 + rows + cols)
    x = (r.standard_normal((bc, rows, cols), dtype=np.float32) * 3).astype(np.float32)
    dy = r.standard_normal((bc, rows, cols), dtype=np.float32)
    dx0 = r.standard_normal((bc, rows, cols), dtype=np.float32)
    yr = np.zeros_like(x)
    orc.call("orc_softmax", orc.ptr(x), orc.ptr(yr), bc, rows, cols, axis, causal)
    dxr = dx0.copy()
    orc.call("orc_softmax_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(dxr), bc, rows, cols, axis)
    gx, gy = B(hip, x), hip.Buffer.zeros(x.shape)
    hip.call("mle_softmax_fwd", None, gx.ptr, gy.ptr, bc, rows, cols, axis, causal)
    y = gy.numpy()
    assert_close(y, yr, what="softmax fwd", **EW)
    gyr, gdy, gdx = B(hip, yr), B(hip, dy), B(hip, dx0)
    hip.call("mle_softmax_bwd", None, gyr.ptr, gdy.ptr, gdx.ptr, bc, rows, cols, axis, 1)
    assert_close(gdx.numpy(), dxr, what="softmax bwd", **EW)
    dxz = np.zeros_like(x)
    orc.call("orc_softmax_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(dxz), bc, rows, cols, axis)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), x.size)
    hip.call("mle_softmax_bwd", None, gyr.ptr, gdy.ptr, gdx.ptr, bc, rows, cols, axis, 0)
    assert_close(gdx.numpy(), dxz, what="softmax bwd assign", **EW)


@pytest.mark.parametrize("cols", [1000, 1500, 2052, 8000])
def test_softmax_xent(hip, orc, cols):
    r = rng(5 + cols)
    rows, batch = 96, 4
    logits = (r.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float32)
    tgt = np.zeros((rows, cols), np.float32)
    tgt[np.arange(rows), r.integers(0, cols, rows)] = 1.0
    pr = np.zeros_like(logits)
    lr_ = orc.call("orc_softmax_xent_fwd", orc.ptr(logits), orc.ptr(tgt), orc.ptr(pr), rows, cols)
    dl = np.zeros_like(logits)
    orc.call("orc_softmax_xent_bwd", orc.ptr(pr), orc.ptr(tgt), None, orc.ptr(dl), rows * cols, batch)
    gl, gt, gp, gloss = B(hip, logits), B(hip, tgt), hip.Buffer.zeros((rows, cols)), hip.Buffer.zeros(1)
    ws = hip.Buffer(hip.lib().mle_loss_ws_bytes(rows * cols))
    hip.call("mle_softmax_xent_fwd", None, gl.ptr, gt.ptr, gp.ptr, rows, cols, gloss.ptr, ws.ptr, ws.nbytes)
    assert_close(gp.numpy(), pr, what="xent probs", **EW)
    assert_close(gloss.numpy(), np.array([lr_], np.float32), what="xent loss", **EW)
    gd = hip.Buffer.zeros((rows, cols))
    hip.call("mle_softmax_xent_bwd", None, gp.ptr, gt.ptr, None, gd.ptr, rows * cols, batch)
    assert_close(gd.numpy(), dl, what="xent bwd", **EW)


@pytest.mark.parametrize("n", [123457, 123456])
def test_mse(hip, orc, n):
    r = rng(6)
    x = r.standard_normal(n, dtype=np.float32)
    t = r.standard_normal(n, dtype=np.float32)
    dx0 = r.standard_normal(n, dtype=np.float32)
    lref = orc.call("orc_mse_loss", orc.ptr(x), orc.ptr(t), n)
    dxr = dx0.copy()
    orc.call("orc_mse_bwd", orc.ptr(x), orc.ptr(t), None, orc.ptr(dxr), n)
    gx, gt, gl, gdx = B(hip, x), B(hip, t), hip.Buffer.zeros(1), B(hip, dx0)
    ws = hip.Buffer(hip.lib().mle_loss_ws_bytes(n))
    hip.call("mle_mse_fwd", None, gx.ptr, gt.ptr, n, gl.ptr, ws.ptr, ws.nbytes)
    hip.call("mle_mse_bwd", None, gx.ptr, gt.ptr, None, gdx.ptr, n, 1)
    assert_close(gl.numpy(), np.array([lref], np.float32), what="mse loss", **EW)
    assert_close(gdx.numpy(), dxr, what="mse bwd", **EW)
    dxz = np.zeros_like(x)
    orc.call("orc_mse_bwd", orc.ptr(x), orc.ptr(t), None, orc.ptr(dxz), n)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), n)
    hip.call("mle_mse_bwd", None, gx.ptr, gt.ptr, None, gdx.ptr, n, 0)
    assert_close(gdx.numpy(), dxz, what="mse bwd assign", **EW)


@pytest.mark.parametrize("n", [123457, 123456, 8 * 1024 * 1024])
@pytest.mark.parametrize("u", [0.75, -3.0e-3])
def test_mse_bwd_upstream(hip, orc, n, u):
    """The loss is not the graph's last node: its gradient (one float, written
    by the consumer) multiplies the derivative, dx += 2 (x - t) u / n
    (deriv_mse_kernel's `!last` branch, Engine/kernels.cu:1846), adding and
    assigning.  8 Mi elements is C5's loss size."""
    r = rng(61 + n % 7)
    x = r.standard_normal(n, dtype=np.float32)
    t = r.standard_normal(n, dtype=np.float32)
    dx0 = r.standard_normal(n, dtype=np.float32)
    up = np.array([u], np.float32)
    gx, gt, gup = B(hip, x), B(hip, t), B(hip, up)
    for acc in (1, 0):
        ref = dx0.copy() if acc else np.zeros_like(x)
        orc.call("orc_mse_bwd", orc.ptr(x), orc.ptr(t), orc.ptr(up), orc.ptr(ref), n)
        gdx = B(hip, dx0) if acc else hip.Buffer.zeros(n)
        if not acc:
            hip.call("mle_fill", None, gdx.ptr, float("nan"), n)
        hip.call("mle_mse_bwd", None, gx.ptr, gt.ptr, gup.ptr, gdx.ptr, n, acc)
        assert_close(gdx.numpy(), ref, what=f"mse bwd upstream acc={acc}", **EW)


@pytest.mark.parametrize("cols", [1000, 8000])
@pytest.mark.parametrize("u", [0.75, -2.5])
def test_softmax_xent_bwd_upstream(hip, orc, cols, u):
    """The cross-entropy is not the last node: dlogits = (p - t) u / batch
    (Engine/engine.cu:2106-2108: ScaleAdd, ScalePtr by the loss node's
    gradient, ScaleValue), assigned, for the dense target and for the id
    target that reads no matrix (ids out of range included)."""
    r = rng(62 + cols)
    batch, clen = 3, 40
    rows = batch * clen
    logits = (r.standard_normal((rows, cols), dtype=np.float32) * 2).astype(np.float32)
    keys = r.integers(0, cols, (batch, clen)).astype(np.int32)
    keys[1, 3] = -1
    keys[2, 0] = cols + 5
    tgt = np.zeros((rows, cols), np.float32)
    for b in range(batch):
        for s_ in range(clen):
            if 0 <= keys[b, s_] < cols:
                tgt[b * clen + s_, keys[b, s_]] = 1.0
    up = np.array([u], np.float32)
    pr = np.zeros_like(logits)
    orc.call("orc_softmax_xent_fwd", orc.ptr(logits), orc.ptr(tgt), orc.ptr(pr), rows, cols)
    ref = np.zeros_like(logits)
    orc.call("orc_softmax_xent_bwd", orc.ptr(pr), orc.ptr(tgt), orc.ptr(up), orc.ptr(ref), rows * cols, batch)
    L = hip.lib()
    n = rows * cols
    gl, gt, gk, gup = B(hip, logits), B(hip, tgt), B(hip, keys), B(hip, up)
    gp, gloss, gst = hip.Buffer.zeros((rows, cols)), hip.Buffer.zeros(1), hip.Buffer.zeros(2 * rows)
    ws = hip.Buffer(L.mle_loss_ws_bytes(n))
    hip.call("mle_softmax_xent_fwd", None, gl.ptr, gt.ptr, gp.ptr, rows, cols, gloss.ptr, ws.ptr, ws.nbytes)
    hip.call("mle_softmax_xent_keys_fwd", None, gl.ptr, gk.ptr, clen, clen, gst.ptr, rows, cols, gloss.ptr, ws.ptr,
             ws.nbytes)
    gd, gd2 = hip.Buffer.zeros((rows, cols)), hip.Buffer.zeros((rows, cols))
    hip.call("mle_fill", None, gd.ptr, float("nan"), n)
    hip.call("mle_fill", None, gd2.ptr, float("nan"), n)
    hip.call("mle_softmax_xent_bwd", None, gp.ptr, gt.ptr, gup.ptr, gd.ptr, n, batch)
    hip.call("mle_softmax_xent_keys_bwd", None, gl.ptr, gst.ptr, gk.ptr, clen, clen, gup.ptr, gd2.ptr, rows, cols,
             batch)
    assert_close(gd.numpy(), ref, what="xent bwd upstream (dense target)", **EW)
    assert_close(gd2.numpy(), ref, what="xent bwd upstream (id target)", **EW)


# ------------------------------------------------------------------------ norms
@pytest.mark.parametrize("batch,channels,hw,groups", [(3, 1, 37 * 45, 1), (2, 1, 256 * 512, 1), (2, 8, 700, 4),
                                                     (2, 64, 4096, 32), (2, 3, 33, 1),
                                                     # 75 chunks per group: lanes merge a second chunk each
                                                     (1, 1, 300 * 1024, 1),
                                                     # the fused Add / MatPE statistics with periods 1024 and
                                                     # 512 (one division per float4 below 1024)
                                                     (2, 1, 512, 1)])
def test_norm(hip, orc, batch, channels, hw, groups):
    r = rng(batch + channels + hw + groups)
    shape = (batch, channels, hw)
    x = (r.standard_normal(shape, dtype=np.float32) * 2 + 0.5).astype(np.float32)
    dy = r.standard_normal(shape, dtype=np.float32)
    dx0 = r.standard_normal(shape, dtype=np.float32)
    yr = np.zeros_like(x)
    st = np.zeros(2 * batch * groups, np.float32)
    orc.call("orc_norm_fwd", orc.ptr(x), orc.ptr(yr), orc.ptr(st), batch, channels, hw, groups, 1e-5)
    dxr = dx0.copy()
    orc.call("orc_norm_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(dxr), orc.ptr(st), batch, channels, hw, groups, 1e-5, 1)
    L = hip.lib()
    ws = hip.Buffer(L.mle_norm_ws_bytes(batch, channels, hw, groups))
    gx, gy, gst = B(hip, x), hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
    hip.call("mle_norm_fwd", None, gx.ptr, gy.ptr, gst.ptr, batch, channels, hw, groups, 1e-5, ws.ptr, ws.nbytes)
    assert_close(gy.numpy(), yr, what="norm fwd", **EW)
    assert_close(gst.numpy(), st, what="norm stats", **EW)
    gyr, gdy, gdx, gstr = B(hip, yr), B(hip, dy), B(hip, dx0), B(hip, st)
    hip.call("mle_norm_bwd", None, gyr.ptr, gdy.ptr, gdx.ptr, gstr.ptr, batch, channels, hw, groups, 1e-5, 1,
             ws.ptr, ws.nbytes, 1)
    assert_close(gdx.numpy(), dxr, what="norm bwd", **EW)
    dxz = np.zeros_like(x)
    orc.call("orc_norm_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(dxz), orc.ptr(st), batch, channels, hw, groups, 1e-5, 1)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), x.size)
    hip.call("mle_norm_bwd", None, gyr.ptr, gdy.ptr, gdx.ptr, gstr.ptr, batch, channels, hw, groups, 1e-5, 1,
             ws.ptr, ws.nbytes, 0)
    assert_close(gdx.numpy(), dxz, what="norm bwd assign", **EW)
    # The statistics pass fused into the producer (residual Add: b of the same
    # size; MatPE: b one sample long, broadcast over the batch) gives the sum,
    # the statistics and the normalised output of add-then-normalise bit for bit.
    total = x.size
    for period in (total, channels * hw):
        a = r.standard_normal(shape, dtype=np.float32)
        bvec = r.standard_normal(period, dtype=np.float32)
        ga, gb = B(hip, a), B(hip, bvec)
        want_s = (a.reshape(-1, period) + bvec).reshape(shape).astype(np.float32)
        gs1, gy1, gst1 = B(hip, want_s), hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
        hip.call("mle_norm_fwd", None, gs1.ptr, gy1.ptr, gst1.ptr, batch, channels, hw, groups, 1e-5, ws.ptr,
                 ws.nbytes)
        gs2, gy2, gst2 = hip.Buffer.zeros(shape), hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
        hip.call("mle_add_norm_partials", None, ga.ptr, gb.ptr, period, gs2.ptr, batch, channels, hw, groups, ws.ptr,
                 ws.nbytes)
        hip.call("mle_norm_fwd_ex", None, gs2.ptr, gy2.ptr, gst2.ptr, batch, channels, hw, groups, 1e-5, ws.ptr,
                 ws.nbytes, 1)
        np.testing.assert_array_equal(gs2.numpy().view(np.uint32), want_s.view(np.uint32))
        np.testing.assert_array_equal(gst2.numpy().view(np.uint32), gst1.numpy().view(np.uint32))
        np.testing.assert_array_equal(gy2.numpy().view(np.uint32), gy1.numpy().view(np.uint32))


@pytest.mark.parametrize("batch,channels,hw,groups", [(2, 64, 4096, 32), (2, 8, 700, 4), (2, 3, 33, 1),
                                                     (3, 128, 4096, 32), (2, 6, 100, 3)])
@pytest.mark.parametrize("kind", [2, 1, 0])  # MLE_SILU, MLE_GELU, MLE_RELU
def test_norm_act_fused(hip, batch, channels, hw, groups, kind):
    """GroupNorm -> activation in one pass each way (mle_norm_fwd_act,
    mle_norm_bwd_act) gives the bits of the normalisation and activation
    kernels run one after the other, assigning and adding the normalisation's
    output gradient."""
    r = rng(batch * 7 + channels + hw + kind)
    shape = (batch, channels, hw)
    n = batch * channels * hw
    x = (r.standard_normal(shape, dtype=np.float32) * 2 + 0.5).astype(np.float32)
    da = r.standard_normal(shape, dtype=np.float32)
    dy0 = r.standard_normal(shape, dtype=np.float32)
    dx0 = r.standard_normal(shape, dtype=np.float32)
    L = hip.lib()
    ws = hip.Buffer(L.mle_norm_ws_bytes(batch, channels, hw, groups))
    gx = B(hip, x)
    y1, a1, st1 = hip.Buffer.zeros(shape), hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
    hip.call("mle_norm_fwd", None, gx.ptr, y1.ptr, st1.ptr, batch, channels, hw, groups, 1e-5, ws.ptr, ws.nbytes)
    hip.call("mle_act_fwd", None, kind, y1.ptr, a1.ptr, n)
    y2, a2, st2 = hip.Buffer.zeros(shape), hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
    hip.call("mle_norm_fwd_act", None, gx.ptr, y2.ptr, a2.ptr, kind, st2.ptr, batch, channels, hw, groups, 1e-5,
             ws.ptr, ws.nbytes, 0)
    for u, v in ((y1, y2), (a1, a2), (st1, st2)):
        np.testing.assert_array_equal(v.numpy().view(np.uint32), u.numpy().view(np.uint32))
    if hw % 4 == 0:
        # with the broadcast channel add after the activation (GroupNorm ->
        # SiLU -> Broadcast_Channel): the bits of mle_broadcast_channel_add
        # over the activation's output
        cb = r.standard_normal(channels, dtype=np.float32)
        gcb = B(hip, cb)
        h1 = hip.Buffer.zeros(shape)
        hip.call("mle_broadcast_channel_add", None, a1.ptr, gcb.ptr, h1.ptr, batch, channels, hw)
        y3, st3 = hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
        h3 = B(hip, np.full(shape, np.nan, np.float32))
        hip.call("mle_norm_fwd_act_bias", None, gx.ptr, y3.ptr, h3.ptr, kind, gcb.ptr, st3.ptr, batch, channels, hw,
                 groups, 1e-5, ws.ptr, ws.nbytes, 0)
        for u, v in ((y1, y3), (h1, h3), (st1, st3)):
            np.testing.assert_array_equal(v.numpy().view(np.uint32), u.numpy().view(np.uint32))
    gda = B(hip, da)
    for acc_dy in (0, 1):
        dy1, dx1 = B(hip, dy0), B(hip, dx0)
        hip.call("mle_act_bwd", None, kind, y1.ptr, gda.ptr, dy1.ptr, n, acc_dy)
        hip.call("mle_norm_bwd", None, y1.ptr, dy1.ptr, dx1.ptr, st1.ptr, batch, channels, hw, groups, 1e-5, 1,
                 ws.ptr, ws.nbytes, 1)
        dy2, dx2 = B(hip, dy0 if acc_dy else np.full(shape, np.nan, np.float32)), B(hip, dx0)
        hip.call("mle_norm_bwd_act", None, y1.ptr, gda.ptr, kind, dy2.ptr, acc_dy, dx2.ptr, st1.ptr, batch, channels,
                 hw, groups, 1e-5, 1, ws.ptr, ws.nbytes, 1)
        np.testing.assert_array_equal(dy2.numpy().view(np.uint32), dy1.numpy().view(np.uint32))
        np.testing.assert_array_equal(dx2.numpy().view(np.uint32), dx1.numpy().view(np.uint32))


@pytest.mark.parametrize("batch,channels,hw,groups,layout", [
    (4, 1, 256 * 64, 1, 1),   # LayerNorm over a [seq x d] sample, vector path
    (3, 1, 4099, 1, 1),       # ragged, scalar path
    (2, 8, 144, 4, 1),        # GroupNorm
    (2, 3, 50, 1, 1),         # LayerNorm with C > 1 under the reference's guard (only batch*hw elements)
])
def test_norm_bwd_apply_add(hip, batch, channels, hw, groups, layout):
    """The normalisation backward split in two passes, the second writing the
    producing Add's gradient and both of its inputs' (mle_norm_bwd_partials +
    mle_norm_bwd_apply_add), gives the bits of mle_norm_bwd followed by the
    Add's backward (mle_accumulate2) -- every assign / add combination, and
    with the second input absent."""
    r = rng(batch * 5 + channels + hw + groups)
    shape = (batch, channels, hw)
    n = batch * channels * hw
    x = (r.standard_normal(shape, dtype=np.float32) * 2 + 0.5).astype(np.float32)
    dy = r.standard_normal(shape, dtype=np.float32)
    g0, a0, b0 = (r.standard_normal(shape, dtype=np.float32) for _ in range(3))
    L = hip.lib()
    ws = hip.Buffer(L.mle_norm_ws_bytes(batch, channels, hw, groups))
    gx, gdy = B(hip, x), B(hip, dy)
    y, st = hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
    hip.call("mle_norm_fwd", None, gx.ptr, y.ptr, st.ptr, batch, channels, hw, groups, 1e-5, ws.ptr, ws.nbytes)
    nan = np.full(shape, np.nan, np.float32)
    for acc, acc_a, acc_b in ((0, 0, 0), (1, 1, 1), (0, 1, 0), (1, 0, 1)):
        g1, a1, b1 = B(hip, g0 if acc else nan), B(hip, a0), B(hip, b0)
        hip.call("mle_norm_bwd", None, y.ptr, gdy.ptr, g1.ptr, st.ptr, batch, channels, hw, groups, 1e-5, layout,
                 ws.ptr, ws.nbytes, acc)
        hip.call("mle_accumulate2", None, g1.ptr, a1.ptr, acc_a, b1.ptr, acc_b, n)
        g2, a2, b2 = B(hip, g0 if acc else nan), B(hip, a0 if acc_a else nan), B(hip, b0 if acc_b else nan)
        hip.call("mle_norm_bwd_partials", None, y.ptr, gdy.ptr, None, -1, 0, batch, channels, hw, groups, layout, ws.ptr,
                 ws.nbytes)
        hip.call("mle_norm_bwd_apply_add", None, y.ptr, gdy.ptr, g2.ptr, acc, None, a2.ptr, acc_a, b2.ptr, acc_b,
                 st.ptr, batch, channels, hw, groups, 1e-5, layout, ws.ptr, ws.nbytes)
        for want, got, what in ((g1, g2, "own"), (a1, a2, "a"), (b1, b2, "b")):
            np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32),
                                          err_msg=f"{what} acc={acc},{acc_a},{acc_b}")
        if acc:  # the same with the values added to held in another buffer (dx_in), dx written whole
            gin, g5 = B(hip, g0), B(hip, nan)
            a5, b5 = B(hip, a0 if acc_a else nan), B(hip, b0 if acc_b else nan)
            hip.call("mle_norm_bwd_apply_add", None, y.ptr, gdy.ptr, g5.ptr, 1, gin.ptr, a5.ptr, acc_a, b5.ptr, acc_b,
                     st.ptr, batch, channels, hw, groups, 1e-5, layout, ws.ptr, ws.nbytes)
            for want, got, what in ((g1, g5, "own"), (a1, a5, "a"), (b1, b5, "b")):
                np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32),
                                              err_msg=f"{what} from dx_in, acc={acc_a},{acc_b}")
            np.testing.assert_array_equal(gin.numpy().view(np.uint32), g0.view(np.uint32), err_msg="dx_in read only")
    # one input only
    g3, a3 = B(hip, nan), B(hip, a0)
    hip.call("mle_norm_bwd_partials", None, y.ptr, gdy.ptr, None, -1, 0, batch, channels, hw, groups, layout, ws.ptr,
                 ws.nbytes)
    hip.call("mle_norm_bwd_apply_add", None, y.ptr, gdy.ptr, g3.ptr, 0, None, a3.ptr, 1, None, 0, st.ptr, batch,
             channels, hw, groups, 1e-5, layout, ws.ptr, ws.nbytes)
    g4 = B(hip, nan)
    hip.call("mle_norm_bwd", None, y.ptr, gdy.ptr, g4.ptr, st.ptr, batch, channels, hw, groups, 1e-5, layout,
             ws.ptr, ws.nbytes, 0)
    np.testing.assert_array_equal(g3.numpy().view(np.uint32), g4.numpy().view(np.uint32))
    np.testing.assert_array_equal(a3.numpy().view(np.uint32), (a0 + g4.numpy()).view(np.uint32))
    with pytest.raises(hip.MLEError):  # the destinations must differ
        hip.call("mle_norm_bwd_apply_add", None, y.ptr, gdy.ptr, g3.ptr, 0, None, g3.ptr, 0, None, 0, st.ptr, batch,
                 channels, hw, groups, 1e-5, layout, ws.ptr, ws.nbytes)
    with pytest.raises(hip.MLEError):  # and dx_in is no destination
        hip.call("mle_norm_bwd_apply_add", None, y.ptr, gdy.ptr, g3.ptr, 1, a3.ptr, a3.ptr, 1, None, 0, st.ptr, batch,
                 channels, hw, groups, 1e-5, layout, ws.ptr, ws.nbytes)


@pytest.mark.parametrize("batch,channels,hw,groups", [(2, 8, 144, 4), (2, 16, 64 * 64, 8)])
def test_norm_bwd_act_apply_add(hip, batch, channels, hw, groups):
    """GroupNorm -> SiLU backward in two passes, the second writing the
    producer's gradient and one input's (as after a MatPE): the bits of
    mle_norm_bwd_act followed by the producer's gradient copy at scale 1, for
    every assign / add combination."""
    r = rng(batch * 11 + channels + hw)
    shape = (batch, channels, hw)
    n = batch * channels * hw
    x = (r.standard_normal(shape, dtype=np.float32) * 2 - 0.3).astype(np.float32)
    da = r.standard_normal(shape, dtype=np.float32)
    dy0, g0, a0 = (r.standard_normal(shape, dtype=np.float32) for _ in range(3))
    L = hip.lib()
    ws = hip.Buffer(L.mle_norm_ws_bytes(batch, channels, hw, groups))
    gx, gda = B(hip, x), B(hip, da)
    y, st = hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * batch * groups)
    hip.call("mle_norm_fwd", None, gx.ptr, y.ptr, st.ptr, batch, channels, hw, groups, 1e-5, ws.ptr, ws.nbytes)
    nan = np.full(shape, np.nan, np.float32)
    silu = 2
    for acc_dy, acc, acc_a in ((0, 0, 0), (1, 1, 1), (0, 1, 0), (1, 0, 1)):
        dy1, g1, a1 = B(hip, dy0 if acc_dy else nan), B(hip, g0 if acc else nan), B(hip, a0)
        hip.call("mle_norm_bwd_act", None, y.ptr, gda.ptr, silu, dy1.ptr, acc_dy, g1.ptr, st.ptr, batch, channels, hw,
                 groups, 1e-5, 1, ws.ptr, ws.nbytes, acc)
        hip.call("mle_accumulate" if acc_a else "mle_scale_assign", None, g1.ptr, a1.ptr, 1.0, n)
        dy2, g2, a2 = (B(hip, dy0 if acc_dy else nan), B(hip, g0 if acc else nan), B(hip, a0 if acc_a else nan))
        hip.call("mle_norm_bwd_partials", None, y.ptr, dy2.ptr, gda.ptr, silu, acc_dy, batch, channels, hw, groups, 1,
                 ws.ptr, ws.nbytes)
        hip.call("mle_norm_bwd_apply_add", None, y.ptr, dy2.ptr, g2.ptr, acc, None, a2.ptr, acc_a, None, 0, st.ptr,
                 batch, channels, hw, groups, 1e-5, 1, ws.ptr, ws.nbytes)
        for want, got, what in ((dy1, dy2, "dy"), (g1, g2, "own"), (a1, a2, "a")):
            np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32),
                                          err_msg=f"{what} acc={acc_dy},{acc},{acc_a}")


@pytest.mark.parametrize("batch,channels,hw", [(4, 3, 25), (16, 128, 64 * 64), (3, 5, 4099), (1, 1, 9000)])
def test_batchnorm(hip, orc, batch, channels, hw):
    r = rng(batch * 3 + channels + hw)
    shape = (batch, channels, hw)
    x = (r.standard_normal(shape, dtype=np.float32) * 1.5 - 0.3).astype(np.float32)
    dy = r.standard_normal(shape, dtype=np.float32)
    dx0 = r.standard_normal(shape, dtype=np.float32)
    yr, st = np.zeros_like(x), np.zeros(2 * channels, np.float32)
    orc.call("orc_batchnorm_fwd", orc.ptr(x), orc.ptr(yr), orc.ptr(st), batch, channels, hw, 1e-5)
    dxr = dx0.copy()
    orc.call("orc_batchnorm_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(dxr), orc.ptr(st), batch, channels, hw, 1e-5)
    ws = hip.Buffer(hip.lib().mle_batchnorm_ws_bytes(batch, channels, hw))
    gx, gy, gst = B(hip, x), hip.Buffer.zeros(shape), hip.Buffer.zeros(2 * channels)
    hip.call("mle_batchnorm_fwd", None, gx.ptr, gy.ptr, gst.ptr, batch, channels, hw, 1e-5, ws.ptr, ws.nbytes)
    assert_close(gy.numpy(), yr, what="batchnorm fwd", **EW)
    assert_close(gst.numpy(), st, what="batchnorm stats", **EW)
    gyr, gdy, gdx, gstr = B(hip, yr), B(hip, dy), B(hip, dx0), B(hip, st)
    hip.call("mle_batchnorm_bwd", None, gyr.ptr, gdy.ptr, gdx.ptr, gstr.ptr, batch, channels, hw, 1e-5, ws.ptr,
             ws.nbytes, 1)
    assert_close(gdx.numpy(), dxr, what="batchnorm bwd", **EW)
    dxz = np.zeros_like(x)
    orc.call("orc_batchnorm_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(dxz), orc.ptr(st), batch, channels, hw, 1e-5)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), x.size)
    hip.call("mle_batchnorm_bwd", None, gyr.ptr, gdy.ptr, gdx.ptr, gstr.ptr, batch, channels, hw, 1e-5, ws.ptr,
             ws.nbytes, 0)
    assert_close(gdx.numpy(), dxz, what="batchnorm bwd assign", **EW)


@pytest.mark.parametrize("bc,rows,cols", [(3, 7, 9), (4, 64, 1000), (2, 300, 33), (16, 64, 64)])
@pytest.mark.parametrize("type_", [0, 1])
def test_rmsnorm(hip, orc, bc, rows, cols, type_):
    r = rng(bc + rows * 3 + cols + type_)
    shape = (bc, rows, cols)
    x = r.standard_normal(shape, dtype=np.float32)
    dy = r.standard_normal(shape, dtype=np.float32)
    dx0 = r.standard_normal(shape, dtype=np.float32)
    nl = bc * (rows if type_ == 0 else cols)
    yr, nr = np.zeros_like(x), np.zeros(nl, np.float32)
    orc.call("orc_rmsnorm_fwd", orc.ptr(x), orc.ptr(yr), orc.ptr(nr), bc, rows, cols, type_)
    dxr = dx0.copy()
    orc.call("orc_rmsnorm_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(nr), orc.ptr(dxr), bc, rows, cols, type_)
    gx, gy, gn = B(hip, x), hip.Buffer.zeros(shape), hip.Buffer.zeros(nl)
    hip.call("mle_rmsnorm_fwd", None, gx.ptr, gy.ptr, gn.ptr, bc, rows, cols, type_)
    assert_close(gy.numpy(), yr, what="rmsnorm fwd", **EW)
    assert_close(gn.numpy(), nr, what="rmsnorm norms", **EW)
    gyr, gdy, gnr, gdx = B(hip, yr), B(hip, dy), B(hip, nr), B(hip, dx0)
    hip.call("mle_rmsnorm_bwd", None, gyr.ptr, gdy.ptr, gnr.ptr, gdx.ptr, bc, rows, cols, type_, 1)
    assert_close(gdx.numpy(), dxr, what="rmsnorm bwd", **EW)
    dxz = np.zeros_like(x)
    orc.call("orc_rmsnorm_bwd", orc.ptr(yr), orc.ptr(dy), orc.ptr(nr), orc.ptr(dxz), bc, rows, cols, type_)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), x.size)
    hip.call("mle_rmsnorm_bwd", None, gyr.ptr, gdy.ptr, gnr.ptr, gdx.ptr, bc, rows, cols, type_, 0)
    assert_close(gdx.numpy(), dxz, what="rmsnorm bwd assign", **EW)


@pytest.mark.parametrize("batch,c1,h1,w1,c2,h,w", [(2, 3, 8, 10, 2, 5, 6), (2, 4, 6, 6, 5, 6, 6),
                                                   (1, 64, 68, 68, 64, 56, 56), (3, 1, 9, 7, 2, 4, 3)])
def test_copy_crop(hip, orc, batch, c1, h1, w1, c2, h, w):
    """Pure data movement: bit-exact against the oracle, both accumulate modes."""
    r = rng(batch + c1 + h1 + w1 + c2)
    x1 = r.standard_normal((batch, c1, h1, w1), dtype=np.float32)
    x2 = r.standard_normal((batch, c2, h, w), dtype=np.float32)
    yr = np.zeros((batch, c1 + c2, h, w), np.float32)
    orc.call("orc_copy_crop_fwd", orc.ptr(x1), orc.ptr(x2), orc.ptr(yr), batch, c1, h1, w1, c2, h, w)
    g1, g2, gy = B(hip, x1), B(hip, x2), hip.Buffer.zeros(yr.shape)
    hip.call("mle_copy_crop_fwd", None, g1.ptr, g2.ptr, gy.ptr, batch, c1, h1, w1, c2, h, w)
    np.testing.assert_array_equal(gy.numpy(), yr)
    dy = r.standard_normal(yr.shape, dtype=np.float32)
    d1, d2 = r.standard_normal(x1.shape, dtype=np.float32), r.standard_normal(x2.shape, dtype=np.float32)
    r1, r2 = d1.copy(), d2.copy()
    orc.call("orc_copy_crop_bwd", orc.ptr(dy), orc.ptr(r1), orc.ptr(r2), batch, c1, h1, w1, c2, h, w)
    gdy, gd1, gd2 = B(hip, dy), B(hip, d1), B(hip, d2)
    hip.call("mle_copy_crop_bwd", None, gdy.ptr, gd1.ptr, gd2.ptr, batch, c1, h1, w1, c2, h, w, 1, 1)
    np.testing.assert_array_equal(gd1.numpy(), r1)
    np.testing.assert_array_equal(gd2.numpy(), r2)
    z1, z2 = np.zeros_like(x1), np.zeros_like(x2)
    orc.call("orc_copy_crop_bwd", orc.ptr(dy), orc.ptr(z1), orc.ptr(z2), batch, c1, h1, w1, c2, h, w)
    hip.call("mle_fill", None, gd1.ptr, float("nan"), x1.size)
    hip.call("mle_fill", None, gd2.ptr, float("nan"), x2.size)
    hip.call("mle_copy_crop_bwd", None, gdy.ptr, gd1.ptr, gd2.ptr, batch, c1, h1, w1, c2, h, w, 0, 0)
    np.testing.assert_array_equal(gd1.numpy(), z1)
    np.testing.assert_array_equal(gd2.numpy(), z2)


def test_copy_crop_rejects_padding_direction(hip):
    g = hip.Buffer.zeros(64)
    with pytest.raises(hip.MLEError):
        hip.call("mle_copy_crop_fwd", None, g.ptr, g.ptr, g.ptr, 1, 1, 3, 3, 1, 4, 4)


@pytest.mark.parametrize("n,cin,h,w,cout,k,pad,stride", [(2, 3, 5, 4, 4, 2, 0, 2), (2, 8, 7, 7, 6, 3, 1, 1),
                                                        (1, 4, 6, 5, 3, 3, 1, 2), (2, 16, 16, 16, 8, 4, 1, 2),
                                                        (4, 128, 32, 32, 64, 2, 0, 2)])
def test_conv_transpose_composition(hip, orc, n, cin, h, w, cout, k, pad, stride):
    """Convolute2DT's kernels: swapped weights + convolution dgrad (forward),
    forward (input gradient) and wgrad (weight gradient), against the oracle's
    restatement of CVT2D / CVT2D_GradInput / GVT2D."""
    r = rng(n + cin * 3 + h + cout + k + stride)
    oh, ow = (h - 1) * stride - 2 * pad + k, (w - 1) * stride - 2 * pad + k
    x = r.standard_normal((n, cin, h, w), dtype=np.float32)
    wt = r.standard_normal((cout, cin, k, k), dtype=np.float32)
    b = r.standard_normal(cout, dtype=np.float32)
    dy = r.standard_normal((n, cout, oh, ow), dtype=np.float32)
    yr = np.zeros((n, cout, oh, ow), np.float32)
    orc.call("orc_convT_fwd", orc.ptr(x), orc.ptr(wt), orc.ptr(b), orc.ptr(yr), n, cin, h, w, cout, k, k, pad, stride)
    dxr, dwr = np.zeros_like(x), np.zeros_like(wt)
    orc.call("orc_convT_dgrad", orc.ptr(dy), orc.ptr(wt), orc.ptr(dxr), n, cin, h, w, cout, k, k, pad, stride)
    orc.call("orc_convT_wgrad", orc.ptr(x), orc.ptr(dy), orc.ptr(dwr), n, cin, h, w, cout, k, k, pad, stride)
    gx, gw, gb, gdy = B(hip, x), B(hip, wt), B(hip, b), B(hip, dy)
    gsw, gy = hip.Buffer.zeros((cin, cout, k, k)), hip.Buffer.zeros(yr.shape)
    hip.call("mle_weight_swap", None, gw.ptr, gsw.ptr, cout, cin, k * k, 0)
    np.testing.assert_array_equal(gsw.numpy(), wt.transpose(1, 0, 2, 3))
    hip.call("mle_fill", None, gy.ptr, float("nan"), yr.size)
    hip.call("mle_conv2d_dgrad", None, gx.ptr, gsw.ptr, gy.ptr, n, cout, oh, ow, cin, k, k, pad, stride, 0)
    hip.call("mle_broadcast_channel_add", None, gy.ptr, gb.ptr, gy.ptr, n, cout, oh * ow)
    assert_close(gy.numpy(), yr, what="convT fwd", **MM)
    gdx = hip.Buffer.zeros(x.shape)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), x.size)
    hip.call("mle_conv2d_fwd", None, gdy.ptr, gsw.ptr, None, gdx.ptr, n, cout, oh, ow, cin, k, k, pad, stride)
    assert_close(gdx.numpy(), dxr, what="convT input gradient", **MM)
    L = hip.lib()
    ws = hip.Buffer(max(1, L.mle_conv2d_wgrad_ws_bytes(n, cout, oh, ow, cin, k, k, pad, stride)))
    gdw_s, gdw = hip.Buffer.zeros((cin, cout, k, k)), hip.Buffer.zeros(wt.shape)
    hip.call("mle_conv2d_wgrad", None, gdy.ptr, gx.ptr, gdw_s.ptr, n, cout, oh, ow, cin, k, k, pad, stride, ws.ptr,
             ws.nbytes)
    hip.call("mle_weight_swap", None, gdw_s.ptr, gdw.ptr, cin, cout, k * k, 0)
    assert_close(gdw.numpy(), dwr, what="convT weight gradient", **MM)


# ------------------------------------------- paired 3 x 3 + 1 x 1 convolution
@pytest.mark.parametrize("n,cin,h,w,cout3,cout1", [
    (2, 64, 64, 64, 128, 128),   # the C5 residual block's conv1 + skip at batch 2
    (2, 8, 12, 12, 16, 16),      # W not dividing 64: the 3 x 3 halo loads
    (3, 16, 8, 8, 32, 48),       # M <= 64 row blocks, images straddling a tile
    (2, 128, 16, 16, 64, 128),   # 128 input channels: dgrad row blocks of 128
    (1, 24, 20, 20, 136, 72),    # rows past M, uneven tile counts (not multiples of 8)
])
def test_conv_pair(hip, orc, n, cin, h, w, cout3, cout1):
    """A 3 x 3 (pad 1) and a 1 x 1 (pad 0) convolution of one input in one
    launch: both forwards (with biases), and the input gradient
    dx (+)= dgrad3(dy3) + dgrad1(dy1) with the 1 x 1 product as extra K stages
    of the 3 x 3 tiles, assigning and adding, against the oracle's separate
    CV2D / CV2D_GradInput passes."""
    r = rng(n + cin + h + cout3 + cout1)
    L = hip.lib()
    assert L.mle_conv2d_pair_supported(n, cin, h, w, cout3, cout1) == 1
    x = r.standard_normal((n, cin, h, w), dtype=np.float32)
    w3 = r.standard_normal((cout3, cin, 3, 3), dtype=np.float32)
    b3 = r.standard_normal(cout3, dtype=np.float32)
    w1 = r.standard_normal((cout1, cin, 1, 1), dtype=np.float32)
    b1 = r.standard_normal(cout1, dtype=np.float32)
    dy3 = r.standard_normal((n, cout3, h, w), dtype=np.float32)
    dy1 = r.standard_normal((n, cout1, h, w), dtype=np.float32)
    dx0 = r.standard_normal(x.shape, dtype=np.float32)
    y3r, y1r = np.zeros((n, cout3, h, w), np.float32), np.zeros((n, cout1, h, w), np.float32)
    orc.call("orc_conv_fwd", orc.ptr(x), orc.ptr(w3), orc.ptr(b3), orc.ptr(y3r), n, cin, h, w, cout3, 3, 3, 1, 1)
    orc.call("orc_conv_fwd", orc.ptr(x), orc.ptr(w1), orc.ptr(b1), orc.ptr(y1r), n, cin, h, w, cout1, 1, 1, 0, 1)
    gx, gw3, gb3, gw1, gb1 = B(hip, x), B(hip, w3), B(hip, b3), B(hip, w1), B(hip, b1)
    gy3 = B(hip, np.full(y3r.shape, np.nan, np.float32))
    gy1 = B(hip, np.full(y1r.shape, np.nan, np.float32))
    hip.call("mle_conv2d_pair_fwd", None, gx.ptr, n, cin, h, w, gw3.ptr, gb3.ptr, gy3.ptr, cout3, gw1.ptr, gb1.ptr,
             gy1.ptr, cout1)
    assert_close(gy3.numpy(), y3r, what="pair fwd 3x3", **MM)
    assert_close(gy1.numpy(), y1r, what="pair fwd 1x1", **MM)
    # the same bits as the per-convolution launches
    gs3, gs1 = hip.Buffer.zeros(y3r.shape), hip.Buffer.zeros(y1r.shape)
    hip.call("mle_conv2d_fwd", None, gx.ptr, gw3.ptr, gb3.ptr, gs3.ptr, n, cin, h, w, cout3, 3, 3, 1, 1)
    hip.call("mle_conv2d_fwd", None, gx.ptr, gw1.ptr, gb1.ptr, gs1.ptr, n, cin, h, w, cout1, 1, 1, 0, 1)
    np.testing.assert_array_equal(gy3.numpy(), gs3.numpy())
    np.testing.assert_array_equal(gy1.numpy(), gs1.numpy())
    gdy3, gdy1 = B(hip, dy3), B(hip, dy1)
    for acc in (1, 0):
        dxr = dx0.copy() if acc else np.zeros_like(x)
        orc.call("orc_conv_dgrad", orc.ptr(dy3), orc.ptr(w3), orc.ptr(dxr), n, cin, h, w, cout3, 3, 3, 1, 1)
        orc.call("orc_conv_dgrad", orc.ptr(dy1), orc.ptr(w1), orc.ptr(dxr), n, cin, h, w, cout1, 1, 1, 0, 1)
        gdx = B(hip, dx0 if acc else np.full(x.shape, np.nan, np.float32))
        hip.call("mle_conv2d_pair_dgrad", None, gdx.ptr, acc, n, cin, h, w, gdy3.ptr, gw3.ptr, cout3, gdy1.ptr, gw1.ptr,
                 cout1)
        assert_close(gdx.numpy(), dxr, what=f"pair dgrad acc={acc}", **MM)
    # shapes off the direct kernels are refused, not computed elsewhere
    assert L.mle_conv2d_pair_supported(n, cin, h, w + 1, cout3, cout1) == 0


# ---------------------------------------------------------------------- conv
@pytest.mark.parametrize("n,cin,h,w,cout,k,pad,stride", [
    (2, 3, 9, 9, 5, 3, 1, 1), (2, 4, 8, 10, 6, 1, 0, 1), (1, 3, 11, 11, 4, 3, 1, 2),
    (2, 16, 16, 16, 32, 3, 1, 1), (1, 8, 7, 7, 8, 5, 0, 1),
    # stride-1 3x3 / 1x1 fast path: two row tiles (cout 130), images straddling
    # a K stage (36 pixels), pad 0 (output smaller than input), multi-stage K
    (3, 20, 6, 6, 130, 3, 1, 1), (2, 8, 12, 12, 16, 3, 0, 1), (4, 64, 16, 16, 128, 3, 1, 1),
    (2, 32, 8, 8, 64, 1, 0, 1),
    # register-direct 3x3 path (stride 1, pad 1, W % 4 == 0): W dividing 64
    # (4, 8, 16, 64), W needing the lane-0 / lane-15 halo loads (12, 20, 128),
    # images straddling a 64-pixel lane row (hw 60, 140), partial pixel tiles,
    # 64-row and 128-row channel tiles with partial rows (72, 40); the weight
    # gradient's pixel splits carry rows and images (W >= 16)
    (3, 8, 4, 4, 8, 3, 1, 1), (2, 24, 8, 8, 40, 3, 1, 1), (2, 8, 5, 12, 16, 3, 1, 1),
    (2, 16, 7, 20, 24, 3, 1, 1), (1, 16, 3, 128, 72, 3, 1, 1), (2, 64, 64, 64, 128, 3, 1, 1),
    (1, 8, 4, 16, 8, 3, 1, 1),  # one pixel split: the weight gradient is written without partials
    # register-direct 1x1 path (stride 1, pad 0): 128-row and 64-row (two-wave
    # K split) blocks, partial pixel tiles and channel groups (hw 60, cin 12,
    # cout 20), a 4-pixel image (weight gradient on the LDS kernel)
    (2, 64, 32, 32, 128, 1, 0, 1), (3, 12, 5, 12, 20, 1, 0, 1), (1, 8, 2, 2, 8, 1, 0, 1),
    # 1x1 weight-gradient wave layouts (row blocks x column blocks x pixel
    # shares): 1x2x2 (cin 100), 1x4x1 (cin 200), 2x2x1 (cin 96); one 16-pixel
    # stage shared by four waves, three of them with no pixels
    (2, 100, 6, 8, 48, 1, 0, 1), (1, 200, 4, 8, 32, 1, 0, 1), (2, 96, 4, 8, 96, 1, 0, 1),
    (1, 12, 4, 4, 20, 1, 0, 1),
])
def test_conv(hip, orc, n, cin, h, w, cout, k, pad, stride):
    r = rng(n * 7 + cin + h + cout + k)
    oh = (2 * pad + h - k) // stride + 1
    ow = (2 * pad + w - k) // stride + 1
    x = r.standard_normal((n, cin, h, w), dtype=np.float32)
    wt = r.standard_normal((cout, cin, k, k), dtype=np.float32)
    b = r.standard_normal(cout, dtype=np.float32)
    dy = r.standard_normal((n, cout, oh, ow), dtype=np.float32)
    dx0 = r.standard_normal(x.shape, dtype=np.float32)
    yr = np.zeros((n, cout, oh, ow), np.float32)
    orc.call("orc_conv_fwd", orc.ptr(x), orc.ptr(wt), orc.ptr(b), orc.ptr(yr), n, cin, h, w, cout, k, k, pad, stride)
    dxr = dx0.copy()
    orc.call("orc_conv_dgrad", orc.ptr(dy), orc.ptr(wt), orc.ptr(dxr), n, cin, h, w, cout, k, k, pad, stride)
    dwr = np.zeros_like(wt)
    orc.call("orc_conv_wgrad", orc.ptr(x), orc.ptr(dy), orc.ptr(dwr), n, cin, h, w, cout, k, k, pad, stride)
    gx, gw, gb, gy = B(hip, x), B(hip, wt), B(hip, b), hip.Buffer.zeros(yr.shape)
    hip.call("mle_conv2d_fwd", None, gx.ptr, gw.ptr, gb.ptr, gy.ptr, n, cin, h, w, cout, k, k, pad, stride)
    assert_close(gy.numpy(), yr, what="conv fwd", **MM)
    # no bias: the oracle's sums with a zero bias
    yr0 = np.zeros_like(yr)
    orc.call("orc_conv_fwd", orc.ptr(x), orc.ptr(wt), orc.ptr(np.zeros_like(b)), orc.ptr(yr0), n, cin, h, w, cout, k,
             k, pad, stride)
    gy0 = B(hip, np.full(yr.shape, np.nan, np.float32))
    hip.call("mle_conv2d_fwd", None, gx.ptr, gw.ptr, None, gy0.ptr, n, cin, h, w, cout, k, k, pad, stride)
    assert_close(gy0.numpy(), yr0, what="conv fwd without bias", **MM)
    gdy, gdx = B(hip, dy), B(hip, dx0)
    hip.call("mle_conv2d_dgrad", None, gdy.ptr, gw.ptr, gdx.ptr, n, cin, h, w, cout, k, k, pad, stride, 1)
    assert_close(gdx.numpy(), dxr, what="conv dgrad", **MM)
    dxz = np.zeros_like(x)
    orc.call("orc_conv_dgrad", orc.ptr(dy), orc.ptr(wt), orc.ptr(dxz), n, cin, h, w, cout, k, k, pad, stride)
    hip.call("mle_fill", None, gdx.ptr, float("nan"), x.size)
    hip.call("mle_conv2d_dgrad", None, gdy.ptr, gw.ptr, gdx.ptr, n, cin, h, w, cout, k, k, pad, stride, 0)
    assert_close(gdx.numpy(), dxz, what="conv dgrad assign", **MM)
    L = hip.lib()
    ws = hip.Buffer(L.mle_conv2d_wgrad_ws_bytes(n, cin, h, w, cout, k, k, pad, stride))
    gdw = B(hip, np.full(wt.shape, 7.0, np.float32))  # wgrad assigns
    hip.call("mle_conv2d_wgrad", None, gx.ptr, gdy.ptr, gdw.ptr, n, cin, h, w, cout, k, k, pad, stride, ws.ptr, ws.nbytes)
    assert_close(gdw.numpy(), dwr, what="conv wgrad", **MM)
    # The bias gradient taken inside the weight-gradient launch: dW the same
    # bits as above, db += the channel sums of dy (Channel_Squeeze1D).
    db0 = r.standard_normal(cout, dtype=np.float32)
    dbr = db0.copy()
    orc.call("orc_channel_squeeze", orc.ptr(dy), orc.ptr(dbr), n, cout, oh * ow, cout)
    gdw2, gdb = B(hip, np.full(wt.shape, -3.0, np.float32)), B(hip, db0)
    hip.call("mle_conv2d_wgrad_bias", None, gx.ptr, gdy.ptr, gdw2.ptr, gdb.ptr, 1, n, cin, h, w, cout, k, k, pad,
             stride, ws.ptr, ws.nbytes)
    np.testing.assert_array_equal(gdw2.numpy(), gdw.numpy())
    assert_close(gdb.numpy(), dbr, what="conv bias grad", **MM)  # a sum over n * oh * ow terms
    # accumulate_db 0: assigned over NaN, the bits of adding into zeros
    gdb0, gdbn = B(hip, np.zeros(cout, np.float32)), B(hip, np.full(cout, np.nan, np.float32))
    hip.call("mle_conv2d_wgrad_bias", None, gx.ptr, gdy.ptr, gdw2.ptr, gdb0.ptr, 1, n, cin, h, w, cout, k, k, pad,
             stride, ws.ptr, ws.nbytes)
    hip.call("mle_conv2d_wgrad_bias", None, gx.ptr, gdy.ptr, gdw2.ptr, gdbn.ptr, 0, n, cin, h, w, cout, k, k, pad,
             stride, ws.ptr, ws.nbytes)
    np.testing.assert_array_equal(gdbn.numpy(), gdb0.numpy())


# ----------------------------------------------------------------- optimizer
@pytest.mark.parametrize("adamw", [0, 1])
@pytest.mark.parametrize("t", [1, 7])
def test_adam(hip, orc, adamw, t):
    r = rng(20 + adamw + t)
    n = 100003
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    m = (r.standard_normal(n) * 1e-4).astype(np.float32)
    v = np.abs(r.standard_normal(n) * 1e-6).astype(np.float32)
    pr, mr, vr = p.copy(), m.copy(), v.copy()
    orc.call("orc_adam", orc.ptr(pr), orc.ptr(g), n, t, orc.ptr(mr), orc.ptr(vr), 0.9, 0.999, 1e-8, 0.01, 3e-4, adamw)
    gp, gg, gm, gv = B(hip, p), B(hip, g), B(hip, m), B(hip, v)
    hip.call("mle_adam_update", None, gp.ptr, gg.ptr, gm.ptr, gv.ptr, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01, adamw, None)
    assert_close(gm.numpy(), mr, what="m", **EW)
    assert_close(gv.numpy(), vr, what="v", **EW)
    assert_close(gp.numpy(), pr, what="p", **EW)


def test_sqnorm_and_fused_clip(hip, orc):
    r = rng(31)
    n = 1_000_003
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    g[r.random(n) < 0.01] *= 100.0
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    acc = np.zeros(1, np.float64)
    orc.call("orc_sumsq", orc.ptr(g), n, orc.ptr(acc))
    s = acc.copy()
    orc.call("orc_sqrt_scale", orc.ptr(s), 1.0)
    gc = g.copy()
    orc.call("orc_clip", orc.ptr(gc), n, orc.ptr(s))
    pr, mr, vr = p.copy(), m.copy(), v.copy()
    orc.call("orc_adam", orc.ptr(pr), orc.ptr(gc), n, 1, orc.ptr(mr), orc.ptr(vr), 0.9, 0.999, 1e-8, 0.01, 3e-4, 1)
    L = hip.lib()
    gg = B(hip, g)
    gacc = B(hip, np.array([0.5], np.float64))
    ws = hip.Buffer(L.mle_sqnorm_ws_bytes(n))
    hip.call("mle_grad_sqnorm", None, gg.ptr, n, gacc.ptr, None, ws.ptr, ws.nbytes)
    np.testing.assert_allclose(gacc.numpy(dtype=np.float64), acc + 0.5, rtol=1e-12)
    hip.call("mle_sqrt_scale", None, gacc.ptr, 1.0)
    gp, gm, gv, gnorm = B(hip, p), B(hip, m), B(hip, v), hip.Buffer.zeros(1, np.float64)
    ws2 = hip.Buffer(L.mle_adamw_clip_ws_bytes(n))
    hip.call("mle_adamw_clip_fused", None, gp.ptr, gg.ptr, gm.ptr, gv.ptr, n, 1, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1, 1.0,
             gnorm.ptr, ws2.ptr, ws2.nbytes)
    np.testing.assert_allclose(gnorm.numpy(dtype=np.float64), s, rtol=1e-12)
    assert_close(gm.numpy(), mr, what="m", **EW)
    assert_close(gv.numpy(), vr, what="v", **EW)
    assert_close(gp.numpy(), pr, what="p", **EW)
    np.testing.assert_array_equal(gg.numpy(), g)  # the fused path leaves g unclipped


@pytest.mark.parametrize("n", [1, 3, 4, 5, 255, 257, 2048 * 4 + 1, 1_000_003, 16_777_216 + 7])
@pytest.mark.parametrize("offset", [0, 1])
def test_sqnorm_shapes_and_sqrt_scale(hip, orc, n, offset):
    """The partial pass's contiguous per-workgroup ranges cover every element
    once, for vector (16-byte aligned) and scalar (offset by one float) data,
    with n % 4 tails and single-workgroup sizes; the sum is fixed-order (two
    calls give the same bits); the NaN / Inf flag; and mle_grad_sqnorm_ex's
    Sqrt_Scale in the finishing launch equals mle_sqrt_scale after the sum."""
    r = rng(32 + n % 97)
    g = (r.standard_normal(n) * 0.3).astype(np.float32)
    acc = np.zeros(1, np.float64)
    orc.call("orc_sumsq", orc.ptr(g), n, orc.ptr(acc))
    s_ref = acc.copy()
    orc.call("orc_sqrt_scale", orc.ptr(s_ref), 1.0)
    L = hip.lib()
    buf = hip.Buffer(4 * (n + 1))
    buf.upload(np.concatenate([np.zeros(offset, np.float32), g]))
    gptr = buf.ptr + 4 * offset
    ws = hip.Buffer(L.mle_sqnorm_ws_bytes(n))
    bad = hip.Buffer.zeros(1, np.int32)
    outs = []
    for _ in range(2):
        gacc = B(hip, np.array([0.25], np.float64))
        hip.call("mle_grad_sqnorm", None, gptr, n, gacc.ptr, bad.ptr, ws.ptr, ws.nbytes)
        outs.append(gacc.numpy(dtype=np.float64))
    np.testing.assert_allclose(outs[0], acc + 0.25, rtol=1e-12)
    np.testing.assert_array_equal(outs[0].view(np.uint64), outs[1].view(np.uint64))
    assert bad.numpy()[0] == 0
    gs = B(hip, np.array([0.0], np.float64))
    hip.call("mle_grad_sqnorm_ex", None, gptr, n, gs.ptr, None, 1, 1.0, ws.ptr, ws.nbytes)
    np.testing.assert_allclose(gs.numpy(dtype=np.float64), s_ref, rtol=1e-12)
    g2 = B(hip, np.array([0.0], np.float64))
    hip.call("mle_grad_sqnorm", None, gptr, n, g2.ptr, None, ws.ptr, ws.nbytes)
    hip.call("mle_sqrt_scale", None, g2.ptr, 1.0)
    np.testing.assert_array_equal(gs.numpy(dtype=np.float64), g2.numpy(dtype=np.float64))
    # a non-finite element anywhere (here the last, in the tail when n % 4 != 0) sets the flag
    g[-1] = np.inf
    buf.upload(np.concatenate([np.zeros(offset, np.float32), g]))
    hip.call("mle_grad_sqnorm", None, gptr, n, gacc.ptr, bad.ptr, ws.ptr, ws.nbytes)
    assert bad.numpy()[0] == 1


def test_events_and_probe_lists(hip):
    """mle_event_*: the time between two events around queued work; the probe
    armed with a comma-separated family list records calls of each family."""
    n = 1 << 22
    g = B(hip, np.ones(n, np.float32))
    L = hip.lib()
    ws = hip.Buffer(L.mle_sqnorm_ws_bytes(n))
    acc = hip.Buffer.zeros(1, np.float64)
    p, m, v = B(hip, np.zeros(n, np.float32)), B(hip, np.zeros(n, np.float32)), B(hip, np.zeros(n, np.float32))
    e0, e1 = hip.Event(), hip.Event()
    hip.call("mle_probe_arm", b"sqnorm,adam_update")
    e0.record()
    hip.call("mle_grad_sqnorm", None, g.ptr, n, acc.ptr, None, ws.ptr, ws.nbytes)
    hip.call("mle_adam_update", None, p.ptr, g.ptr, m.ptr, v.ptr, n, 1, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, None)
    hip.call("mle_fill", None, p.ptr, 0.0, n)  # not a probed family
    e1.record()
    ms = e1.ms_since(e0)
    import ctypes as C
    k, tot, fl, by = C.c_int(), C.c_double(), C.c_double(), C.c_double()
    hip.call("mle_probe_read", C.byref(k), C.byref(tot), C.byref(fl), C.byref(by))
    hip.call("mle_probe_arm", None)
    assert k.value == 2
    assert by.value == 4.0 * n + 28.0 * n
    assert 0.0 < tot.value <= ms
    assert acc.numpy(dtype=np.float64)[0] == n


# ------------------------------------------------------------ integer paths
def test_gather_onehot_argmax_scatter(hip, orc):
    r = rng(41)
    batch, clen, maxc, dim, vocab = 4, 50, 64, 48, 37
    keys = r.integers(0, vocab, (batch, maxc)).astype(np.int32)
    keys[0, 3] = -1
    keys[1, 5] = np.iinfo(np.int32).min
    keys[2, 7] = vocab + 3  # out of range for one-hot and scatter
    table = r.standard_normal((vocab + 8, dim), dtype=np.float32)
    out_r = np.zeros((batch, clen, dim), np.float32)
    orc.call("orc_gather", orc.ptr(out_r), orc.ptr(table), orc.ptr(keys), batch, clen, maxc, dim)
    gk, gt, go = B(hip, keys), B(hip, table), hip.Buffer.zeros((batch, clen, dim))
    hip.call("mle_embed_gather", None, go.ptr, gt.ptr, gk.ptr, batch, clen, maxc, dim)
    np.testing.assert_array_equal(go.numpy(), out_r)

    # incremental one-hot over two different key sets
    prev = B(hip, np.full(batch * clen, -1, np.int32))
    goh2 = hip.Buffer.zeros((batch * clen, vocab))
    keys2 = r.integers(0, vocab, (batch, maxc)).astype(np.int32)
    for kk in (keys, keys2):
        oh_k = np.zeros((batch * clen, vocab), np.float32)
        orc.call("orc_onehot", orc.ptr(oh_k), orc.ptr(kk), batch, clen, maxc, vocab)
        gkk = B(hip, kk)
        hip.call("mle_onehot_update", None, goh2.ptr, prev.ptr, gkk.ptr, batch, clen, maxc, vocab)
        np.testing.assert_array_equal(goh2.numpy(), oh_k)

    oh_r = np.zeros((batch * clen, vocab), np.float32)
    orc.call("orc_onehot", orc.ptr(oh_r), orc.ptr(keys), batch, clen, maxc, vocab)
    goh = hip.Buffer.zeros((batch * clen, vocab))
    hip.call("mle_onehot", None, goh.ptr, gk.ptr, batch, clen, maxc, vocab)
    np.testing.assert_array_equal(goh.numpy(), oh_r)

    x = r.standard_normal((33, 501), dtype=np.float32)
    x[3, 10] = x[3, 400] = 50.0  # tie -> first index
    x[5, :] = -np.inf
    x[6, 0] = np.nan
    am_r = np.zeros(33, np.int32)
    orc.call("orc_argmax", orc.ptr(x), 33, 501, orc.ptr(am_r))
    gx, gam = B(hip, x), hip.Buffer.zeros(33, np.int32)
    hip.call("mle_argmax", None, gx.ptr, 33, 501, gam.ptr)
    np.testing.assert_array_equal(gam.numpy(), am_r)

    grad = r.standard_normal((batch, clen, dim), dtype=np.float32)
    tab_r = table[:vocab].copy()
    orc.call("orc_scatter_add", orc.ptr(tab_r), orc.ptr(grad), orc.ptr(keys), batch, clen, maxc, dim, vocab, 1.0)
    gtab, gg = B(hip, table[:vocab].copy()), B(hip, grad)
    ws = hip.Buffer(hip.lib().mle_embed_scatter_ws_bytes(batch, clen))
    hip.call("mle_embed_scatter_add", None, gtab.ptr, gg.ptr, gk.ptr, batch, clen, maxc, dim, vocab, 1.0, ws.ptr, ws.nbytes)
    assert_close(gtab.numpy(), tab_r, what="scatter add", **EW)


@pytest.mark.parametrize("batch,clen,dim,vocab,hot", [
    (4, 600, 64, 300, 0), (2, 50, 1100, 40, 0), (3, 300, 700, 500, 0), (32, 256, 512, 8000, 0),  # counting sort
    (40, 300, 16, 1000, 0),    # 12000 tokens: two counting-sort chunks, applied in order
    (4, 100, 33, 50, 0),       # rows not a multiple of 4 floats: scalar segment sums
    (8, 1024, 32, 100, 1),     # one id on most tokens: a run of ~7000 rows
    (2, 100, 64, 20000, 0),    # vocabulary beyond the LDS histogram: row-centric path
    (64, 1024, 8, 20000, 0)])  # ... and beyond that, the bitonic-sort path
def test_scatter_add_paths(hip, orc, batch, clen, dim, vocab, hot):
    """Every scatter-add path against the oracle's serial KeyUpdate, ids outside
    [0, vocab) included, and bit-identical when run twice (fixed summation
    order per table row)."""
    r = rng(batch + clen + dim)
    keys = r.integers(-2, vocab, (batch, clen)).astype(np.int32)
    keys[:, :5] = 3  # repeated key
    if hot:
        keys[r.random((batch, clen)) < 0.85] = 7
    keys[0, -1] = np.iinfo(np.int32).min
    grad = r.standard_normal((batch, clen, dim), dtype=np.float32)
    table = r.standard_normal((vocab, dim), dtype=np.float32)
    ref = table.copy()
    orc.call("orc_scatter_add", orc.ptr(ref), orc.ptr(grad), orc.ptr(keys), batch, clen, clen, dim, vocab, -0.5)
    gg, gk = B(hip, grad), B(hip, keys)
    ws = hip.Buffer(hip.lib().mle_embed_scatter_ws_bytes(batch, clen))
    outs = []
    for _ in range(2):
        gt = B(hip, table)
        hip.call("mle_embed_scatter_add", None, gt.ptr, gg.ptr, gk.ptr, batch, clen, clen, dim, vocab, -0.5, ws.ptr,
                 ws.nbytes)
        outs.append(gt.numpy())
    # rows that many tokens add into are sums of many terms: judged on their size
    counts = np.bincount(keys[(keys >= 0) & (keys < vocab)].ravel(), minlength=vocab).astype(np.float64)
    assert_close(outs[0], ref, what="scatter add", rtol=1e-5,
                 atol_scale=1e-6 * max(1.0, float(np.sqrt(counts.max()))))
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    # mle_embed_grad (scale 1): accumulate 1 is scatter-add; accumulate 0
    # assigns over NaN (rows no token reaches become 0) with the bits of
    # scatter-adding into zeros
    want = []
    for base in (table, np.zeros_like(table)):
        gt = B(hip, base)
        hip.call("mle_embed_scatter_add", None, gt.ptr, gg.ptr, gk.ptr, batch, clen, clen, dim, vocab, 1.0, ws.ptr,
                 ws.nbytes)
        want.append(gt.numpy())
    for accumulate, base, w in ((1, table, want[0]), (0, np.full_like(table, np.nan), want[1])):
        gt = B(hip, base)
        hip.call("mle_embed_grad", None, gt.ptr, gg.ptr, gk.ptr, batch, clen, clen, dim, vocab, accumulate, ws.ptr,
                 ws.nbytes)
        np.testing.assert_array_equal(gt.numpy().view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("batch,clen,maxc,dim,vocab,hot", [
    (32, 256, 256, 512, 8000, 0),  # the C4 embedding
    (4, 600, 600, 64, 300, 0), (2, 50, 50, 1100, 40, 0), (3, 300, 310, 700, 500, 0),  # padded key rows
    (40, 300, 300, 16, 1000, 0),   # 12000 tokens: two chunks, summed chunk by chunk
    (3, 5000, 5000, 8, 70, 1),     # two chunks with one id on most tokens
    (4, 100, 100, 33, 50, 0),      # rows not a multiple of 4 floats
    (8, 1024, 1024, 32, 100, 1),   # one id on ~7000 tokens of one chunk
    (2, 64, 64, 4, 16384, 0),      # the largest vocabulary with an index
    (0, 16, 16, 8, 130, 0)])       # no tokens: every row empty
def test_embed_index(hip, batch, clen, maxc, dim, vocab, hot):
    """The gather that indexes the tokens per table row, and the gradient from
    that index: the gather's bits are mle_embed_gather's, the index lists each
    row's tokens in token order starting at the count of valid smaller keys,
    and the gradient's bits are mle_embed_grad's (chunk-wise sums included),
    assigning and accumulating."""
    L = hip.lib()
    r = rng(batch * 7 + clen + dim + vocab)
    keys = r.integers(-2, vocab, (max(batch, 1), maxc)).astype(np.int32)[:batch]
    if hot and batch:
        keys[r.random(keys.shape) < 0.85] = 7
    if batch:
        keys[:, :3] = 3
        keys[0, clen - 1] = np.iinfo(np.int32).min
    keys = np.ascontiguousarray(keys)
    table = r.standard_normal((vocab, dim), dtype=np.float32)
    grad = r.standard_normal((max(batch * clen, 1), dim), dtype=np.float32)
    nb = L.mle_embed_index_bytes(batch, clen, vocab)
    assert nb >= vocab * 16 + batch * clen * 4 and nb % 256 == 0
    assert L.mle_embed_index_bytes(batch, clen, 16385) == 0
    gk = B(hip, keys if batch else np.zeros((1, maxc), np.int32))
    gt, gg = B(hip, table), B(hip, grad)
    idx = hip.Buffer(nb)
    out = hip.Buffer.zeros((max(batch * clen, 1), dim))
    hip.call("mle_embed_gather_indexed", None, out.ptr, gt.ptr, gk.ptr, batch, clen, maxc, dim, vocab, idx.ptr, nb)
    if batch:
        ref = hip.Buffer.zeros((batch * clen, dim))
        hip.call("mle_embed_gather", None, ref.ptr, gt.ptr, gk.ptr, batch, clen, maxc, dim)
        np.testing.assert_array_equal(out.numpy().view(np.uint32), ref.numpy().view(np.uint32))
    # the index against numpy
    raw = idx.numpy(dtype=np.int32)
    rinfo = raw[:4 * vocab].reshape(vocab, 4)
    flat = keys[:, :clen].ravel()
    valid = (flat >= 0) & (flat < vocab)
    counts = np.bincount(flat[valid], minlength=vocab)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    np.testing.assert_array_equal(rinfo[:, 0], starts)
    np.testing.assert_array_equal(rinfo[:, 1], counts)
    order = np.argsort(np.where(valid, flat, vocab), kind="stable")[:int(valid.sum())]
    lst = raw[4 * vocab:4 * vocab + order.size]
    np.testing.assert_array_equal(lst, order)
    firsts = np.full((vocab, 2), -1, np.int64)
    for j in (0, 1):
        has = counts > j
        firsts[has, j] = order[starts[has] + j]
    np.testing.assert_array_equal(rinfo[:, 2:], firsts)
    # the gradient from the index: mle_embed_grad's bits
    ws = hip.Buffer(L.mle_embed_scatter_ws_bytes(batch, clen))
    for accumulate, base in ((0, np.full_like(table, np.nan)), (1, table)):
        want, got = B(hip, base), B(hip, base)
        if batch:
            hip.call("mle_embed_grad", None, want.ptr, gg.ptr, gk.ptr, batch, clen, maxc, dim, vocab, accumulate,
                     ws.ptr, ws.nbytes)
        else:
            want = B(hip, np.zeros_like(table) if accumulate == 0 else table)
        hip.call("mle_embed_grad_indexed", None, got.ptr, gg.ptr, idx.ptr, batch, clen, dim, vocab, accumulate)
        np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32))


@pytest.mark.parametrize("kind", [2, 1, 0])  # MLE_SILU, MLE_GELU, MLE_RELU
@pytest.mark.parametrize("n", [4099 * 4, 1001])  # float4 body; a scalar tail
def test_add_act_fused(hip, kind, n):
    """The residual Add and the activation after it in one pass each way
    (mle_add_act_fwd, mle_act_bwd_add) give the bits of mle_scale_add +
    mle_act_fwd and mle_act_bwd + mle_accumulate2, for every combination of
    assigning and adding the three gradients."""
    r = rng(n + kind)
    a, b, da, dz0, ga0, gb0 = (r.standard_normal(n, dtype=np.float32) for _ in range(6))
    A, Bb, DA = B(hip, a), B(hip, b), B(hip, da)
    z1, y1, z2, y2 = (hip.Buffer.zeros(n) for _ in range(4))
    hip.call("mle_scale_add", None, A.ptr, Bb.ptr, z1.ptr, 1.0, n)
    hip.call("mle_act_fwd", None, kind, z1.ptr, y1.ptr, n)
    hip.call("mle_add_act_fwd", None, A.ptr, Bb.ptr, z2.ptr, y2.ptr, kind, n)
    np.testing.assert_array_equal(z2.numpy().view(np.uint32), z1.numpy().view(np.uint32))
    np.testing.assert_array_equal(y2.numpy().view(np.uint32), y1.numpy().view(np.uint32))
    for acc_z in (0, 1):
        for acc_a in (0, 1):
            for acc_b in (0, 1):
                dz1, ga1, gb1 = B(hip, dz0), B(hip, ga0), B(hip, gb0)
                hip.call("mle_act_bwd", None, kind, z1.ptr, DA.ptr, dz1.ptr, n, acc_z)
                hip.call("mle_accumulate2", None, dz1.ptr, ga1.ptr, acc_a, gb1.ptr, acc_b, n)
                dz2, ga2, gb2 = (B(hip, x if acc else np.full(n, np.nan, np.float32))
                                 for x, acc in ((dz0, acc_z), (ga0, acc_a), (gb0, acc_b)))
                hip.call("mle_act_bwd_add", None, z1.ptr, DA.ptr, kind, dz2.ptr, acc_z, ga2.ptr, acc_a, gb2.ptr, acc_b,
                         n)
                for u, v in ((dz1, dz2), (ga1, ga2), (gb1, gb2)):
                    np.testing.assert_array_equal(v.numpy().view(np.uint32), u.numpy().view(np.uint32),
                                                  err_msg=f"acc {acc_z}{acc_a}{acc_b}")


@pytest.mark.parametrize("off", [0, 1])  # 1: float offsets, so the scalar path runs
def test_accumulate2_matches_two_accumulates(hip, orc, off):
    """mle_accumulate2 (Add backward's two gradients in one pass) equals
    mle_accumulate / mle_scale_assign at scale 1 on each destination, bit for bit."""
    r = rng(52 + off)
    n = 4099
    x = r.standard_normal(n + 1, dtype=np.float32)
    gx = B(hip, x)
    xo = np.ascontiguousarray(x[off:off + n])  # held while the oracle reads it
    for acc_a in (0, 1):
        for acc_b in (0, 1):
            ya, yb = (r.standard_normal(n + 1, dtype=np.float32) for _ in range(2))
            want = []
            for y, acc in ((ya, acc_a), (yb, acc_b)):
                w = y[off:off + n].copy() if acc else np.zeros(n, np.float32)
                orc.call("orc_accumulate", orc.ptr(xo), orc.ptr(w), 1.0, n)
                want.append(w)
            ga = B(hip, ya if acc_a else np.full_like(ya, np.nan))
            gb = B(hip, yb if acc_b else np.full_like(yb, np.nan))
            hip.call("mle_accumulate2", None, gx.ptr + 4 * off, ga.ptr + 4 * off, acc_a, gb.ptr + 4 * off, acc_b, n)
            for g, w, y, acc in ((ga, want[0], ya, acc_a), (gb, want[1], yb, acc_b)):
                got = g.numpy()
                np.testing.assert_array_equal(got[off:off + n], w)
                edge = got[:off] if off else got[n:]
                np.testing.assert_array_equal(edge, (y[:off] if off else y[n:]) if acc else np.full_like(edge, np.nan))
    with pytest.raises(hip.MLEError):  # one destination twice
        hip.call("mle_accumulate2", None, gx.ptr, ga.ptr, 1, ga.ptr, 1, n)


# ------------------------------------------------------ elementwise / layout
def test_elementwise_and_layout(hip, orc):
    r = rng(51)
    n = 4099
    x = r.standard_normal(n, dtype=np.float32)
    y = r.standard_normal(n, dtype=np.float32)
    z = np.zeros(n, np.float32)
    orc.call("orc_scale_add", orc.ptr(x), orc.ptr(y), orc.ptr(z), -1.0, n)
    gx, gy, gz = B(hip, x), B(hip, y), hip.Buffer.zeros(n)
    hip.call("mle_scale_add", None, gx.ptr, gy.ptr, gz.ptr, -1.0, n)
    np.testing.assert_array_equal(gz.numpy(), z)
    acc = y.copy()
    orc.call("orc_accumulate", orc.ptr(x), orc.ptr(acc), 0.125, n)
    hip.call("mle_accumulate", None, gx.ptr, gy.ptr, 0.125, n)
    np.testing.assert_array_equal(gy.numpy(), acc)
    # scale_assign is accumulate into zeros, bit for bit, without reading y
    for sc in (0.125, 0.3, 1.0):
        acc0 = np.zeros(n, np.float32)
        orc.call("orc_accumulate", orc.ptr(x), orc.ptr(acc0), sc, n)
        hip.call("mle_fill", None, gy.ptr, float("nan"), n)
        hip.call("mle_scale_assign", None, gx.ptr, gy.ptr, sc, n)
        np.testing.assert_array_equal(gy.numpy(), acc0)

    bsz, heads, seq, hd = 2, 4, 9, 8
    flat = r.standard_normal((bsz, 1, seq, heads * hd), dtype=np.float32)
    for flag in range(4):
        src = flat if flag in (0, 3) else r.standard_normal((bsz, heads, seq, hd), dtype=np.float32)
        init = r.standard_normal(flat.size).astype(np.float32)
        ref = init.copy()
        src = np.ascontiguousarray(src)  # held while the oracle reads it
        orc.call("orc_headify", orc.ptr(src), orc.ptr(ref), bsz, heads, seq, hd, flag)
        gs, gd = B(hip, src), B(hip, init)
        hip.call("mle_headify", None, gs.ptr, gd.ptr, bsz, heads, seq, hd, flag)
        np.testing.assert_array_equal(gd.numpy(), ref)

    xs = r.standard_normal((3, 17, 24), dtype=np.float32)
    pe_r = np.zeros_like(xs)
    orc.call("orc_matpe", orc.ptr(xs), orc.ptr(pe_r), 3, 17, 24, 0)
    gxs, gpe = B(hip, xs), hip.Buffer.zeros(xs.shape)
    hip.call("mle_matpe", None, gxs.ptr, gpe.ptr, 3, 17, 24, 0)
    assert_close(gpe.numpy(), pe_r, what="matpe", rtol=1e-6, atol_scale=1e-7)
    for bt, rw, cl, st in ((11, 9, 32, 5), (2, 7, 26, 3)):  # ragged batch chunk; cols not a multiple of 4
        xm = r.standard_normal((bt, rw, cl), dtype=np.float32)
        pm = np.zeros_like(xm)
        orc.call("orc_matpe", orc.ptr(xm), orc.ptr(pm), bt, rw, cl, st)
        gxm, gpm = B(hip, xm), hip.Buffer.zeros(xm.shape)
        hip.call("mle_matpe", None, gxm.ptr, gpm.ptr, bt, rw, cl, st)
        assert_close(gpm.numpy(), pm, what=f"matpe {bt}x{rw}x{cl}", rtol=1e-6, atol_scale=1e-7)
    # the tabulated encoding plus a broadcast add equals mle_matpe bit for bit
    # (32 x 256 x 512 is the C4 shape; the others are ragged / unaligned)
    for bt, rw, cl, st, off in ((32, 256, 512, 0, 0), (11, 9, 32, 5, 0), (2, 7, 26, 3, 0), (3, 5, 8, 2, 1)):
        xm = r.standard_normal(bt * rw * cl + off, dtype=np.float32)
        gxm, gy1, gy2 = B(hip, xm), hip.Buffer.zeros(xm.size), hip.Buffer.zeros(xm.size)
        gtab = hip.Buffer.zeros(rw * cl + off)
        hip.call("mle_matpe", None, gxm.ptr + 4 * off, gy1.ptr + 4 * off, bt, rw, cl, st)
        hip.call("mle_matpe_table", None, gtab.ptr + 4 * off, rw, cl, st)
        hip.call("mle_add_broadcast", None, gxm.ptr + 4 * off, gtab.ptr + 4 * off, gy2.ptr + 4 * off, bt, rw * cl)
        np.testing.assert_array_equal(gy2.numpy().view(np.uint32), gy1.numpy().view(np.uint32))
    tp_r = np.zeros(256, np.float32)
    orc.call("orc_pe", orc.ptr(tp_r), 517, 256)
    gtp = hip.Buffer.zeros(256)
    hip.call("mle_timestep_pe", None, gtp.ptr, 517, 256)
    assert_close(gtp.numpy(), tp_r, what="timestep pe", rtol=1e-6, atol_scale=1e-7)

    rows, cols = 37, 12
    yb = r.standard_normal((rows, cols), dtype=np.float32)
    bb = r.standard_normal(cols, dtype=np.float32)
    ybr = yb.copy()
    orc.call("orc_bcumadd", orc.ptr(ybr), orc.ptr(bb), rows, cols)
    gyb, gbb = B(hip, yb), B(hip, bb)
    hip.call("mle_bias_add_rows", None, gyb.ptr, gbb.ptr, rows, cols)
    np.testing.assert_array_equal(gyb.numpy(), ybr)

    cs_r = np.full(cols, 0.5, np.float32)
    orc.call("orc_bcompress", orc.ptr(yb), orc.ptr(cs_r), rows, cols, 1.0)
    gcs, gyb2 = B(hip, np.full(cols, 0.5, np.float32)), B(hip, yb)
    hip.call("mle_colsum", None, gyb2.ptr, rows, cols, gcs.ptr, 1.0)
    assert_close(gcs.numpy(), cs_r, what="colsum", **EW)

    bt, ch, hw = 3, 16, 50
    xc = r.standard_normal((bt, ch, hw), dtype=np.float32)
    bc_ = r.standard_normal(ch, dtype=np.float32)
    outc = np.zeros_like(xc)
    orc.call("orc_broadcast_add", orc.ptr(xc), orc.ptr(bc_), orc.ptr(outc), bt, ch, hw)
    gxc, gbc, goc = B(hip, xc), B(hip, bc_), hip.Buffer.zeros(xc.shape)
    hip.call("mle_broadcast_channel_add", None, gxc.ptr, gbc.ptr, goc.ptr, bt, ch, hw)
    np.testing.assert_array_equal(goc.numpy(), outc)
    for nred in (ch, 7):
        sq = np.full(ch, 0.25, np.float32)
        orc.call("orc_channel_squeeze", orc.ptr(xc), orc.ptr(sq), bt, ch, hw, nred)
        gsq = B(hip, np.full(ch, 0.25, np.float32))
        hip.call("mle_channel_sum", None, gxc.ptr, bt, ch, hw, nred, gsq.ptr)
        assert_close(gsq.numpy(), sq, what=f"channel_sum {nred}", **EW)
        # assign mode over NaN: the first nred sums (the bits of adding into 0),
        # the rest of a 2*ch-float destination (a [2, ch] gradient) set to 0
        g0, gn = B(hip, np.zeros(2 * ch, np.float32)), B(hip, np.full(2 * ch, np.nan, np.float32))
        hip.call("mle_channel_sum_ex", None, gxc.ptr, bt, ch, hw, nred, g0.ptr, 2 * ch, 1)
        hip.call("mle_channel_sum_ex", None, gxc.ptr, bt, ch, hw, nred, gn.ptr, 2 * ch, 0)
        np.testing.assert_array_equal(gn.numpy(), g0.numpy())
        assert not np.isnan(gn.numpy()).any()

    gf = hip.Buffer.zeros(1001)
    hip.call("mle_fill", None, gf.ptr, 3.5, 1001)
    np.testing.assert_array_equal(gf.numpy(), np.full(1001, 3.5, np.float32))


# ----------------------------------------- cross-entropy from token-id targets
@pytest.mark.parametrize("batch,clen,max_clen,cols", [(4, 24, 24, 1000), (3, 10, 13, 10), (2, 7, 9, 9001),
                                                      (2, 16, 16, 8000), (3, 9, 11, 1500), (2, 5, 5, 4096),
                                                      (9, 520, 523, 1000)])
def test_softmax_xent_keys_matches_dense(hip, orc, batch, clen, max_clen, cols):
    """The id path equals the dense one-hot path bit for bit (loss and
    gradient), ids outside [0, cols) included, and matches the oracle.  The
    4680-row case covers the backward's row walk past its 1024 workgroup rows
    (rows not a multiple of 1024)."""
    r = rng(batch * 17 + clen + cols)
    rows = batch * clen
    logits = (r.standard_normal((rows, cols), dtype=np.float32) * 3).astype(np.float32)
    keys = r.integers(0, cols, (batch, max_clen)).astype(np.int32)
    keys[0, 1] = -1
    keys[-1, 0] = cols + 3
    keys[-1, -1] = np.iinfo(np.int32).min
    tgt = np.zeros((rows, cols), np.float32)
    for b in range(batch):
        for s in range(clen):
            k = keys[b, s]
            if 0 <= k < cols:
                tgt[b * clen + s, k] = 1.0
    L = hip.lib()
    n = rows * cols
    gl, gt, gk = B(hip, logits), B(hip, tgt), B(hip, keys)
    gp, gloss, gloss2 = hip.Buffer.zeros((rows, cols)), hip.Buffer.zeros(1), hip.Buffer.zeros(1)
    gst = hip.Buffer.zeros(2 * rows)
    ws = hip.Buffer(L.mle_loss_ws_bytes(n))
    hip.call("mle_softmax_xent_fwd", None, gl.ptr, gt.ptr, gp.ptr, rows, cols, gloss.ptr, ws.ptr, ws.nbytes)
    hip.call("mle_softmax_xent_keys_fwd", None, gl.ptr, gk.ptr, clen, max_clen, gst.ptr, rows, cols, gloss2.ptr,
             ws.ptr, ws.nbytes)
    np.testing.assert_array_equal(gloss2.numpy(), gloss.numpy())
    up = B(hip, np.array([0.75], np.float32))
    for upstream in (None, up.ptr):
        gd, gd2 = hip.Buffer.zeros((rows, cols)), hip.Buffer.zeros((rows, cols))
        hip.call("mle_softmax_xent_bwd", None, gp.ptr, gt.ptr, upstream, gd.ptr, n, batch)
        hip.call("mle_fill", None, gd2.ptr, float("nan"), n)
        hip.call("mle_softmax_xent_keys_bwd", None, gl.ptr, gst.ptr, gk.ptr, clen, max_clen, upstream, gd2.ptr, rows,
                 cols, batch)
        np.testing.assert_array_equal(gd2.numpy(), gd.numpy())
    pr = np.zeros_like(logits)
    lref = orc.call("orc_softmax_xent_fwd", orc.ptr(logits), orc.ptr(tgt), orc.ptr(pr), rows, cols)
    assert_close(gloss2.numpy(), np.array([lref], np.float32), what="keys loss", **EW)


def _rowstats_ref(c: np.ndarray) -> np.ndarray:
    """(max, sum exp(c - max)) per row and 64-column block, in float64."""
    rows, cols = c.shape
    nblk = (cols + 63) // 64
    out = np.zeros((rows, nblk, 2))
    for b in range(nblk):
        blk = c[:, b * 64:(b + 1) * 64].astype(np.float64)
        m = blk.max(1)
        out[:, b, 0] = m
        out[:, b, 1] = np.exp(blk - m[:, None]).sum(1)
    return out


@pytest.mark.parametrize("ta,tb,M,N,K", [
    (0, 0, 4100, 4000, 64),    # persistent kernel: statistics from the epilogue (ragged last block and rows)
    (0, 1, 3000, 2900, 192),
    (0, 0, 300, 130, 70),      # other kernels: statistics from a second pass over C
    (1, 0, 1000, 8000, 48),
])
def test_gemm_rowstats(hip, orc, ta, tb, M, N, K):
    """mle_gemm_rowstats writes the GEMM result (with bias) and, per row and
    64-column block, the block max (exactly the max of the written C) and the
    sum of exp(C - max) (1e-5 relative)."""
    r = rng(M + 3 * N + K)
    A = r.standard_normal((K, M) if ta else (M, K), dtype=np.float32)
    Bm = r.standard_normal((N, K) if tb else (K, N), dtype=np.float32)
    bias = r.standard_normal(N, dtype=np.float32)
    ref = np.zeros((M, N), np.float32)
    orc.call("orc_bcmm", ta * 2 + tb, orc.ptr(A), orc.ptr(Bm), orc.ptr(ref), 1, 1, M, K, N, 0, 3, 3, 3, 1.0)
    ref += bias
    nblk = (N + 63) // 64
    ldp = 2 * nblk + 2
    gA, gB, gbias = B(hip, A), B(hip, Bm), B(hip, bias)
    gC = hip.Buffer.zeros((M, N))
    gp = B(hip, np.full(M * ldp, 7.0, np.float32))
    L = hip.lib()
    ws = hip.Buffer(max(L.mle_gemm_ws_bytes(M, N, K, 1), 4))
    hip.call("mle_gemm_rowstats", None, ta, tb, M, N, K, 1.0, gA.ptr, M if ta else K, gB.ptr, K if tb else N, 0.0,
             gC.ptr, N, gbias.ptr, gp.ptr, ldp, ws.ptr, ws.nbytes)
    c = gC.numpy()
    assert_close(c, ref, what="gemm_rowstats C", **MM)
    part = gp.numpy().reshape(M, ldp)
    want = _rowstats_ref(c)
    np.testing.assert_array_equal(part[:, 0:2 * nblk:2], want[:, :, 0].astype(np.float32))
    assert_close(part[:, 1:2 * nblk:2], want[:, :, 1], what="block sum of exp", **EW)
    assert np.all(part[:, 2 * nblk:] == 7.0), "padding of a row's partials written"


@pytest.mark.parametrize("batch,clen,cols", [(4, 64, 8000), (3, 10, 1000), (2, 7, 130)])
def test_softmax_xent_keys_rowstats(hip, batch, clen, cols):
    """The loss from row statistics equals the keys path that reads the logits:
    the row max bit for bit, the row sum and the loss within 1e-5."""
    r = rng(batch * 31 + clen + cols)
    rows = batch * clen
    logits = (r.standard_normal((rows, cols), dtype=np.float32) * 3).astype(np.float32)
    keys = r.integers(0, cols, (batch, clen)).astype(np.int32)
    keys[0, 1] = -1
    keys[-1, 0] = cols + 3
    nblk = (cols + 63) // 64
    part = _rowstats_ref(logits)
    ldp = 2 * nblk
    gl, gk = B(hip, logits), B(hip, keys)
    gpart = B(hip, part.astype(np.float32).reshape(rows, ldp))
    gst, gst2 = hip.Buffer.zeros(2 * rows), hip.Buffer.zeros(2 * rows)
    gloss, gloss2 = hip.Buffer.zeros(1), hip.Buffer.zeros(1)
    L = hip.lib()
    ws = hip.Buffer(L.mle_loss_ws_bytes(rows * cols))
    hip.call("mle_softmax_xent_keys_fwd", None, gl.ptr, gk.ptr, clen, clen, gst.ptr, rows, cols, gloss.ptr, ws.ptr,
             ws.nbytes)
    hip.call("mle_softmax_xent_keys_fwd_rowstats", None, gl.ptr, gpart.ptr, ldp, gk.ptr, clen, clen, gst2.ptr, rows,
             cols, gloss2.ptr, ws.ptr, ws.nbytes)
    st, st2 = gst.numpy().reshape(rows, 2), gst2.numpy().reshape(rows, 2)
    np.testing.assert_array_equal(st2[:, 0], st[:, 0])
    assert_close(st2[:, 1], st[:, 1], what="row sums", **EW)
    assert_close(gloss2.numpy(), gloss.numpy(), what="loss", **EW)
    # The loss with its read-back (the finishing kernel publishes the value):
    # the same device loss and stats bits, and the host value equal to the
    # device value, on two calls in a row.
    for rep in range(2):
        gst3, gloss3 = hip.Buffer.zeros(2 * rows), hip.Buffer.zeros(1)
        host = C.c_float(float("nan"))
        hip.call("mle_softmax_xent_keys_fwd_rowstats_read", None, gl.ptr, gpart.ptr, ldp, gk.ptr, clen, clen, gst3.ptr,
                 rows, cols, gloss3.ptr, ws.ptr, ws.nbytes, C.byref(host))
        np.testing.assert_array_equal(gst3.numpy(), gst2.numpy())
        np.testing.assert_array_equal(gloss3.numpy().view(np.uint32), gloss2.numpy().view(np.uint32))
        assert np.float32(host.value).view(np.uint32) == gloss2.numpy().view(np.uint32)[0], (rep, host.value)


@pytest.mark.parametrize("batch,clen,cols,hidden,bias", [
    (64, 1, 10, 256, True),   # C1's head: 4 tiles, 4 waves each
    (3, 12, 33, 100, False),  # 3 x 3 ragged tiles, K tails, no bias
    (16, 1, 64, 70, True),    # 4 tile columns
    (16, 16, 16, 64, True),   # 16 tiles: one wave each
    (20, 5, 64, 50, True),    # 28 tiles: the two-launch path
])
def test_linear_xent_keys_small(hip, orc, batch, clen, cols, hidden, bias):
    """A classifier head (Linear, then the cross-entropy against ids) in one
    launch: the logits against the oracle's product plus bias, and the row
    statistics, loss, host read-back and gradient the bits of
    mle_softmax_xent_keys_small_read on those logits, on two calls in a row."""
    r = rng(batch + clen * 5 + cols + hidden)
    rows = batch * clen
    X = r.standard_normal((rows, hidden), dtype=np.float32)
    W = (r.standard_normal((hidden, cols), dtype=np.float32) * 0.5).astype(np.float32)
    b = r.standard_normal(cols, dtype=np.float32)
    keys = r.integers(0, cols, (batch, clen)).astype(np.int32)
    keys[0, 0] = -1
    keys[-1, -1] = cols + 2
    want = np.zeros((rows, cols), np.float32)
    orc.call("orc_bcmm", 0, orc.ptr(X), orc.ptr(W), orc.ptr(want), 1, 1, rows, hidden, cols, 0, 3, 3, 3, 1.0)
    if bias:
        want += b
    gX, gW, gb, gk = B(hip, X), B(hip, W), B(hip, b), B(hip, keys)
    for rep in range(2):
        glog = B(hip, np.full((rows, cols), np.nan, np.float32))
        gst, gloss = B(hip, np.full(2 * rows, np.nan, np.float32)), hip.Buffer.zeros(1)
        gd = B(hip, np.full((rows, cols), np.nan, np.float32))
        host = C.c_float(float("nan"))
        hip.call("mle_linear_xent_keys_small_read", None, rows, hidden, cols, gX.ptr, gW.ptr, gb.ptr if bias else None,
                 glog.ptr, gk.ptr, clen, clen, gst.ptr, batch, gloss.ptr, gd.ptr, C.byref(host))
        assert_close(glog.numpy(), want, what="head logits", **MM)
        gst2, gloss2 = hip.Buffer.zeros(2 * rows), hip.Buffer.zeros(1)
        gd2 = hip.Buffer.zeros((rows, cols))
        host2 = C.c_float(float("nan"))
        hip.call("mle_softmax_xent_keys_small_read", None, glog.ptr, gk.ptr, clen, clen, gst2.ptr, rows, cols, batch,
                 gloss2.ptr, gd2.ptr, C.byref(host2))
        for got, ref, what in ((gst, gst2, "stats"), (gloss, gloss2, "loss"), (gd, gd2, "gradient")):
            np.testing.assert_array_equal(got.numpy().view(np.uint32), ref.numpy().view(np.uint32), err_msg=what)
        assert np.float32(host.value).view(np.uint32) == np.float32(host2.value).view(np.uint32), rep


@pytest.mark.parametrize("batch,clen,cols,hidden", [(64, 1, 10, 256), (4, 16, 64, 32), (3, 5, 7, 40), (16, 64, 33, 8)])
def test_softmax_xent_keys_small(hip, orc, batch, clen, cols, hidden):
    """A classifier head's cross-entropy in one launch (rows <= 1024,
    cols <= 64): the row statistics, loss, host read-back and gradient are the
    bits of the three-launch path the engine takes otherwise -- the GEMM with
    row statistics, mle_softmax_xent_keys_fwd_rowstats_read and
    mle_softmax_xent_keys_bwd -- on the GEMM's logits; keys out of range
    included; and the loss within 1e-5 of the oracle's dense one-hot loss."""
    r = rng(batch + clen * 3 + cols + hidden)
    rows = batch * clen
    X = r.standard_normal((rows, hidden), dtype=np.float32)
    W = (r.standard_normal((hidden, cols), dtype=np.float32) * 0.5).astype(np.float32)
    bias = r.standard_normal(cols, dtype=np.float32)
    keys = r.integers(0, cols, (batch, clen)).astype(np.int32)
    keys[0, 0] = -1
    keys[-1, -1] = cols + 2
    L = hip.lib()
    gX, gW, gb, gk = B(hip, X), B(hip, W), B(hip, bias), B(hip, keys)
    nblk = (cols + 63) // 64
    ldp = 2 * nblk
    glog, gpart = hip.Buffer.zeros((rows, cols)), hip.Buffer.zeros(rows * ldp)
    wsg = hip.Buffer(max(256, L.mle_gemm_ws_bytes(rows, cols, hidden, 1)))
    hip.call("mle_gemm_rowstats", None, 0, 0, rows, cols, hidden, 1.0, gX.ptr, hidden, gW.ptr, cols, 0.0, glog.ptr, cols,
             gb.ptr, gpart.ptr, ldp, wsg.ptr, wsg.nbytes)
    ws = hip.Buffer(L.mle_loss_ws_bytes(rows * cols))
    gst, gloss = hip.Buffer.zeros(2 * rows), hip.Buffer.zeros(1)
    host = C.c_float(float("nan"))
    hip.call("mle_softmax_xent_keys_fwd_rowstats_read", None, glog.ptr, gpart.ptr, ldp, gk.ptr, clen, clen, gst.ptr,
             rows, cols, gloss.ptr, ws.ptr, ws.nbytes, C.byref(host))
    gd = hip.Buffer.zeros((rows, cols))
    hip.call("mle_softmax_xent_keys_bwd", None, glog.ptr, gst.ptr, gk.ptr, clen, clen, None, gd.ptr, rows, cols, batch)
    for with_grad in (True, False):
        gst2, gloss2 = B(hip, np.full(2 * rows, np.nan, np.float32)), hip.Buffer.zeros(1)
        gd2 = B(hip, np.full((rows, cols), np.nan, np.float32))
        host2 = C.c_float(float("nan"))
        hip.call("mle_softmax_xent_keys_small_read", None, glog.ptr, gk.ptr, clen, clen, gst2.ptr, rows, cols, batch,
                 gloss2.ptr, gd2.ptr if with_grad else None, C.byref(host2))
        np.testing.assert_array_equal(gst2.numpy().view(np.uint32), gst.numpy().view(np.uint32))
        np.testing.assert_array_equal(gloss2.numpy().view(np.uint32), gloss.numpy().view(np.uint32))
        assert np.float32(host2.value).view(np.uint32) == np.float32(host.value).view(np.uint32)
        if with_grad:
            np.testing.assert_array_equal(gd2.numpy().view(np.uint32), gd.numpy().view(np.uint32))
        else:
            assert np.all(np.isnan(gd2.numpy()))
    logits = glog.numpy()
    tgt = np.zeros((rows, cols), np.float32)
    for b in range(batch):
        for s_ in range(clen):
            if 0 <= keys[b, s_] < cols:
                tgt[b * clen + s_, keys[b, s_]] = 1.0
    pr = np.zeros_like(logits)
    lref = orc.call("orc_softmax_xent_fwd", orc.ptr(logits), orc.ptr(tgt), orc.ptr(pr), rows, cols)
    assert_close(gloss.numpy(), np.array([lref], np.float32), what="small-logits loss", **EW)


@pytest.mark.parametrize("kind", ["silu", "gelu", "relu", "tanh"])
@pytest.mark.parametrize("n", [7, 123456, 123457, 8 << 20])
def test_mse_act_fwd_bwd_read(hip, orc, kind, n):
    """The last MSE node's forward on an activation's output, reading the
    activation's input z: the loss (device and host), the prediction's
    gradient and z's gradient are the bits of mle_act_fwd, then
    mle_mse_fwd_bwd_read on its output, then an assigning mle_act_bwd; both
    partial paths (n % 4); and against the oracle's MSE and derivative."""
    r = rng(n % 1000 + 11 + hip.ACT[kind])
    k = hip.ACT[kind]
    z = (r.standard_normal(n, dtype=np.float32) * 2).astype(np.float32)
    t = r.standard_normal(n, dtype=np.float32)
    gz, gt = B(hip, z), B(hip, t)
    ws = hip.Buffer(hip.lib().mle_loss_ws_bytes(n))
    gx, gl, gdx, gdz = hip.Buffer.zeros(n), hip.Buffer.zeros(1), hip.Buffer.zeros(n), hip.Buffer.zeros(n)
    host = C.c_float(float("nan"))
    hip.call("mle_act_fwd", None, k, gz.ptr, gx.ptr, n)
    hip.call("mle_mse_fwd_bwd_read", None, gx.ptr, gt.ptr, n, gl.ptr, gdx.ptr, ws.ptr, ws.nbytes, C.byref(host))
    hip.call("mle_act_bwd", None, k, gz.ptr, gdx.ptr, gdz.ptr, n, 0)
    for rep in range(2):
        gl2 = hip.Buffer.zeros(1)
        gdx2, gdz2 = B(hip, np.full(n, np.nan, np.float32)), B(hip, np.full(n, np.nan, np.float32))
        host2 = C.c_float(float("nan"))
        hip.call("mle_mse_act_fwd_bwd_read", None, gz.ptr, gt.ptr, n, k, gl2.ptr, gdx2.ptr, gdz2.ptr, ws.ptr, ws.nbytes,
                 C.byref(host2))
        for got, want, what in ((gl2, gl, "loss"), (gdx2, gdx, "dx"), (gdz2, gdz, "dz")):
            np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32), err_msg=what)
        assert np.float32(host2.value).view(np.uint32) == np.float32(host.value).view(np.uint32), rep
    if n <= 123457:
        x = np.zeros_like(z)
        orc.call("orc_act_fwd", k, orc.ptr(z), orc.ptr(x), n)
        dz_ref = np.zeros_like(z)
        dx_ref = (2.0 * (x.astype(np.float64) - t) / n).astype(np.float32)
        orc.call("orc_act_bwd", k, orc.ptr(z), orc.ptr(dx_ref), orc.ptr(dz_ref), n)
        assert_close(gdz.numpy(), dz_ref, what=f"mse + {kind} dz", **EW)
        lref = np.mean((x.astype(np.float64) - t) ** 2)
        assert_close(gl.numpy(), np.array([lref], np.float32), what="mse loss", **EW)


@pytest.mark.parametrize("kind", ["silu", "gelu", "relu"])
@pytest.mark.parametrize("n", [7, 123456, 123457, 8 << 20])
def test_add_mse_act_fwd_bwd_read(hip, kind, n):
    """An Add, the activation after it and the last MSE node in one pass: z,
    the loss (device and host) and both gradients are the bits of
    mle_add_act_fwd followed by mle_mse_act_fwd_bwd_read on its z, on both
    partial paths (n % 4), twice in a row, and without storing z (z NULL);
    aliasing outputs are refused."""
    r = rng(n % 1000 + 29 + hip.ACT[kind])
    k = hip.ACT[kind]
    a = r.standard_normal(n, dtype=np.float32)
    b = (r.standard_normal(n, dtype=np.float32) * 2).astype(np.float32)
    t = r.standard_normal(n, dtype=np.float32)
    ga, gb, gt = B(hip, a), B(hip, b), B(hip, t)
    ws = hip.Buffer(hip.lib().mle_loss_ws_bytes(n))
    gz, gy, gl, gdx, gdz = (hip.Buffer.zeros(n), hip.Buffer.zeros(n), hip.Buffer.zeros(1), hip.Buffer.zeros(n),
                            hip.Buffer.zeros(n))
    host = C.c_float(float("nan"))
    hip.call("mle_add_act_fwd", None, ga.ptr, gb.ptr, gz.ptr, gy.ptr, k, n)
    hip.call("mle_mse_act_fwd_bwd_read", None, gz.ptr, gt.ptr, n, k, gl.ptr, gdx.ptr, gdz.ptr, ws.ptr, ws.nbytes,
             C.byref(host))
    for rep in range(2):
        gz2, gl2 = B(hip, np.full(n, np.nan, np.float32)), hip.Buffer.zeros(1)
        gdx2, gdz2 = B(hip, np.full(n, np.nan, np.float32)), B(hip, np.full(n, np.nan, np.float32))
        host2 = C.c_float(float("nan"))
        hip.call("mle_add_mse_act_fwd_bwd_read", None, ga.ptr, gb.ptr, gz2.ptr, gt.ptr, n, k, gl2.ptr, gdx2.ptr,
                 gdz2.ptr, ws.ptr, ws.nbytes, C.byref(host2))
        for got, want, what in ((gz2, gz, "z"), (gl2, gl, "loss"), (gdx2, gdx, "dx"), (gdz2, gdz, "dz")):
            np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32),
                                          err_msg=f"{what} rep {rep}")
        assert np.float32(host2.value).view(np.uint32) == np.float32(host.value).view(np.uint32), rep
    # z = NULL: the same loss and gradients, z not stored
    gl3, host3 = hip.Buffer.zeros(1), C.c_float(float("nan"))
    gdx3, gdz3 = B(hip, np.full(n, np.nan, np.float32)), B(hip, np.full(n, np.nan, np.float32))
    hip.call("mle_add_mse_act_fwd_bwd_read", None, ga.ptr, gb.ptr, None, gt.ptr, n, k, gl3.ptr, gdx3.ptr, gdz3.ptr,
             ws.ptr, ws.nbytes, C.byref(host3))
    for got, want, what in ((gl3, gl, "loss"), (gdx3, gdx, "dx"), (gdz3, gdz, "dz")):
        np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32), err_msg=f"{what} z=NULL")
    assert np.float32(host3.value).view(np.uint32) == np.float32(host.value).view(np.uint32)
    if n == 7:  # z may not alias an input, and dz may not be z here
        for args in ((ga.ptr, gb.ptr, ga.ptr, gdx.ptr, gdz.ptr), (ga.ptr, gb.ptr, gz.ptr, gdx.ptr, gz.ptr)):
            a_, b_, z_, dx_, dz_ = args
            rc = hip.lib().mle_add_mse_act_fwd_bwd_read(None, a_, b_, z_, gt.ptr, C.c_size_t(n), k, gl.ptr, dx_, dz_,
                                                        ws.ptr, C.c_size_t(ws.nbytes), C.byref(host))
            assert rc != 0


@pytest.mark.parametrize("n", [5, 1000, 123457, 123456, 8 << 20])
def test_mse_fwd_read(hip, n):
    """mle_mse_fwd_read: the loss of mle_mse_fwd bit for bit, on the device and
    on the host, on both partial paths (n % 4) and from one partial to the
    2048-partial cap; two calls in a row with another read in between."""
    r = rng(n % 1000 + 7)
    x = r.standard_normal(n, dtype=np.float32)
    t = r.standard_normal(n, dtype=np.float32)
    gx, gt = B(hip, x), B(hip, t)
    ws = hip.Buffer(hip.lib().mle_loss_ws_bytes(n))
    gl, gl2 = hip.Buffer.zeros(1), hip.Buffer.zeros(1)
    hip.call("mle_mse_fwd", None, gx.ptr, gt.ptr, n, gl.ptr, ws.ptr, ws.nbytes)
    want = gl.numpy().view(np.uint32)[0]
    for rep in range(2):
        host = C.c_float(float("nan"))
        hip.call("mle_mse_fwd_read", None, gx.ptr, gt.ptr, n, gl2.ptr, ws.ptr, ws.nbytes, C.byref(host))
        assert gl2.numpy().view(np.uint32)[0] == want, rep
        assert np.float32(host.value).view(np.uint32) == want, (rep, host.value)
        other = C.c_float(0.0)
        hip.call("mle_read_scalar", None, gx.ptr, C.byref(other))
        assert other.value == x[0]
    # the loss and the last node's gradient from one pass: the bits of
    # mle_mse_fwd_read followed by an assigning mle_mse_bwd
    dx1 = hip.Buffer.zeros(n)
    hip.call("mle_mse_bwd", None, gx.ptr, gt.ptr, None, dx1.ptr, n, 0)
    dx2 = B(hip, np.full(n, np.nan, np.float32))
    host = C.c_float(float("nan"))
    hip.call("mle_mse_fwd_bwd_read", None, gx.ptr, gt.ptr, n, gl2.ptr, dx2.ptr, ws.ptr, ws.nbytes, C.byref(host))
    assert gl2.numpy().view(np.uint32)[0] == want
    assert np.float32(host.value).view(np.uint32) == want
    np.testing.assert_array_equal(dx2.numpy().view(np.uint32), dx1.numpy().view(np.uint32))


@pytest.mark.parametrize("kind", ["relu", "gelu", "silu", "tanh"])
@pytest.mark.parametrize("M,N,K,ws", [(4100, 4000, 64, False), (300, 130, 70, False),
                                      # split along K: the reduce that completes C writes Y
                                      (64, 256, 784, True), (64, 10, 256, True), (70, 130, 900, True)])
def test_gemm_act_fwd(hip, orc, kind, M, N, K, ws):
    """C = A B + bias and Y = act(C) (the persistent kernel's epilogue for
    ReLU / GELU / SiLU on the large shape, the split reduce's for small split
    products, the activation kernel otherwise) against the oracle's GEMM and
    activation."""
    r = rng(M + N + K + hip.ACT[kind])
    A = r.standard_normal((M, K), dtype=np.float32) * 0.25
    Bm = r.standard_normal((K, N), dtype=np.float32) * 0.25
    bias = r.standard_normal(N, dtype=np.float32)
    c_ref = np.zeros((M, N), np.float32)
    orc.call("orc_bcmm", 0, orc.ptr(A), orc.ptr(Bm), orc.ptr(c_ref), 1, 1, M, K, N, 0, 3, 3, 3, 1.0)
    c_ref += bias
    y_ref = np.zeros_like(c_ref)
    orc.call("orc_act_fwd", hip.ACT[kind], orc.ptr(c_ref), orc.ptr(y_ref), M * N)
    gA, gB, gb = B(hip, A), B(hip, Bm), B(hip, bias)
    gC, gY = hip.Buffer.zeros((M, N)), hip.Buffer.zeros((M, N))
    wsb = hip.lib().mle_gemm_ws_bytes(M, N, K, 1) if ws else 0
    if ws:
        assert wsb > 0  # the shape splits along K
    gws = hip.Buffer(max(wsb, 256)) if ws else None
    hip.call("mle_gemm_act_fwd", None, 0, 0, M, N, K, 1.0, gA.ptr, K, gB.ptr, N, 0.0, gC.ptr, gb.ptr, hip.ACT[kind],
             gY.ptr, gws.ptr if ws else None, wsb)
    assert_close(gC.numpy(), c_ref, what=f"gemm_act_fwd C", **MM)
    assert_close(gY.numpy(), y_ref, what=f"gemm_act_fwd {kind}", **MM)
    # the epilogue applies the activation kernels' function to the stored C
    gY2 = hip.Buffer.zeros((M, N))
    hip.call("mle_act_fwd", None, hip.ACT[kind], gC.ptr, gY2.ptr, M * N)
    if ws:  # the same function on the same values: the same bits
        np.testing.assert_array_equal(gY.numpy().view(np.uint32), gY2.numpy().view(np.uint32))
    assert_close(gY.numpy(), gY2.numpy(), what=f"{kind} of the stored C", rtol=1e-6, atol_scale=1e-7)


@pytest.mark.parametrize("kind", ["relu", "gelu", "silu", "tanh"])
@pytest.mark.parametrize("M,N,K,beta,acc", [(3000, 2900, 192, 0.0, 0), (3000, 2900, 192, 1.0, 1),
                                            (300, 130, 70, 1.0, 1), (64, 256, 10, 0.0, 0), (64, 256, 10, 1.0, 1)])
def test_gemm_act_bwd(hip, orc, kind, M, N, K, beta, acc):
    """C (+)= A B^T (the activation output's gradient) and dX (+)= C * act'(X)
    against the oracle's GEMM and activation derivative: the persistent
    kernel's epilogue (large), the K-split kernel's (300 x 130 x 70) and the
    one-thread-per-output kernel's (K = 10)."""
    r = rng(M + 2 * N + K + hip.ACT[kind] + acc)
    A = r.standard_normal((M, K), dtype=np.float32) * 0.25
    Bm = r.standard_normal((N, K), dtype=np.float32) * 0.25
    C0 = r.standard_normal((M, N), dtype=np.float32)
    X = (r.standard_normal((M, N), dtype=np.float32) * 2).astype(np.float32)
    dX0 = r.standard_normal((M, N), dtype=np.float32)
    c_ref = C0.copy() if beta else np.zeros((M, N), np.float32)
    orc.call("orc_bcmm", 1, orc.ptr(A), orc.ptr(Bm), orc.ptr(c_ref), 1, 1, M, K, N, 1, 3, 3, 3, 1.0)
    dx_ref = dX0.copy() if acc else np.zeros_like(dX0)
    orc.call("orc_act_bwd", hip.ACT[kind], orc.ptr(X), orc.ptr(c_ref), orc.ptr(dx_ref), M * N)
    gA, gB, gC, gX, gdX = B(hip, A), B(hip, Bm), B(hip, C0), B(hip, X), B(hip, dX0)
    if not acc:
        hip.call("mle_fill", None, gdX.ptr, float("nan"), M * N)  # assign: dX is not read
    hip.call("mle_gemm_act_bwd", None, 0, 1, M, N, K, 1.0, gA.ptr, K, gB.ptr, K, beta, gC.ptr, hip.ACT[kind], gX.ptr,
             gdX.ptr, acc, None, 0)
    assert_close(gC.numpy(), c_ref, what="gemm_act_bwd C", **MM)
    assert_close(gdX.numpy(), dx_ref, what=f"gemm_act_bwd d{kind}", **MM)


@pytest.mark.parametrize("kind", ["relu", "gelu"])
@pytest.mark.parametrize("rows,inp,out,acc", [
    (64, 256, 10, 0),      # both products one thread per output: the activation in their launch
    (64, 256, 10, 1),
    (64, 784, 256, 1),     # both on the K-split kernel: the activation in their launch
    (300, 130, 70, 0),
    (8192, 384, 128, 1),   # register-direct pair: the activation pass after it
    (4224, 2048, 128, 0),  # dX on the persistent kernel: the activation pass after it
    (4224, 2048, 128, 1),
])
def test_linear_bwd_act(hip, orc, kind, rows, inp, out, acc):
    """mle_linear_bwd_act: a Linear's backward with the backward of the
    activation before it.  dX, dW and db have the bits of mle_linear_bwd_ex
    and the activation gradient those of mle_act_bwd on that dX (the same
    formula, the product rounded before the add); both against the oracle."""
    r = rng(rows + 3 * inp + out + acc + hip.ACT[kind])
    k = hip.ACT[kind]
    X = r.standard_normal((rows, inp), dtype=np.float32)
    dY = r.standard_normal((rows, out), dtype=np.float32)
    W = r.standard_normal((inp, out), dtype=np.float32)
    Z = (r.standard_normal((rows, inp), dtype=np.float32) * 2).astype(np.float32)
    dX0 = r.standard_normal((rows, inp), dtype=np.float32)
    dZ0 = r.standard_normal((rows, inp), dtype=np.float32)
    dW0 = r.standard_normal((inp, out), dtype=np.float32)
    db0 = r.standard_normal(out, dtype=np.float32)
    L = hip.lib()
    need = L.mle_linear_bwd_ws_bytes(rows, inp, out, 1)
    ws = hip.Buffer(max(need, 4))
    gX, gdY, gW, gZ = B(hip, X), B(hip, dY), B(hip, W), B(hip, Z)
    # unfused: the Linear's products, then the activation pass
    udX, udW, udb, udZ = B(hip, dX0), B(hip, dW0), B(hip, db0), B(hip, dZ0)
    hip.call("mle_linear_bwd_ex", None, rows, inp, out, 1, gX.ptr, gdY.ptr, 0, gW.ptr, 0, udX.ptr, acc, udW.ptr,
             udb.ptr, 0, 1, ws.ptr, need)
    hip.call("mle_act_bwd", None, k, gZ.ptr, udX.ptr, udZ.ptr, rows * inp, acc)
    # fused; with acc 0 the destinations start as NaN (assigned, never read)
    nan = np.full((rows, inp), np.nan, np.float32)
    fdX, fdW, fdb, fdZ = B(hip, dX0 if acc else nan), B(hip, dW0), B(hip, db0), B(hip, dZ0 if acc else nan)
    hip.call("mle_linear_bwd_act", None, rows, inp, out, gX.ptr, gdY.ptr, gW.ptr, fdX.ptr, acc, fdW.ptr, fdb.ptr, 1, k,
             gZ.ptr, fdZ.ptr, acc, ws.ptr, need)
    for got, want, what in ((fdX, udX, "dX"), (fdW, udW, "dW"), (fdb, udb, "db"), (fdZ, udZ, "activation dX")):
        np.testing.assert_array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32), err_msg=what)
    # against the oracle
    want_dx = dX0.copy() if acc else np.zeros_like(dX0)
    orc.call("orc_bcmm", 1, orc.ptr(dY), orc.ptr(W), orc.ptr(want_dx), 1, 1, rows, out, inp, 1, 3, 3, 3, 1.0)
    want_dz = dZ0.copy() if acc else np.zeros_like(dZ0)
    orc.call("orc_act_bwd", k, orc.ptr(Z), orc.ptr(want_dx), orc.ptr(want_dz), rows * inp)
    want_dw = dW0.copy()
    orc.call("orc_bcmm", 2, orc.ptr(X), orc.ptr(dY), orc.ptr(want_dw), 1, 1, inp, rows, out, 1, 3, 3, 3, 1.0)
    assert_close(fdX.numpy(), want_dx, what="linear_bwd_act dX", **MM)
    assert_close(fdZ.numpy(), want_dz, what=f"linear_bwd_act d{kind}", **MM)
    assert_close(fdW.numpy(), want_dw, what="linear_bwd_act dW", **MM)
    assert_close(fdb.numpy(), db0 + dY.astype(np.float64).sum(0), what="linear_bwd_act db", **EW)
    if rows == 64 and kind == "relu" and acc == 0:  # the activation gradient may not overwrite an operand
        for alias in (fdX, gdY, gX, gW):
            with pytest.raises(hip.MLEError):
                hip.call("mle_linear_bwd_act", None, rows, inp, out, gX.ptr, gdY.ptr, gW.ptr, fdX.ptr, 0, fdW.ptr,
                         fdb.ptr, 1, k, gZ.ptr, alias.ptr, 0, ws.ptr, need)


# ------------------------------------------------------------------ arena
def test_arena_bump_allocation(hip):
    """mle_arena_*: 256-byte aligned bump allocation inside one device buffer,
    exhaustion reported as MLE_ERR_OOM, reset reuses the space, and the memory
    is usable by a kernel (fill, read back)."""
    L = hip.lib()
    arena = C.c_void_p()
    hip.call("mle_arena_create", 1000, C.byref(arena))
    assert L.mle_arena_capacity(arena) == 1024 and L.mle_arena_used(arena) == 0
    ptrs = []
    for nbytes in (4, 300, 256):
        p = C.c_void_p()
        hip.call("mle_arena_alloc", arena, nbytes, C.byref(p))
        ptrs.append(p.value)
    assert [q - ptrs[0] for q in ptrs] == [0, 256, 768]
    assert L.mle_arena_used(arena) == 1024
    p = C.c_void_p()
    assert L.mle_arena_alloc(arena, 1, C.byref(p)) == -3  # MLE_ERR_OOM
    assert b"requested" in L.mle_last_error()
    hip.call("mle_fill", None, ptrs[1], 2.5, 75)
    out = np.empty(75, np.float32)
    hip.call("mle_memcpy_d2h", out.ctypes.data, ptrs[1], out.nbytes, None)
    assert np.all(out == 2.5)
    hip.call("mle_arena_reset", arena)
    assert L.mle_arena_used(arena) == 0
    hip.call("mle_arena_alloc", arena, 1024, C.byref(p))
    assert p.value == ptrs[0]
    hip.call("mle_arena_destroy", arena)


def test_read_scalar_bits(hip):
    """mle_read_scalar returns the stored float bit for bit (signed zero, NaN
    payloads, subnormals, infinities), after the work queued before it on the
    same stream, on many calls in a row; null pointers are rejected."""
    vals = np.array([1.5, -0.0, np.inf, -np.inf, 1e-45, 3.4e38, -7.25e-39], np.float32)
    nan_bits = np.array([0x7FC00001, 0xFFBADBAD, 0x7F800001], np.uint32)
    bits = np.concatenate([vals.view(np.uint32), nan_bits])
    buf = hip.Buffer.from_array(bits)
    got_bits = C.c_uint32()  # read as bits: a float round trip through Python would quiet signalling NaNs
    for rep in range(3):
        for i, b in enumerate(bits):
            hip.call("mle_read_scalar", None, buf.ptr + 4 * i, C.byref(got_bits))
            assert got_bits.value == b, (rep, i, hex(got_bits.value), hex(b))
    got = C.c_float()
    # queued work first: a fill on the stream, then the read sees its value
    stream = C.c_void_p()
    hip.call("mle_stream_create", C.byref(stream))
    big = hip.Buffer.empty((1 << 22,))
    for v in (2.5, -3.75, 0.125):
        hip.call("mle_fill", stream, big.ptr, v, 1 << 22)
        hip.call("mle_read_scalar", stream, big.ptr + 4 * ((1 << 22) - 1), C.byref(got))
        assert got.value == v
    hip.call("mle_stream_destroy", stream)
    assert hip.lib().mle_read_scalar(None, None, C.byref(got)) != 0


def test_gemm_simple_fusions(hip, orc):
    """The small-product path (a lane per output element, K split over the
    workgroup's four waves) with the Linear fusions: bias in the
    epilogue (the forward on one row) and the column sum of dY (db) in the
    weight-gradient product with K = 1, against the oracle."""
    r = rng(404)
    x = r.standard_normal((1, 256), dtype=np.float32)
    W = r.standard_normal((256, 128), dtype=np.float32)
    b = r.standard_normal(128, dtype=np.float32)
    y_ref = np.zeros((1, 128), np.float32)
    orc.call("orc_bcmm", 0, orc.ptr(x), orc.ptr(W), orc.ptr(y_ref), 1, 1, 1, 256, 128, 0, 3, 0, 3, 1.0)
    y_ref += b
    gx, gW, gb, gy = B(hip, x), B(hip, W), B(hip, b), hip.Buffer.zeros((1, 128))
    hip.call("mle_gemm_ex", None, 0, 0, 1, 128, 256, 1.0, gx.ptr, 256, 0, gW.ptr, 128, 0, 0.0, gy.ptr, 128, 0, 1, None,
             gb.ptr, None, 0)
    assert_close(gy.numpy(), y_ref, what="one-row Linear forward", **MM)
    dy = r.standard_normal((1, 128), dtype=np.float32)
    dW0 = r.standard_normal((256, 128), dtype=np.float32)
    db0 = r.standard_normal(128, dtype=np.float32)
    dW_ref, db_ref = dW0.copy(), db0.copy()
    orc.call("orc_bcmm", 2, orc.ptr(x), orc.ptr(dy), orc.ptr(dW_ref), 1, 1, 256, 1, 128, 1, 3, 3, 0, 1.0)
    orc.call("orc_bcompress", orc.ptr(dy), orc.ptr(db_ref), 1, 128, 1.0)
    gdy, gdW, gdb = B(hip, dy), B(hip, dW0), B(hip, db0)
    hip.call("mle_gemm", None, 1, 0, 256, 128, 1, 1.0, gx.ptr, 256, 0, gdy.ptr, 128, 0, 1.0, gdW.ptr, 128, 0, 1, gdb.ptr)
    assert_close(gdW.numpy(), dW_ref, what="one-row weight gradient", **MM)
    assert_close(gdb.numpy(), db_ref, what="one-row bias gradient", **MM)

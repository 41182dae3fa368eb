// ORACLE -- test infrastructure only (see oracle.cpp).
//
// CPU restatement of one training step of the benchmark configurations, built
// from the oracle primitives in the order the reference graph runs them:
// forward in topological order, backward in reverse (GraphOperations::forward /
// backward, Engine/engine.cu:3386-3432), then AdamParameter::update for every
// parameter (Engine/engine.cu:283-292).  Parameter tables are passed as arrays
// of pointers in the fixed order documented per function.
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <vector>

#define OEXPORT extern "C" __attribute__((visibility("default")))

extern "C" {
void orc_bcmm(int kind, const float* a, const float* b, float* c, int batch, int channels, int m, int n, int p,
              int backward, int fa, int fb, int fc, float scale);
void orc_bcompress(const float* x, float* y, long long rows, int cols, float scale);
void orc_bcumadd(float* x, const float* y, long long rows, int cols);
void orc_channel_squeeze(const float* x, float* avg, int batch, int depth, long long spatial, int nblocks);
void orc_broadcast_add(const float* x, const float* bias, float* out, int batch, int kernels, long long hw);
void orc_scale_add(const float* x, const float* y, float* z, float scale, long long n);
void orc_accumulate(const float* x, float* y, double scale, long long n);
void orc_scale_write(const float* x, float* y, float scale, long long n);
void orc_act_fwd(int kind, const float* x, float* y, long long n);
void orc_act_bwd(int kind, const float* x, const float* dy, float* dx, long long n);
void orc_headify(const float* in, float* out, int batch, int heads, int seq, int hd, int flag);
void orc_matpe(const float* x, float* out, int batch, int row, int col, int start_idx);
void orc_pe(float* x, int t, int dim);
void orc_softmax(const float* x, float* y, int bc, int rows, int cols, int type, int masked);
void orc_softmax_bwd(const float* y, const float* dy, float* dx, int bc, int rows, int cols, int type);
void orc_norm_fwd(const float* x, float* y, float* stats, int batch, int channels, long long hw, int groups, float eps);
void orc_norm_bwd(const float* y, const float* dy, float* dx, const float* stats, int batch, int channels, long long hw,
                  int groups, float eps, int reference_layout);
void orc_conv_fwd(const float* x, const float* w, const float* bias, float* y, int N, int Cin, int H, int W, int Cout,
                  int KH, int KW, int pad, int stride);
void orc_conv_dgrad(const float* dy, const float* w, float* dx, int N, int Cin, int H, int W, int Cout, int KH, int KW,
                    int pad, int stride);
void orc_conv_wgrad(const float* x, const float* dy, float* dw, int N, int Cin, int H, int W, int Cout, int KH, int KW,
                    int pad, int stride);
float orc_mse_loss(const float* x, const float* t, long long n);
void orc_mse_bwd(const float* x, const float* t, const float* up, float* dx, long long n);
float orc_softmax_xent_fwd(const float* logits, const float* target, float* probs, int rows, int cols);
void orc_softmax_xent_bwd(const float* probs, const float* target, const float* up, float* dl, long long n, int batch);
void orc_adam(float* out, const float* grad, long long n, int t, float* m, float* v, float b1, float b2, float eps,
              float lambda, float lr, int adamw);
void orc_gather(float* out, const float* table, const int32_t* keys, int batch, int c, int max_c, int dim);
void orc_scatter_add(float* table, const float* grad, const int32_t* keys, int batch, int c, int max_c, int dim,
                     int vocab, float scale);
void orc_onehot(float* out, const int32_t* keys, int batch, int clen, int max_clen, int vocab);
}

namespace {
using Vec = std::vector<float>;
Vec zeros(long long n) { return Vec((size_t)n, 0.0f); }

// Linear::forward (Engine/engine.cu:3536-3548) with the batch folded into rows:
// bcmm flags (3, 0, 3) then BCumAdd.
void linear_fwd(const float* x, const float* w, const float* b, float* y, long long rows, int in, int out) {
  orc_bcmm(0, x, w, y, 1, 1, (int)rows, in, out, 0, 3, 0, 3, 1.0f);
  if (b) orc_bcumadd(y, b, rows, out);
}
// Linear backward (Engine/engine.cu:3550-3563): dX += dY W^T, dW += X^T dY, db += colsum dY.
void linear_bwd(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db, long long rows,
                int in, int out) {
  orc_bcmm(1, dy, w, dx, 1, 1, (int)rows, out, in, 1, 3, 0, 3, 1.0f);
  orc_bcmm(2, x, dy, dw, 1, 1, in, (int)rows, out, 1, 3, 3, 0, 1.0f);
  if (db) orc_bcompress(dy, db, rows, out, 1.0f);
}
}  // namespace

// ---------------------------------------------------------------------------
// C1: Linear(in, hid) -> ReLU -> Linear(hid, cls) -> SoftMaxCrossEntropy, then
// Adam(W) on every parameter.
// params/grads/m/v order: W1 [in x hid], b1 [hid], W2 [hid x cls], b2 [cls].
// dx (nullable) receives the input gradient.  Returns the loss.
OEXPORT float orc_c1_step(int batch, int in, int hid, int cls, const float* x, const int32_t* labels, float** params,
                          float** grads, float** ms, float** vs, float lr, int t, int adamw, float* dx) {
  Vec h = zeros((long long)batch * hid), r = zeros((long long)batch * hid), z = zeros((long long)batch * cls);
  Vec onehot = zeros((long long)batch * cls), probs = zeros((long long)batch * cls);
  linear_fwd(x, params[0], params[1], h.data(), batch, in, hid);
  orc_act_fwd(0, h.data(), r.data(), h.size());
  linear_fwd(r.data(), params[2], params[3], z.data(), batch, hid, cls);
  orc_onehot(onehot.data(), labels, batch, 1, 1, cls);
  const float loss = orc_softmax_xent_fwd(z.data(), onehot.data(), probs.data(), batch, cls);
  Vec dz = zeros(z.size()), dr = zeros(r.size()), dh = zeros(h.size());
  Vec dxl = zeros((long long)batch * in);
  orc_softmax_xent_bwd(probs.data(), onehot.data(), nullptr, dz.data(), dz.size(), batch);
  linear_bwd(r.data(), params[2], dz.data(), dr.data(), grads[2], grads[3], batch, hid, cls);
  orc_act_bwd(0, h.data(), dr.data(), dh.data(), h.size());
  linear_bwd(x, params[0], dh.data(), dxl.data(), grads[0], grads[1], batch, in, hid);
  if (dx) memcpy(dx, dxl.data(), dxl.size() * sizeof(float));
  const long long sz[4] = {(long long)in * hid, hid, (long long)hid * cls, cls};
  if (lr != 0.0f)
    for (int i = 0; i < 4; ++i) orc_adam(params[i], grads[i], sz[i], t, ms[i], vs[i], 0.9f, 0.999f, 1e-8f, 0.01f, lr, adamw);
  return loss;
}

// ---------------------------------------------------------------------------
// C4: transformer encoder block step around MultiHeadAttention::forward
// (Engine/transformer.cu:647-661): x = Gather(E, ids) + PE; h = LN(x);
// x2 = x + MHA(h, causal); f = W2 GELU(W1 LN(x2)); x3 = x2 + f;
// logits = Wl x3; SoftMaxCrossEntropy(logits, onehot(targets), last).
// params order: E [V x D], Wq, bq, Wk, bk, Wv, bv, Wo, bo (D x D, D),
// W1 [D x F], b1 [F], W2 [F x D], b2 [D], Wl [D x V], bl [V]   (15 tensors).
// ids / targets: int32 [B x S].  exact_bmmabt = 0 reproduces the reference's
// BMMABT backward for B (bcmmT(A, dZ), Engine/engine.cu:2307); 1 uses dZ^T A.
// lr == 0 skips the AdamW update.  Returns the loss.
OEXPORT float orc_c4_step(int B, int S, int D, int H, int F, int V, const int32_t* ids, const int32_t* targets,
                          float** params, float** grads, float** ms, float** vs, float lr, int t, int exact_bmmabt) {
  const long long T = (long long)B * S;
  const int hd = D / H;
  const long long nTD = T * D, nTF = T * F, nTV = T * V, nSS = (long long)B * H * S * S;
  float *E = params[0], *Wq = params[1], *bq = params[2], *Wk = params[3], *bk = params[4], *Wv = params[5],
        *bv = params[6], *Wo = params[7], *bo = params[8], *W1 = params[9], *b1 = params[10], *W2 = params[11],
        *b2 = params[12], *Wl = params[13], *bl = params[14];
  // forward
  Vec x0 = zeros(nTD), x = zeros(nTD), h = zeros(nTD), st1 = zeros(2 * B);
  orc_gather(x0.data(), E, ids, B, S, S, D);
  orc_matpe(x0.data(), x.data(), B, S, D, 0);
  orc_norm_fwd(x.data(), h.data(), st1.data(), B, 1, (long long)S * D, 1, 1e-5f);
  Vec q = zeros(nTD), k = zeros(nTD), v = zeros(nTD);
  linear_fwd(h.data(), Wq, bq, q.data(), T, D, D);
  linear_fwd(h.data(), Wk, bk, k.data(), T, D, D);
  linear_fwd(h.data(), Wv, bv, v.data(), T, D, D);
  Vec Q = zeros(nTD), K = zeros(nTD), Vh = zeros(nTD);
  orc_headify(q.data(), Q.data(), B, H, S, hd, 0);
  orc_headify(k.data(), K.data(), B, H, S, hd, 0);
  orc_headify(v.data(), Vh.data(), B, H, S, hd, 0);
  Vec sc = zeros(nSS), scs = zeros(nSS), A = zeros(nSS);
  orc_bcmm(1, Q.data(), K.data(), sc.data(), B, H, S, hd, S, 0, 3, 3, 3, 1.0f);  // BMMABT
  const float scale = 1.0f / sqrtf((float)hd);
  orc_scale_write(sc.data(), scs.data(), scale, nSS);
  orc_softmax(scs.data(), A.data(), B * H, S, S, 1, 1);  // SOFTMASK type 1
  Vec O = zeros(nTD), o = zeros(nTD), a = zeros(nTD);
  orc_bcmm(0, A.data(), Vh.data(), O.data(), B, H, S, S, hd, 0, 3, 3, 3, 1.0f);  // BMM
  orc_headify(O.data(), o.data(), B, H, S, hd, 2);  // DeHeadify
  linear_fwd(o.data(), Wo, bo, a.data(), T, D, D);
  Vec x2 = zeros(nTD), h2 = zeros(nTD), st2 = zeros(2 * B);
  orc_scale_add(x.data(), a.data(), x2.data(), 1.0f, nTD);
  orc_norm_fwd(x2.data(), h2.data(), st2.data(), B, 1, (long long)S * D, 1, 1e-5f);
  Vec f1 = zeros(nTF), g1 = zeros(nTF), f2 = zeros(nTD), x3 = zeros(nTD);
  linear_fwd(h2.data(), W1, b1, f1.data(), T, D, F);
  orc_act_fwd(1, f1.data(), g1.data(), nTF);
  linear_fwd(g1.data(), W2, b2, f2.data(), T, F, D);
  orc_scale_add(x2.data(), f2.data(), x3.data(), 1.0f, nTD);
  Vec logits = zeros(nTV), probs = zeros(nTV), onehot = zeros(nTV);
  linear_fwd(x3.data(), Wl, bl, logits.data(), T, D, V);
  orc_onehot(onehot.data(), targets, B, S, S, V);
  const float loss = orc_softmax_xent_fwd(logits.data(), onehot.data(), probs.data(), (int)T, V);

  // backward (reverse topological order)
  Vec dlog = zeros(nTV), dx3 = zeros(nTD);
  orc_softmax_xent_bwd(probs.data(), onehot.data(), nullptr, dlog.data(), nTV, B);
  linear_bwd(x3.data(), Wl, dlog.data(), dx3.data(), grads[13], grads[14], T, D, V);
  Vec dx2 = zeros(nTD), df2 = zeros(nTD);
  orc_accumulate(dx3.data(), dx2.data(), 1.0, nTD);  // Add backward
  orc_accumulate(dx3.data(), df2.data(), 1.0, nTD);
  Vec dg1 = zeros(nTF), df1 = zeros(nTF), dh2 = zeros(nTD);
  linear_bwd(g1.data(), W2, df2.data(), dg1.data(), grads[11], grads[12], T, F, D);
  orc_act_bwd(1, f1.data(), dg1.data(), df1.data(), nTF);
  linear_bwd(h2.data(), W1, df1.data(), dh2.data(), grads[9], grads[10], T, D, F);
  orc_norm_bwd(h2.data(), dh2.data(), dx2.data(), st2.data(), B, 1, (long long)S * D, 1, 1e-5f, 1);
  Vec dx = zeros(nTD), da = zeros(nTD);
  orc_accumulate(dx2.data(), dx.data(), 1.0, nTD);
  orc_accumulate(dx2.data(), da.data(), 1.0, nTD);
  Vec do_ = zeros(nTD), dO = zeros(nTD);
  linear_bwd(o.data(), Wo, da.data(), do_.data(), grads[7], grads[8], T, D, D);
  orc_headify(do_.data(), dO.data(), B, H, S, hd, 3);  // DeHeadify backward
  Vec dA = zeros(nSS), dV = zeros(nTD);
  orc_bcmm(1, dO.data(), Vh.data(), dA.data(), B, H, S, hd, S, 1, 3, 3, 3, 1.0f);  // dA += dO V^T
  orc_bcmm(2, A.data(), dO.data(), dV.data(), B, H, S, S, hd, 1, 3, 3, 3, 1.0f);   // dV += A^T dO
  Vec dscs = zeros(nSS), dsc = zeros(nSS);
  orc_softmax_bwd(A.data(), dA.data(), dscs.data(), B * H, S, S, 1);
  orc_accumulate(dscs.data(), dsc.data(), (double)scale, nSS);  // Scale backward
  Vec dQ = zeros(nTD), dK = zeros(nTD);
  orc_bcmm(0, dsc.data(), K.data(), dQ.data(), B, H, S, S, hd, 1, 3, 3, 3, 1.0f);  // dA += dZ B
  if (exact_bmmabt) orc_bcmm(2, dsc.data(), Q.data(), dK.data(), B, H, S, S, hd, 1, 3, 3, 3, 1.0f);
  else orc_bcmm(3, Q.data(), dsc.data(), dK.data(), B, H, hd, S, S, 1, 3, 3, 3, 1.0f);
  Vec dq = zeros(nTD), dk = zeros(nTD), dv = zeros(nTD);
  orc_headify(dQ.data(), dq.data(), B, H, S, hd, 1);
  orc_headify(dK.data(), dk.data(), B, H, S, hd, 1);
  orc_headify(dV.data(), dv.data(), B, H, S, hd, 1);
  Vec dh = zeros(nTD);
  linear_bwd(h.data(), Wv, dv.data(), dh.data(), grads[5], grads[6], T, D, D);
  linear_bwd(h.data(), Wk, dk.data(), dh.data(), grads[3], grads[4], T, D, D);
  linear_bwd(h.data(), Wq, dq.data(), dh.data(), grads[1], grads[2], T, D, D);
  orc_norm_bwd(h.data(), dh.data(), dx.data(), st1.data(), B, 1, (long long)S * D, 1, 1e-5f, 1);
  Vec dx0 = zeros(nTD);
  orc_accumulate(dx.data(), dx0.data(), 1.0, nTD);  // MatrixPositionalEncoding backward
  orc_scatter_add(grads[0], dx0.data(), ids, B, S, S, D, V, 1.0f);

  if (lr != 0.0f) {
    const long long sz[15] = {(long long)V * D, (long long)D * D, D, (long long)D * D, D, (long long)D * D, D,
                              (long long)D * D, D, (long long)D * F, F, (long long)F * D, D, (long long)D * V, V};
    for (int i = 0; i < 15; ++i) orc_adam(params[i], grads[i], sz[i], t, ms[i], vs[i], 0.9f, 0.999f, 1e-8f, 0.01f, lr, 1);
  }
  return loss;
}

// ---------------------------------------------------------------------------
// C5: ResidualBlock::forward (Engine/diffusion.cu:129-137) with GroupNorm(groups),
// Linear time projection of PositionalEncoding(t, tdim), MSE loss, AdamW.
// params order: W1 [C x Cin x 3 x 3], b1 [C], W2 [C x C x 3 x 3], b2 [C],
// Ws [C x Cin x 1 x 1], bs [C], Wt [tdim x C], bt [C]   (8 tensors).
// exact_bcast = 0 reproduces Broadcast_Channel's bias-gradient launch of
// `width` blocks (Engine/engine.cu:1435); 1 reduces every channel.
OEXPORT float orc_c5_step(int N, int Cin, int C, int Hs, int Ws_, int groups, int tdim, int t, const float* x,
                          const float* noise, float** params, float** grads, float** ms, float** vs, float lr, int ts,
                          int exact_bcast) {
  const long long hw = (long long)Hs * Ws_;
  const long long nC = (long long)N * C * hw;
  float *W1 = params[0], *b1 = params[1], *W2 = params[2], *b2 = params[3], *Wsk = params[4], *bsk = params[5],
        *Wt = params[6], *bt = params[7];
  Vec c1 = zeros(nC), g1 = zeros(nC), s1 = zeros(nC), hh = zeros(nC), c2 = zeros(nC), g2 = zeros(nC);
  Vec sk = zeros(nC), a = zeros(nC), out = zeros(nC);
  Vec st1 = zeros(2LL * N * groups), st2 = zeros(2LL * N * groups);
  Vec temb = zeros(tdim), tm = zeros(C);
  orc_conv_fwd(x, W1, b1, c1.data(), N, Cin, Hs, Ws_, C, 3, 3, 1, 1);
  orc_norm_fwd(c1.data(), g1.data(), st1.data(), N, C, hw, groups, 1e-5f);
  orc_act_fwd(2, g1.data(), s1.data(), nC);
  orc_pe(temb.data(), t, tdim);
  linear_fwd(temb.data(), Wt, bt, tm.data(), 1, tdim, C);
  orc_broadcast_add(s1.data(), tm.data(), hh.data(), N, C, hw);
  orc_conv_fwd(hh.data(), W2, b2, c2.data(), N, C, Hs, Ws_, C, 3, 3, 1, 1);
  orc_norm_fwd(c2.data(), g2.data(), st2.data(), N, C, hw, groups, 1e-5f);
  orc_conv_fwd(x, Wsk, bsk, sk.data(), N, Cin, Hs, Ws_, C, 1, 1, 0, 1);
  orc_scale_add(g2.data(), sk.data(), a.data(), 1.0f, nC);
  orc_act_fwd(2, a.data(), out.data(), nC);
  const float loss = orc_mse_loss(out.data(), noise, nC);

  Vec dout = zeros(nC), da = zeros(nC), dg2 = zeros(nC), dsk = zeros(nC), dc2 = zeros(nC), dhh = zeros(nC);
  Vec ds1 = zeros(nC), dg1 = zeros(nC), dc1 = zeros(nC), dxin = zeros((long long)N * Cin * hw);
  Vec dtm = zeros(C), dtemb = zeros(tdim);
  orc_mse_bwd(out.data(), noise, nullptr, dout.data(), nC);
  orc_act_bwd(2, a.data(), dout.data(), da.data(), nC);
  orc_accumulate(da.data(), dg2.data(), 1.0, nC);
  orc_accumulate(da.data(), dsk.data(), 1.0, nC);
  orc_conv_wgrad(x, dsk.data(), grads[4], N, Cin, Hs, Ws_, C, 1, 1, 0, 1);
  orc_channel_squeeze(dsk.data(), grads[5], N, C, hw, C);
  orc_conv_dgrad(dsk.data(), Wsk, dxin.data(), N, Cin, Hs, Ws_, C, 1, 1, 0, 1);
  orc_norm_bwd(g2.data(), dg2.data(), dc2.data(), st2.data(), N, C, hw, groups, 1e-5f, 1);
  orc_conv_wgrad(hh.data(), dc2.data(), grads[2], N, C, Hs, Ws_, C, 3, 3, 1, 1);
  orc_channel_squeeze(dc2.data(), grads[3], N, C, hw, C);
  orc_conv_dgrad(dc2.data(), W2, dhh.data(), N, C, Hs, Ws_, C, 3, 3, 1, 1);
  orc_accumulate(dhh.data(), ds1.data(), 1.0, nC);
  orc_channel_squeeze(dhh.data(), dtm.data(), N, C, hw, exact_bcast ? C : Ws_);
  linear_bwd(temb.data(), Wt, dtm.data(), dtemb.data(), grads[6], grads[7], 1, tdim, C);
  orc_act_bwd(2, g1.data(), ds1.data(), dg1.data(), nC);
  orc_norm_bwd(g1.data(), dg1.data(), dc1.data(), st1.data(), N, C, hw, groups, 1e-5f, 1);
  orc_conv_wgrad(x, dc1.data(), grads[0], N, Cin, Hs, Ws_, C, 3, 3, 1, 1);
  orc_channel_squeeze(dc1.data(), grads[1], N, C, hw, C);
  orc_conv_dgrad(dc1.data(), W1, dxin.data(), N, Cin, Hs, Ws_, C, 3, 3, 1, 1);

  if (lr != 0.0f) {
    const long long sz[8] = {(long long)C * Cin * 9, C, (long long)C * C * 9, C, (long long)C * Cin, C,
                             (long long)tdim * C, C};
    for (int i = 0; i < 8; ++i) orc_adam(params[i], grads[i], sz[i], ts, ms[i], vs[i], 0.9f, 0.999f, 1e-8f, 0.01f, lr, 1);
  }
  return loss;
}

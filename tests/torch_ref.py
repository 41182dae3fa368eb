"""Independent float64 references written with torch CPU autograd (test
infrastructure).  They restate the benchmark steps from the mathematics of
each op -- not from the oracle's code -- so that agreement pins the oracle:
  * LayerNorm over the whole C*H*W sample = F.layer_norm(x, x.shape[1:])
  * GroupNorm = F.group_norm, gamma = 1, beta = 0
  * causal column softmax = softmax over the query axis with key > query masked
  * GELU (tanh form) = F.gelu(approximate="tanh"), SiLU = F.silu
  * softmax cross-entropy gradient (p - t) / batch = d/dlogits of
    -sum(t * log_softmax(logits)) / batch
These implement the true gradients (the oracle's exact modes); the reference's
deviations (BMMABT's B gradient, Broadcast_Channel's channel count) are pinned
separately against closed-form identities.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as Fn

D64 = torch.float64


def t64(a, grad=True):
    return torch.tensor(np.asarray(a, dtype=np.float64), dtype=D64, requires_grad=grad)


def sinusoid(rows: int, cols: int) -> torch.Tensor:
    pos = torch.arange(rows, dtype=D64)[:, None]
    i = torch.arange(cols, dtype=D64)[None, :]
    ang = pos / torch.pow(torch.tensor(10000.0, dtype=D64), (2.0 * torch.floor(i / 2)) / cols)
    return torch.where((torch.arange(cols) % 2 == 0)[None, :], torch.sin(ang), torch.cos(ang))


def c1_step(x, labels, params, batch, classes):
    W1, b1, W2, b2 = [t64(p) for p in params]
    xt = t64(x, grad=False)
    z = torch.relu(xt @ W1 + b1) @ W2 + b2
    onehot = Fn.one_hot(torch.tensor(labels, dtype=torch.long), classes).to(D64)
    (-(onehot * Fn.log_softmax(z, dim=-1)).sum() / batch).backward()
    p = torch.softmax(z, dim=-1)
    loss = float((-(onehot * torch.log(p.detach() + 1e-27))).sum() / p.numel())
    return loss, [t.grad.numpy() for t in (W1, b1, W2, b2)]


def c4_step(ids, tgt, params, B, S, D, H, F, V):
    ps = [t64(p) for p in params]
    E, Wq, bq, Wk, bk, Wv, bv, Wo, bo, W1, b1, W2, b2, Wl, bl = ps
    hd = D // H
    x = E[torch.tensor(ids, dtype=torch.long)] + sinusoid(S, D)[None]
    ln = lambda z: Fn.layer_norm(z, z.shape[1:], eps=1e-5)
    h = ln(x)
    heads = lambda z: z.view(B, S, H, hd).transpose(1, 2)
    Q, K, Vv = heads(h @ Wq + bq), heads(h @ Wk + bk), heads(h @ Wv + bv)
    sc = (Q @ K.transpose(-1, -2)) * (1.0 / math.sqrt(hd))
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), diagonal=1)  # key (col) > query (row)
    A = torch.softmax(sc.masked_fill(mask, float("-inf")), dim=-2)
    o = (A @ Vv).transpose(1, 2).reshape(B, S, D)
    x2 = x + (o @ Wo + bo)
    f = Fn.gelu(ln(x2) @ W1 + b1, approximate="tanh") @ W2 + b2
    logits = (x2 + f) @ Wl + bl
    onehot = Fn.one_hot(torch.tensor(tgt, dtype=torch.long), V).to(D64)
    (-(onehot * Fn.log_softmax(logits, dim=-1)).sum() / B).backward()
    p = torch.softmax(logits, dim=-1)
    loss = float((-(onehot * torch.log(p.detach() + 1e-27))).sum() / p.numel())
    return loss, [t.grad.numpy().reshape(-1) for t in ps]


def pe_timestep(t: int, dim: int) -> torch.Tensor:
    half = dim // 2
    i = torch.arange(dim, dtype=D64)
    fi = torch.where(i < half, i, i - half)
    ang = t * torch.exp(-fi * math.log(10000.0) / (half - 1))
    return torch.where(i < half, torch.cos(ang), torch.sin(ang))


def c5_step(x, noise, t, params, groups):
    ps = [t64(p) for p in params]
    W1, b1, W2, b2, Ws, bs, Wt, bt = ps
    xt = t64(x, grad=False)
    h = Fn.silu(Fn.group_norm(Fn.conv2d(xt, W1, b1, padding=1), groups, eps=1e-5))
    h = h + (pe_timestep(t, Wt.shape[0]) @ Wt + bt)[None, :, None, None]
    h = Fn.group_norm(Fn.conv2d(h, W2, b2, padding=1), groups, eps=1e-5)
    out = Fn.silu(h + Fn.conv2d(xt, Ws, bs))
    loss = Fn.mse_loss(out, t64(noise, grad=False))
    loss.backward()
    return float(loss.detach()), [q.grad.numpy().reshape(-1) for q in ps]

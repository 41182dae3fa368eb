"""Synthetic inputs and parameters of the benchmark configurations (C1-C5),
seeded and generated on the host with numpy, so the GPU engine and the CPU
oracle receive identical values.

Initialisations follow the configuration text; where it names none, the
reference's AdamParameter formula U(-1, 1) * sqrt(6 / (in*row*col))
(Engine/engine.cu:128-134) is used with the parameter's own shape.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def _unif(r: np.random.Generator, shape, bound: float) -> np.ndarray:
    return ((r.random(shape, dtype=np.float64) * 2.0 - 1.0) * bound).astype(np.float32)


# ---------------------------------------------------------------- C1: MLP
@dataclass
class MLPConfig:
    batch: int = 64
    inp: int = 784
    hidden: int = 256
    classes: int = 10
    lr: float = 1e-3

    def dims(self):
        return [self.batch, self.inp, self.hidden, self.classes]


def mlp_data(cfg: MLPConfig, seed: int = 0):
    r = np.random.default_rng(seed)
    x = r.random((cfg.batch, cfg.inp), dtype=np.float32)
    labels = r.integers(0, cfg.classes, cfg.batch).astype(np.int32)
    xav = lambda fi, fo: math.sqrt(6.0 / (fi + fo))  # Xavier-uniform (C1 text)
    params = [
        _unif(r, (cfg.inp, cfg.hidden), xav(cfg.inp, cfg.hidden)),
        _unif(r, (cfg.hidden,), math.sqrt(6.0 / cfg.hidden)),
        _unif(r, (cfg.hidden, cfg.classes), xav(cfg.hidden, cfg.classes)),
        _unif(r, (cfg.classes,), math.sqrt(6.0 / cfg.classes)),
    ]
    return x, labels, params


# ----------------------------------------------------- C2: flat AdamW + clip
@dataclass
class FlatConfig:
    total: int = 100_000_000
    tensors: int = 64
    lo: int = 4096
    hi: int = 8_388_608
    lr: float = 3e-4
    max_norm: float = 1.0
    steps: int = 10


def flat_sizes(cfg: FlatConfig, seed: int = 2) -> list[int]:
    """Log-uniform sizes rescaled to sum to `total`, multiples of 64, the last
    absorbing the remainder."""
    r = np.random.default_rng(seed)
    s = np.exp(r.uniform(math.log(cfg.lo), math.log(cfg.hi), cfg.tensors))
    s = s / s.sum() * cfg.total
    sizes = [max(64, int(round(v / 64.0)) * 64) for v in s[:-1]]
    sizes.append(cfg.total - sum(sizes))
    assert sizes[-1] > 0
    return sizes


def flat_data(cfg: FlatConfig, seed: int = 2):
    sizes = flat_sizes(cfg, seed)
    r = np.random.default_rng(seed + 100)
    p = r.standard_normal(cfg.total, dtype=np.float32)
    p *= 0.02  # in place: the same float32 products as p * 0.02, without a second 400 MB array
    g = r.standard_normal(cfg.total, dtype=np.float32)
    g *= 1e-3
    spikes = np.random.default_rng(seed + 200).random(cfg.total) < 0.01
    g[spikes] *= 100.0
    return sizes, p, g


# -------------------------------------------------- C3: Linear GEMM backward
@dataclass
class GemmConfig:
    m: int = 8192
    k: int = 1024
    n: int = 4096


def gemm_data(cfg: GemmConfig, seed: int = 1):
    r = np.random.default_rng(seed)
    X = r.standard_normal((cfg.m, cfg.k), dtype=np.float32)
    W = r.standard_normal((cfg.k, cfg.n), dtype=np.float32)
    dY = r.standard_normal((cfg.m, cfg.n), dtype=np.float32)
    return X, W, dY


# ------------------------------------------------ C4: transformer block step
@dataclass
class BlockConfig:
    batch: int = 32
    seq: int = 256
    d_model: int = 512
    heads: int = 8
    ffn: int = 2048
    vocab: int = 8000
    lr: float = 1e-4

    def dims(self):
        return [self.batch, self.seq, self.d_model, self.heads, self.ffn, self.vocab]

    @property
    def gemm_flop(self) -> float:
        """Forward GEMM flops x 3 (forward + dX + dW), matching the configuration's accounting."""
        T, D, F, V, S, H = self.batch * self.seq, self.d_model, self.ffn, self.vocab, self.seq, self.heads
        fwd = 2 * T * D * D * 4 + 2 * T * D * F * 2 + 2 * self.batch * H * S * S * (D // H) * 2 + 2 * T * D * V
        return 3.0 * fwd


def block_data(cfg: BlockConfig, seed: int = 3):
    """Token ids U{0..V-1}: S+1 per sequence, inputs ids[:, :S], targets ids[:, 1:]."""
    r = np.random.default_rng(seed)
    ids = r.integers(0, cfg.vocab, (cfg.batch, cfg.seq + 1)).astype(np.int32)
    inputs = np.ascontiguousarray(ids[:, : cfg.seq])
    targets = np.ascontiguousarray(ids[:, 1:])
    D, F, V = cfg.d_model, cfg.ffn, cfg.vocab
    lin = lambda i, o: [_unif(r, (i, o), math.sqrt(6.0 / (i * o))), _unif(r, (o,), math.sqrt(6.0 / o))]
    params = [(r.standard_normal((V, D), dtype=np.float32) * 0.02).astype(np.float32)]
    for _ in range(4):
        params += lin(D, D)
    params += lin(D, F) + lin(F, D) + lin(D, V)
    return inputs, targets, params


# ------------------------------------------------- C5: U-Net residual block
@dataclass
class ResBlockConfig:
    batch: int = 16
    cin: int = 64
    cout: int = 128
    h: int = 64
    w: int = 64
    groups: int = 32
    tdim: int = 256
    lr: float = 1e-4

    def dims(self, t: int):
        return [self.batch, self.cin, self.cout, self.h, self.w, self.groups, self.tdim, t]

    @property
    def conv_flop(self) -> float:
        hw = self.h * self.w
        f = 2.0 * self.batch * hw * (self.cout * self.cin * 9 + self.cout * self.cout * 9 + self.cout * self.cin)
        return 3.0 * f


def resblock_data(cfg: ResBlockConfig, seed: int = 4):
    r = np.random.default_rng(seed)
    x = r.standard_normal((cfg.batch, cfg.cin, cfg.h, cfg.w), dtype=np.float32)
    noise = r.standard_normal((cfg.batch, cfg.cout, cfg.h, cfg.w), dtype=np.float32)
    t = int(r.integers(0, 1000))
    C, Ci, T = cfg.cout, cfg.cin, cfg.tdim
    params = [
        _unif(r, (C, Ci, 3, 3), math.sqrt(6.0 / (Ci * 9))), _unif(r, (C,), math.sqrt(6.0 / C)),
        _unif(r, (C, C, 3, 3), math.sqrt(6.0 / (C * 9))), _unif(r, (C,), math.sqrt(6.0 / C)),
        _unif(r, (C, Ci, 1, 1), math.sqrt(6.0 / Ci)), _unif(r, (C,), math.sqrt(6.0 / C)),
        _unif(r, (T, C), math.sqrt(6.0 / (T * C))), _unif(r, (C,), math.sqrt(6.0 / C)),
    ]
    return x, noise, t, params

"""Benchmark: fwd+bwd+AdamW steps/sec of the transformer encoder block (C4) on
one MI355X, driven through the C++ GraphOperations engine.

A step is one `zero_grad -> forward(calc_loss) -> backward -> ParameterUpdate`
over one batch of synthetic data (32 x 256 tokens, d 512, 8 heads, FFN 2048,
vocab 8000), with inputs and parameters resident in HBM.  The JSON line also
carries:
  roofline      the dominant kernel family (the GEMM layout with the most time),
                timed per launch with HIP events on the engine stream during the
                timed steps; achieved = algorithmic flop per launch / duration;
                traffic = that family's HBM bytes per launch from the committed
                rocprofv3 counter passes (profiles/c4_gemm_traffic.md)
  cpu_baseline  the CPU oracle (OpenMP restatement of the reference math) on a
                bounded sample of the same step, scaled to steps/s
  extras        C3 (Linear GEMM backward) TFLOP/s, C2 (fused clip + AdamW
                over 100 M parameters) GB/s, C1 (MLP, latency-bound) and C5
                (U-Net residual block, conv-bound) steps/s, measured in the same run
Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu] [--no-extras] [--only c1|c2|c3|c5]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from ml_engine_amd import hip  # noqa: E402
from ml_engine_amd.configs import (BlockConfig, FlatConfig, GemmConfig, MLPConfig, ResBlockConfig,  # noqa: E402
                                   block_data, flat_data, gemm_data, mlp_data, resblock_data)
from ml_engine_amd.models import STEP_ALL, Model  # noqa: E402

PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense fp32 matrix
PEAK_HBM = 8000.0       # GB/s
GEMM_FAMILIES = ["gemm_nn", "gemm_nt", "gemm_tn", "gemm_tt", "gemm_pair"]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def probe_read():
    n, ms, fl, by = C.c_int(), C.c_double(), C.c_double(), C.c_double()
    hip.call("mle_probe_read", C.byref(n), C.byref(ms), C.byref(fl), C.byref(by))
    return n.value, ms.value, fl.value, by.value


def build_block(cfg: BlockConfig) -> Model:
    ids, tgt, params = block_data(cfg, seed=3)
    m = Model("block", cfg.dims(), seed=3)
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, ids)
    m.input(1, tgt)
    m.sync()
    return m


def measured_traffic(fam: str):
    """HBM bytes per launch of a GEMM family from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (profiles/c4_gemm_traffic.md), or None."""
    try:
        data = json.loads((ROOT / "profiles" / "c4_gemm_traffic.json").read_text())
        return round(data[fam]["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def dominant_family(m: Model, lr: float) -> str:
    """One probed step per GEMM layout (untimed); the layout with the most time wins."""
    best, best_ms = GEMM_FAMILIES[0], -1.0
    for fam in GEMM_FAMILIES:
        hip.call("mle_probe_arm", fam.encode())
        m.step(lr, STEP_ALL)
        m.sync()
        n, ms, _, _ = probe_read()
        log(f"[bench] probe {fam}: {n} launches, {ms:.3f} ms per step")
        if ms > best_ms:
            best, best_ms = fam, ms
    hip.call("mle_probe_arm", None)
    return best


def cpu_baseline(cfg: BlockConfig, sample_batch: int) -> dict:
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as orc  # the CPU restatement; only this leg loads it

    scfg = BlockConfig(batch=sample_batch, seq=cfg.seq, d_model=cfg.d_model, heads=cfg.heads, ffn=cfg.ffn,
                       vocab=cfg.vocab, lr=cfg.lr)
    ids, tgt, params = block_data(scfg, seed=3)
    op = [np.ascontiguousarray(p.reshape(-1)).copy() for p in params]
    og = [np.zeros_like(p) for p in op]
    om = [np.zeros_like(p) for p in op]
    ov = [np.zeros_like(p) for p in op]
    T = orc.ptr_table
    threads = int(orc.call("orc_num_threads"))
    t0 = time.perf_counter()
    orc.call("orc_c4_step", scfg.batch, scfg.seq, scfg.d_model, scfg.heads, scfg.ffn, scfg.vocab, orc.ptr(ids),
             orc.ptr(tgt), T(op), T(og), T(om), T(ov), scfg.lr, 1, 0)
    dt = time.perf_counter() - t0
    # steps/s of the full workload: the sample is sample_batch/batch of one step's tokens
    return {"value": round((sample_batch / cfg.batch) / dt, 5), "unit": "steps/s", "cores": threads, "kind": "port",
            "sample": f"one oracle step at batch {sample_batch} of {cfg.batch} ({dt:.2f} s), scaled by "
                      f"{sample_batch}/{cfg.batch}"}


def extras_gemm() -> dict:
    """C3: dX = dY W^T and dW = X^T dY (+ fused db) at 8192 x 1024 x 4096."""
    cfg = GemmConfig()
    X, W, dY = gemm_data(cfg, seed=1)
    gX, gW, gdY = hip.Buffer.from_array(X), hip.Buffer.from_array(W), hip.Buffer.from_array(dY)
    gdX, gdW, gdb = hip.Buffer.zeros(X.shape), hip.Buffer.zeros(W.shape), hip.Buffer.zeros(cfg.n)
    M, K, N = cfg.m, cfg.k, cfg.n

    def run():
        hip.call("mle_gemm", None, 0, 1, M, K, N, 1.0, gdY.ptr, N, 0, gW.ptr, N, 0, 1.0, gdX.ptr, K, 0, 1, None)
        hip.call("mle_gemm", None, 1, 0, K, N, M, 1.0, gX.ptr, K, 0, gdY.ptr, N, 0, 1.0, gdW.ptr, N, 0, 1, gdb.ptr)

    for _ in range(3):
        run()
    hip.sync()
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    hip.sync()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    flop = 2.0 * 2.0 * M * N * K
    return {"workload": "C3 Linear backward dX, dW, db (8192x1024x4096)", "ms": round(ms, 4),
            "tflops": round(flop / ms / 1e9, 2), "frac_fp32_mfma": round(flop / ms / 1e9 / PEAK_FP32_MFMA, 4)}


def extras_adamw(steps: int = 10) -> dict:
    """C2: accumulate + clipNorm + ParameterUpdate over 100 M params in 64 tensors."""
    cfg = FlatConfig()
    sizes, p, g = flat_data(cfg, seed=2)
    m = Model("flat", [len(sizes)] + sizes, seed=2)
    off = 0
    for i, s in enumerate(sizes):
        m.set(i, p[off:off + s], 0)
        m.set(i, g[off:off + s], 1)
        off += s
    del p, g
    m.step(cfg.lr, 8, cfg.max_norm)
    m.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.step(cfg.lr, 8, cfg.max_norm)
    m.sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    m.close()
    gbs = 32.0 * cfg.total / (ms * 1e-3) / 1e9
    return {"workload": "C2 fused clip + AdamW, 100M params / 64 tensors", "ms_per_step": round(ms, 4),
            "gb_per_s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4), "bytes_per_param": 32}


def timed_steps(m: Model, lr: float, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        m.step(lr, STEP_ALL)
    m.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.step(lr, STEP_ALL)
    m.sync()
    return (time.perf_counter() - t0) * 1e3 / steps


def extras_mlp(steps: int = 200) -> dict:
    """C1: Linear 784->256 -> ReLU -> Linear 256->10 -> softmax CE, batch 64, Adam."""
    cfg = MLPConfig()
    x, labels, params = mlp_data(cfg, seed=0)
    m = Model("mlp", cfg.dims())
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, x)
    m.input(1, labels)
    ms = timed_steps(m, cfg.lr, steps, 5)
    m.close()
    return {"workload": "C1 MLP 784-256-10 step (fwd + bwd + Adam), batch 64", "ms_per_step": round(ms, 4),
            "steps_per_s": round(1e3 / ms, 1)}


def extras_resblock(steps: int = 10) -> dict:
    """C5: conv3x3 64->128, GN(32), SiLU, time projection, conv3x3 128->128, GN, 1x1 skip, MSE; AdamW."""
    cfg = ResBlockConfig()
    x, noise, t, params = resblock_data(cfg, seed=4)
    m = Model("resblock", cfg.dims(t))
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, x)
    m.input(1, noise)
    ms = timed_steps(m, cfg.lr, steps, 2)
    m.close()
    tf = cfg.conv_flop / (ms * 1e-3) / 1e12
    return {"workload": "C5 U-Net residual block step (fwd + bwd + AdamW), 16x64x64x64", "ms_per_step": round(ms, 4),
            "steps_per_s": round(1e3 / ms, 2), "conv_gflop_per_step": round(cfg.conv_flop / 1e9, 2),
            "conv_tflops_whole_step": round(tf, 2)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=8)
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c5"],
                    help="run just this secondary workload (for profiling) and print its JSON object")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (every box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    hip.init(0)
    if args.only:
        run = {"c1": lambda: extras_mlp(), "c2": lambda: extras_adamw(args.steps),
               "c3": lambda: extras_gemm(), "c5": lambda: extras_resblock(args.steps)}[args.only]
        print(json.dumps(run()), flush=True)
        return 0
    cfg = BlockConfig()
    log(f"[bench] building C4 block: {cfg}")
    m = build_block(cfg)
    for _ in range(args.warmup):
        m.step(cfg.lr, STEP_ALL)
    m.sync()
    fam = dominant_family(m, cfg.lr)
    log(f"[bench] dominant kernel family: {fam}")

    hip.call("mle_probe_arm", fam.encode())
    m.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.step(cfg.lr, STEP_ALL)
    m.sync()
    dt = time.perf_counter() - t0
    n, kms, kflop, kbytes = probe_read()
    hip.call("mle_probe_arm", None)
    ms_step = dt * 1e3 / args.steps
    log(f"[bench] {args.steps} steps in {dt:.3f} s: {ms_step:.3f} ms/step, loss {m.loss:.6g}")

    avg_ms = kms / max(n, 1)
    achieved = (kflop / max(n, 1)) / (avg_ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": fam, "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA, 4),
                "traffic": measured_traffic(fam), "alg_bytes_per_launch": round(kbytes / max(n, 1)),
                "launches": n, "avg_launch_ms": round(avg_ms, 5),
                "flop_per_launch": kflop / max(n, 1)}
    m.close()

    extras = {}
    if not args.no_extras:
        log("[bench] extras: C3 GEMM backward")
        extras["gemm_backward"] = extras_gemm()
        log("[bench] extras: C2 fused clip + AdamW")
        extras["adamw_clip"] = extras_adamw()
        log("[bench] extras: C1 MLP")
        extras["mlp"] = extras_mlp()
        log("[bench] extras: C5 residual block")
        extras["resblock"] = extras_resblock()
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle)")
        cpu = cpu_baseline(cfg, args.cpu_sample_batch)

    out = {
        "metric": "fwd+bwd+AdamW steps/sec (transformer block); HBM GB/s & MFMA % of peak",
        "value": round(1e3 / ms_step, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C4 transformer encoder block train step (fwd + bwd + AdamW)", "global_batch": cfg.batch,
                   "seq_len": cfg.seq, "d_model": cfg.d_model, "heads": cfg.heads, "ffn": cfg.ffn,
                   "vocab": cfg.vocab, "gemm_gflop_per_step": round(cfg.gemm_flop / 1e9, 2),
                   "parallelism": "single GPU"},
        "gemm_tflops_per_step": round(cfg.gemm_flop / (ms_step * 1e-3) / 1e12, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

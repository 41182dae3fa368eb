"""Summaries of rocprofv3 databases: kernel time, HBM traffic and MFMA
utilisation per kernel.

rocprofv3 writes one SQLite database per run (`-o NAME` -> NAME_results.db).
Counter runs (`--pmc`) hold at most a few counters each, so traffic needs two
runs (FETCH_SIZE, then WRITE_SIZE) and MFMA utilisation a third
(SQ_VALU_MFMA_BUSY_CYCLES with GRBM_GUI_ACTIVE).

Calibration.  FETCH_SIZE and WRITE_SIZE count KiB per dispatch as the memory
side sees them.  They are scaled by what the same counter reads for a plain
copy of N floats (N*4 bytes read, N*4 written):  factor = 4 N / counter_bytes.
MFMA utilisation = SQ_VALU_MFMA_BUSY_CYCLES / (cycles x CUs x 4 SIMDs), with
cycles = GRBM_GUI_ACTIVE per counter instance (the mean over its instances).

Usage (on the GPU box; rocprofv3 puts the program itself after `--`):
  python3 -m ml_engine_amd.profiling copy N
      a plain copy of N floats (mle_scale_write, scale 1), run 5 times: the
      calibration workload
  python3 -m ml_engine_amd.profiling trace DB STEPS [MARKER]
      markdown table of a --kernel-trace database: calls, total, average and
      per-step time of every kernel -- over the whole trace divided by STEPS,
      or with MARKER (a substring of the kernel that ends each step) over the
      last STEPS steps only
  python3 -m ml_engine_amd.profiling counters FETCH.db WRITE.db CFETCH.db CWRITE.db N [MFMA.db]
      markdown table per kernel: calibrated fetch / write bytes per launch and,
      with MFMA.db, the MFMA-busy fraction and shader clock
  python3 -m ml_engine_amd.profiling family FAMILY FETCH.db WRITE.db CFETCH.db CWRITE.db N OUT.json
      the same traffic averaged over one launch-probe family (gemm_nn, gemm_nt,
      gemm_tn, gemm_tt: a GEMM layout; gemm_pair: the Linear backward dX + dW
      launch; conv_fwd, conv_dgrad, conv_wgrad; adam_update; sqnorm; attn_fwd,
      attn_bwd), each launch with the split reduce that completes it -- the
      `traffic` bench.py reports for its roofline kernel
  python3 -m ml_engine_amd.profiling families FETCH.db WRITE.db CFETCH.db CWRITE.db N OUT.json
      `family` for every family present, into one JSON object
"""
from __future__ import annotations

import json
import re
import sqlite3
import sys
from collections import defaultdict

FAMILIES = {"gemm_nn": (0, 0), "gemm_nt": (0, 1), "gemm_tn": (1, 0), "gemm_tt": (1, 1)}
GEMM_KERNEL = re.compile(r"gemm_(?:direct_|stream_)?kernel<(\d), (\d)")
PAIR_KERNEL = re.compile(r"gemm_pair_kernel<")
COPY_KERNEL = "ScaleWriteOp"
CUS, SIMDS = 256, 4
NAME_WIDTH = 100


def short(name: str) -> str:
    return name if len(name) <= NAME_WIDTH else name[: NAME_WIDTH - 3] + "..."


def per_dispatch(db: str, counter: str) -> list[tuple[int, str, float, float]]:
    """(dispatch id, kernel name, counter value summed over instances, duration ns) per dispatch."""
    con = sqlite3.connect(db)
    rows = con.execute(
        "select dispatch_id, kernel_name, sum(value), max(duration) from counters_collection "
        "where counter_name = ? group by dispatch_id order by dispatch_id", (counter,)).fetchall()
    return [(d, name, float(v), float(t)) for d, name, v, t in rows]


def instances(db: str, counter: str) -> dict[int, int]:
    """Number of raw counter values (hardware instances) per dispatch."""
    con = sqlite3.connect(db)
    rows = con.execute(
        "select K.dispatch_id, count(*) from rocpd_pmc_event E "
        "join rocpd_info_pmc I on I.id = E.pmc_id and I.guid = E.guid "
        "join rocpd_kernel_dispatch K on K.event_id = E.event_id and K.guid = E.guid "
        "where I.name = ? group by K.dispatch_id", (counter,)).fetchall()
    return {d: n for d, n in rows}


CONV_DIRECT = re.compile(r"conv[13]_direct_kernel<(\w+)")
OTHER_FAMILIES = [("conv_wgrad", re.compile(r"conv[13]_wgrad_kernel<")),
                  ("adam_update", re.compile(r"adam(_vec)?_kernel<")),
                  ("sqnorm", re.compile(r"sqnorm_partial<")),
                  ("attn_fwd", re.compile(r"attn_(stats|fwd)_kernel<")),
                  ("attn_bwd", re.compile(r"attn_bwd_(kv|q)_kernel<"))]


def family_of(name: str) -> str | None:
    """The launch-probe family (bench.py's roofline kernels) a kernel belongs to."""
    if PAIR_KERNEL.search(name):
        return "gemm_pair"
    m = GEMM_KERNEL.search(name)
    if m:
        key = (int(m.group(1)), int(m.group(2)))
        return next((f for f, v in FAMILIES.items() if v == key), None)
    m = CONV_DIRECT.search(name)
    if m:
        return "conv_dgrad" if m.group(1) in ("true", "1") else "conv_fwd"
    return next((f for f, rx in OTHER_FAMILIES if rx.search(name)), None)


def mean(values: list[float]) -> float:
    return sum(values) / len(values) if values else float("nan")


def calibration(cfetch_db: str, cwrite_db: str, n: int) -> tuple[float, float]:
    cf = [1024.0 * v for _, k, v, _ in per_dispatch(cfetch_db, "FETCH_SIZE") if COPY_KERNEL in k]
    cw = [1024.0 * v for _, k, v, _ in per_dispatch(cwrite_db, "WRITE_SIZE") if COPY_KERNEL in k]
    return 4.0 * n / mean(cf), 4.0 * n / mean(cw)


def families(fetch_db: str, write_db: str, cfetch_db: str, cwrite_db: str, n: int) -> dict:
    """family() for every probe family that has launches in the counter runs."""
    found = {family_of(k) for _, k, _, _ in per_dispatch(fetch_db, "FETCH_SIZE")} - {None}
    return {f: family(f, fetch_db, write_db, cfetch_db, cwrite_db, n) for f in sorted(found)}


REDUCE_KERNEL = "split_reduce_kernel<"


def family_bytes(db: str, counter: str, fam: str) -> list[float]:
    """Bytes (uncalibrated) of each launch of a family: the family's kernel
    plus, when the next dispatch is a split reduce, that reduce -- it is
    launched by the same call and completes the family's output, and the
    launch probe times both."""
    rows = per_dispatch(db, counter)
    out = []
    for i, (_, k, v, _) in enumerate(rows):
        if family_of(k) != fam:
            continue
        if i + 1 < len(rows) and REDUCE_KERNEL in rows[i + 1][1]:
            v += rows[i + 1][2]
        out.append(1024.0 * v)
    return out


def family(fam: str, fetch_db: str, write_db: str, cfetch_db: str, cwrite_db: str, n: int) -> dict:
    fetch = family_bytes(fetch_db, "FETCH_SIZE", fam)
    write = family_bytes(write_db, "WRITE_SIZE", fam)
    f_fetch, f_write = calibration(cfetch_db, cwrite_db, n)
    out = {
        "family": fam,
        "launches": len(fetch),
        "fetch_bytes_per_launch_raw": mean(fetch),
        "write_bytes_per_launch_raw": mean(write),
        "copy_floats": n,
        "calibration_fetch": f_fetch,
        "calibration_write": f_write,
        "fetch_bytes_per_launch": mean(fetch) * f_fetch,
        "write_bytes_per_launch": mean(write) * f_write,
    }
    out["traffic_bytes_per_launch"] = out["fetch_bytes_per_launch"] + out["write_bytes_per_launch"]
    return out


def trace_table(db: str, steps: int, marker: str | None = None) -> str:
    """Per-kernel time over the whole trace divided by `steps`, or, with a
    marker (a substring of the kernel that ends every step, the optimizer's),
    over the last `steps` steps only: the launches after the marker's
    (steps+1)-th last dispatch up to its last one -- steady state, without the
    model's construction and warm-up."""
    con = sqlite3.connect(db)
    if marker:
        seq = con.execute("select name, duration from kernels order by start").fetchall()
        ends = [i for i, (nm, _) in enumerate(seq) if marker in nm]
        if len(ends) <= steps:
            raise SystemExit(f"trace: {len(ends)} '{marker}' dispatches, fewer than {steps} + 1")
        window = seq[ends[-1 - steps] + 1:ends[-1] + 1]
        agg: dict[str, list[float]] = defaultdict(list)
        for nm, d in window:
            agg[nm].append(d)
        rows = sorted(((nm, len(v), sum(v), sum(v) / len(v)) for nm, v in agg.items()), key=lambda r: -r[2])
    else:
        rows = con.execute("select name, count(*), sum(duration), avg(duration) from kernels group by name "
                           "order by sum(duration) desc").fetchall()
    total = sum(r[2] for r in rows)
    out = ["| kernel | calls | total us | avg us | % | us per step |", "|---|---:|---:|---:|---:|---:|"]
    for name, n, s, a in rows:
        out.append(f"| `{short(name)}` | {n} | {s / 1e3:.1f} | {a / 1e3:.2f} | {100 * s / total:.2f} | "
                   f"{s / 1e3 / steps:.1f} |")
    out.append("")
    out.append(f"All kernels: {total / 1e3 / steps:.1f} us per step.")
    return "\n".join(out)


def counter_table(fetch_db: str, write_db: str, cfetch_db: str, cwrite_db: str, n: int, mfma_db: str | None) -> str:
    f_fetch, f_write = calibration(cfetch_db, cwrite_db, n)
    acc: dict[str, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    for _, k, v, t in per_dispatch(fetch_db, "FETCH_SIZE"):
        acc[k]["fetch"].append(1024.0 * v * f_fetch)
        acc[k]["t"].append(t)
    for _, k, v, _ in per_dispatch(write_db, "WRITE_SIZE"):
        acc[k]["write"].append(1024.0 * v * f_write)
    if mfma_db:
        busy = {d: (k, v) for d, k, v, _ in per_dispatch(mfma_db, "SQ_VALU_MFMA_BUSY_CYCLES")}
        inst = instances(mfma_db, "GRBM_GUI_ACTIVE")
        for d, k, v, t in per_dispatch(mfma_db, "GRBM_GUI_ACTIVE"):
            cycles = v / max(inst.get(d, 1), 1)
            acc[k]["clock"].append(cycles / t if t > 0 else float("nan"))  # GHz
            if d in busy:
                acc[k]["mfma"].append(busy[d][1] / (cycles * CUS * SIMDS) if cycles > 0 else float("nan"))
    ct = [t for _, k, _, t in per_dispatch(cfetch_db, "FETCH_SIZE") if COPY_KERNEL in k]
    lines = [f"Calibration (copy of {n} floats): FETCH_SIZE x {f_fetch:.3f}, WRITE_SIZE x {f_write:.3f}; "
             f"the copy itself ran {mean(ct) / 1e3:.1f} us per launch in that counter run, "
             f"{8.0 * n / mean(ct):.0f} GB/s (read + write): the streaming rate of data that does not fit the "
             f"256 MB Infinity Cache, at equal reads and writes (kernels that mostly read, or whose reads that "
             f"cache serves, run faster).", ""]
    head = "| kernel | launches | avg us (counter run) | fetch MB/launch | write MB/launch | HBM MB/launch | GB/s |"
    sep = "|---|---:|---:|---:|---:|---:|---:|"
    if mfma_db:
        head += " MFMA busy | clock GHz |"
        sep += "---:|---:|"
    lines += [head, sep]
    order = sorted(acc.items(), key=lambda kv: -sum(kv[1]["t"]))
    for k, d in order:
        if not d["fetch"]:
            continue
        fe, wr, t = mean(d["fetch"]), mean(d["write"]), mean(d["t"])
        row = (f"| `{short(k)}` | {len(d['fetch'])} | {t / 1e3:.2f} | {fe / 1e6:.2f} | {wr / 1e6:.2f} | "
               f"{(fe + wr) / 1e6:.2f} | {(fe + wr) / t:.0f} |")
        if mfma_db:
            mf = mean(d["mfma"]) if d["mfma"] else float("nan")
            ck = mean(d["clock"]) if d["clock"] else float("nan")
            row += f" {100 * mf:.1f} % | {ck:.2f} |"
        lines.append(row)
    return "\n".join(lines)


def run_copy(n: int) -> None:
    from ml_engine_amd import hip

    hip.init(0)
    src, dst = hip.Buffer(4 * n), hip.Buffer(4 * n)
    hip.call("mle_fill", None, src.ptr, 1.0, n)
    for _ in range(5):
        hip.call("mle_scale_write", None, src.ptr, dst.ptr, 1.0, n)
    hip.sync()
    print(f"copy of {n} floats x 5 done", flush=True)


def main(argv: list[str]) -> int:
    if len(argv) == 2 and argv[0] == "copy":
        run_copy(int(argv[1]))
        return 0
    if len(argv) in (3, 4) and argv[0] == "trace":
        print(trace_table(argv[1], int(argv[2]), argv[3] if len(argv) == 4 else None))
        return 0
    if len(argv) in (6, 7) and argv[0] == "counters":
        print(counter_table(argv[1], argv[2], argv[3], argv[4], int(argv[5]), argv[6] if len(argv) == 7 else None))
        return 0
    if len(argv) == 7 and argv[0] == "families":
        res = families(argv[1], argv[2], argv[3], argv[4], int(argv[5]))
        with open(argv[6], "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps({k: round(v["traffic_bytes_per_launch"]) for k, v in res.items()}))
        return 0
    if len(argv) == 8 and argv[0] == "family":
        res = family(argv[1], argv[2], argv[3], argv[4], argv[5], int(argv[6]))
        with open(argv[7], "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res))
        return 0
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))

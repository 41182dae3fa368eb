"""HBM traffic per kernel launch from rocprofv3 counter databases.

rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE report KiB per dispatch (they
need separate runs).  The counters are calibrated against a plain copy of a
known size: the copy reads and writes exactly 4 bytes per float, so
    factor = 4 * n / counter_bytes
and a kernel's HBM traffic is its counter bytes times that factor.

Usage (on the GPU box; rocprofv3 puts the program itself after `--`):
  python3 -m ml_engine_amd.pmc_traffic copy N
      a plain copy of N floats (mle_scale_write with scale 1), run 5 times
  python3 -m ml_engine_amd.pmc_traffic summarize FAMILY FETCH.db WRITE.db COPY_FETCH.db COPY_WRITE.db N OUT.json
      average fetch / write bytes per launch of the GEMM family FAMILY (a
      layout: gemm_nn, gemm_nt, gemm_tn, gemm_tt; or gemm_pair, the Linear
      backward dX + dW launch), raw and calibrated
"""
from __future__ import annotations

import json
import re
import sqlite3
import sys

FAMILIES = {"gemm_nn": (0, 0), "gemm_nt": (0, 1), "gemm_tn": (1, 0), "gemm_tt": (1, 1)}
GEMM_KERNEL = re.compile(r"gemm_(?:direct_|stream_)?kernel<(\d), (\d)")
PAIR_KERNEL = re.compile(r"gemm_pair_kernel<")


def per_dispatch(db: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, counter value in bytes) per dispatch."""
    con = sqlite3.connect(db)
    rows = con.execute(
        "select dispatch_id, kernel_name, sum(value) from counters_collection where counter_name = ? "
        "group by dispatch_id order by dispatch_id", (counter,)).fetchall()
    return [(name, 1024.0 * value) for _, name, value in rows]


def family_of(name: str) -> str | None:
    if PAIR_KERNEL.search(name):
        return "gemm_pair"
    m = GEMM_KERNEL.search(name)
    if not m:
        return None
    key = (int(m.group(1)), int(m.group(2)))
    return next((f for f, v in FAMILIES.items() if v == key), None)


def mean(values: list[float]) -> float:
    return sum(values) / len(values) if values else float("nan")


def summarize(family: str, fetch_db: str, write_db: str, cfetch_db: str, cwrite_db: str, n: int) -> dict:
    fetch = [v for k, v in per_dispatch(fetch_db, "FETCH_SIZE") if family_of(k) == family]
    write = [v for k, v in per_dispatch(write_db, "WRITE_SIZE") if family_of(k) == family]
    copy = "ScaleWriteOp"
    cf = [v for k, v in per_dispatch(cfetch_db, "FETCH_SIZE") if copy in k]
    cw = [v for k, v in per_dispatch(cwrite_db, "WRITE_SIZE") if copy in k]
    f_fetch = 4.0 * n / mean(cf)
    f_write = 4.0 * n / mean(cw)
    out = {
        "family": family,
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
    if len(argv) >= 2 and argv[0] == "copy":
        run_copy(int(argv[1]))
        return 0
    if len(argv) == 8 and argv[0] == "summarize":
        res = summarize(argv[1], argv[2], argv[3], argv[4], argv[5], int(argv[6]))
        with open(argv[7], "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res))
        return 0
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))

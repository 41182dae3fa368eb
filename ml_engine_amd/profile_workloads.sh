#!/bin/bash
# Kernel-trace and counter passes for the benchmark workloads, run on the GPU
# box from the repository root:
#     bash ml_engine_amd/profile_workloads.sh [c4] [c5] [c3] [c2] [c1] [copy]
# Per workload W it writes gpurun_out/prof/W/{trace,counters}.md and
# traffic.json (HBM bytes per launch of every launch-probe family, the
# `traffic` field bench.py reads from profiles/W_traffic.json).  `copy` makes
# the calibration passes the counter tables need (run it once, first).
# Each rocprofv3 run has its own time limit; the script stops at the first
# failing step.
set -u
R=${GRAFT_REPO_ROOT:-$(pwd)}
OUT=$R/gpurun_out/prof
N=67108864
mkdir -p "$OUT"
cd /tmp && export TMPDIR=/tmp
export PYTHONPATH="$R${PYTHONPATH:+:$PYTHONPATH}"

step() {  # label limit_s log -- command...
  local label=$1 limit=$2 log=$3
  shift 4
  echo "[prof] $label" >&2
  echo "$*" >> "$OUT/commands.txt"
  timeout -k 10 "$limit" "$@" > "$log" 2>&1
  local rc=$?
  if [ $rc -ne 0 ]; then
    echo "[prof] $label failed with status $rc; last lines of $log:" >&2
    tail -5 "$log" >&2
    exit $rc
  fi
}

# bench.py arguments for the traced run, and how its per-step figures are
# taken: the last N steps between two launches of the update kernel (steady
# state), or, for C3 (no optimizer), the whole trace over its N passes.
# The profiled runs launch every kernel from the host (--no-graph): the same
# kernels the graph replays, traced one dispatch at a time.
args_trace() {
  case $1 in
    c4) echo "--steps 10 --warmup 5 --no-cpu --no-extras --no-graph" ;;
    c5) echo "--only c5 --no-cpu --no-graph --steps 10" ;;
    c3) echo "--only c3 --no-cpu" ;;                          # 40 + 40 + 2 x 5 + 10 = 100 (dX + dW) passes
    c2) echo "--only c2 --no-cpu --steps 5" ;;
    c1) echo "--only c1 --no-cpu --no-graph" ;;
  esac
}
steps_trace() {
  case $1 in c4) echo "5 adam" ;; c5) echo "5 adam" ;; c3) echo 100 ;; c2) echo "5 adam" ;; c1) echo "20 adam" ;; esac
}
args_pmc() {
  case $1 in
    c4) echo "--steps 3 --warmup 1 --no-cpu --no-extras --no-graph" ;;
    c5) echo "--only c5 --no-cpu --no-graph --steps 2" ;;
    c2) echo "--only c2 --no-cpu --steps 2" ;;
    *) args_trace "$1" ;;
  esac
}

for w in "$@"; do
  if [ "$w" = copy ]; then
    mkdir -p "$OUT/copy"
    step "copy FETCH_SIZE" 90 "$OUT/copy/f.log" -- rocprofv3 --pmc FETCH_SIZE -d "$OUT/copy/f" -o t -- \
      python3 -m ml_engine_amd.profiling copy $N
    step "copy WRITE_SIZE" 90 "$OUT/copy/w.log" -- rocprofv3 --pmc WRITE_SIZE -d "$OUT/copy/w" -o t -- \
      python3 -m ml_engine_amd.profiling copy $N
    continue
  fi
  D=$OUT/$w
  mkdir -p "$D"
  step "$w kernel trace" 300 "$D/trace.log" -- rocprofv3 --kernel-trace --stats -d "$D/trace" -o t -- \
    python3 "$R/bench.py" $(args_trace $w)
  step "$w FETCH_SIZE" 240 "$D/f.log" -- rocprofv3 --pmc FETCH_SIZE -d "$D/f" -o t -- python3 "$R/bench.py" $(args_pmc $w)
  step "$w WRITE_SIZE" 240 "$D/w.log" -- rocprofv3 --pmc WRITE_SIZE -d "$D/w" -o t -- python3 "$R/bench.py" $(args_pmc $w)
  step "$w MFMA busy" 240 "$D/m.log" -- rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE -d "$D/m" -o t -- \
    python3 "$R/bench.py" $(args_pmc $w)
  P="python3 -m ml_engine_amd.profiling"
  C=$OUT/copy
  {
    echo "Trace: rocprofv3 --kernel-trace --stats -d \$OUT/$w/trace -o t -- python3 bench.py $(args_trace $w)"
    echo "Summary: python3 -m ml_engine_amd.profiling trace t_results.db $(steps_trace $w)"
    echo ""
    $P trace "$D/trace/t_results.db" $(steps_trace $w)
  } > "$D/trace.md" || exit 1
  {
    echo "Counter runs (one rocprofv3 --pmc pass each): python3 bench.py $(args_pmc $w)"
    echo ""
    $P counters "$D/f/t_results.db" "$D/w/t_results.db" "$C/f/t_results.db" "$C/w/t_results.db" $N "$D/m/t_results.db"
  } > "$D/counters.md" || exit 1
  $P families "$D/f/t_results.db" "$D/w/t_results.db" "$C/f/t_results.db" "$C/w/t_results.db" $N "$D/traffic.json" \
    > /dev/null || exit 1
  echo "[prof] $w summaries written" >&2
done

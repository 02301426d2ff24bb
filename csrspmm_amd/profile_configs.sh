#!/bin/bash
# rocprofv3 passes behind the summaries in profiles/ (run on the MI355X box
# from the repository root; outputs under gpurun_out/prof/, summarised by
# `python -m csrspmm_amd.profile_summary`).
#
#   bash csrspmm_amd/profile_configs.sh NAME:CONFIG:ALGO[:plan|:nopanels] ...
#   bash csrspmm_amd/profile_configs.sh bench     # the default bench run, traced
#
# Per spec, five runs of csrspmm_amd/profile_run.py: a kernel trace with
# --stats (20 calls), FETCH_SIZE and WRITE_SIZE (3 calls each, with a 1 GiB
# device copy that calibrates them), TCC_HIT_sum TCC_MISS_sum VALUBusy, and
# TCC_BUSY_avr GRBM_GUI_ACTIVE TA_BUSY_avr (3 calls each).  Counters get runs
# of their own, never with a trace domain.
set -o pipefail
cd /tmp && export TMPDIR=/tmp && cd "${GRAFT_REPO_ROOT:-$(dirname "$0")/..}" || exit 1
OUT=gpurun_out/prof
mkdir -p "$OUT"
for spec in "$@"; do
  if [ "$spec" = bench ]; then
    echo "[profile] bench trace"
    timeout -k 10 300 rocprofv3 --kernel-trace --stats -d "$OUT/bench_xl/trace" -o bench_xl \
      --output-format csv -- python3 bench.py --cpu-seconds 0 --variants none --plan-algo none --configs none \
      > "$OUT/bench_xl.log" 2>&1 || exit 1
    continue
  fi
  IFS=: read -r name cfg algo mode <<< "$spec"
  extra=""
  [ "$mode" = plan ] && extra="--plan"
  [ "$mode" = nopanels ] && extra="--no-panels"
  run="python3 -m csrspmm_amd.profile_run --config $cfg --algo $algo $extra"
  echo "[profile] $name: trace"
  timeout -k 10 300 rocprofv3 --kernel-trace --stats -d "$OUT/$name/trace" -o "$name" \
    --output-format csv -- $run --calls 20 > "$OUT/$name.trace.log" 2>&1 || exit 1
  for c in FETCH_SIZE WRITE_SIZE; do
    echo "[profile] $name: $c"
    d=$(echo "$c" | cut -d_ -f1 | tr A-Z a-z)
    timeout -s KILL 120 rocprofv3 --pmc "$c" -d "$OUT/$name/$d" -o "$name" --output-format csv \
      -- $run --calls 3 --copy-mib 1024 > "$OUT/$name.$d.log" 2>&1 || exit 1
  done
  echo "[profile] $name: hit rate, VALU busy"
  timeout -s KILL 120 rocprofv3 --pmc TCC_HIT_sum TCC_MISS_sum VALUBusy -d "$OUT/$name/hit" \
    -o "$name" --output-format csv -- $run --calls 3 > "$OUT/$name.hit.log" 2>&1 || exit 1
  echo "[profile] $name: L2 and TA busy"
  timeout -s KILL 120 rocprofv3 --pmc TCC_BUSY_avr GRBM_GUI_ACTIVE TA_BUSY_avr -d "$OUT/$name/busy" \
    -o "$name" --output-format csv -- $run --calls 3 > "$OUT/$name.busy.log" 2>&1 || exit 1
done

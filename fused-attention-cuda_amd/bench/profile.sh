#!/usr/bin/env bash
# profile.sh -- rocprofv3 capture of one stage on one problem (the MI355X counterpart of
# ref:scripts/profile.sh, which runs Nsight Compute on the reference's fa_bench).
#
#   usage: profile.sh <stage> <cfg> <dtype> <outdir> [causal] [bench-workload]
#   e.g.   profile.sh 5 C64 fp16 prof/s5_C64
#          FA_FORCE_BR=64 FA_FORCE_BC=64 profile.sh 5 B8_H12_N1024_D64 fp16 prof/gpt_narrow 1
#          profile.sh 5 C64 fp16 prof/headline 0 C64      # bench.py --only --workload C64
#
# The program profiled is the torch-free fa_bench, launches back to back over 4 rotating input
# sets (FA_BENCH_FLUSH=1: a 1 GiB flush before every launch, the reference's protocol, whose
# write-back overlaps the next launch), or, when a bench-workload is named, bench.py's headline
# measurement (`bench.py --only`: three timed loops of host-issued launches over input sets twice
# the last-level cache), whose last 200 dispatches are the last timed loop. FA_FORCE_BR / FA_FORCE_BC / FA_FORCE_SPLITS, when set,
# pass through to the library and are recorded with the commands.
#
# Passes, each its own rocprofv3 run under its own time limit (counters never share a run with a
# trace domain, and each counter pass stays within the per-block counter limits: FETCH_SIZE and
# WRITE_SIZE in separate passes, at most 8 SQ counters and one GRBM counter per pass):
#   trace  --kernel-trace --stats: per-dispatch durations and launch resources
#   fetch  --pmc FETCH_SIZE   (KiB read from HBM per dispatch)
#   write  --pmc WRITE_SIZE   (KiB written to HBM per dispatch)
#   sq     --pmc instruction counts, MFMA busy and VALU/MFMA co-execution
#   stall  --pmc wave-cycles resident, waiting, and issuing by instruction type
#   lds    --pmc LDS bandwidth and bank conflicts
# then prof_summary.py turns the CSVs into <outdir>/summary.md. rocprofv3 is a Python script; it
# is run by the interpreter directly, and the program under it is fa_bench or python3 itself, so
# no launcher sits between the profiler and the program (the profiler library initialises the
# GPU before the program runs, and a process that has done so must not exec another program).
set -euo pipefail
STAGE=${1:?usage: profile.sh <stage> <cfg> <dtype> <outdir> [causal] [bench-workload]}
CFG=${2:?cfg}; DTYPE=${3:?dtype}; OUT=${4:?outdir}; CAUSAL=${5:-0}; WORKLOAD=${6:-}
HERE=$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
ROCPROFV3=${ROCPROFV3:-/opt/rocm/bin/rocprofv3}
mkdir -p "$OUT"
OUT=$(cd "$OUT" && pwd)
export TMPDIR=/tmp
# Provenance for fa_bench's CSV row, resolved here: fa_bench itself starts no other program.
FA_COMMIT=${FA_COMMIT:-$(git -C "$HERE" rev-parse --short HEAD 2>/dev/null || echo unknown)}
FA_ROCPROF_VERSION=${FA_ROCPROF_VERSION:-$(python3 "$ROCPROFV3" --version 2>/dev/null | head -1 || true)}
export FA_COMMIT FA_ROCPROF_VERSION
if [ -n "$WORKLOAD" ]; then
  TRACE_PROG=(python3 "$ROOT/bench.py" --only --workload "$WORKLOAD" --stage "$STAGE" --steps 200)
  PMC_PROG=(python3 "$ROOT/bench.py" --only --workload "$WORKLOAD" --stage "$STAGE" --steps 10 --warmup 2)
  LAST=200
else
  BENCH=$HERE/fa_bench
  [ -x "$BENCH" ] || { echo "profile.sh: $BENCH is not built (python fused-attention-cuda_amd/build.py)"; exit 1; }
  TRACE_PROG=("$BENCH" --stage "$STAGE" --cfg "$CFG" --dtype "$DTYPE" --causal "$CAUSAL" --iters 20 --warmup 3
              --flush "${FA_BENCH_FLUSH:-0}")
  PMC_PROG=("${TRACE_PROG[@]}")
  LAST=0
fi
FORCED=""
for var in FA_FORCE_BR FA_FORCE_BC FA_FORCE_SPLITS; do
  if [ -n "${!var:-}" ]; then FORCED="$FORCED$var=${!var} "; fi
done
META=$OUT/commands.txt
: > "$META"
cat > "$OUT/meta.txt" <<EOF
stage=$STAGE
cfg=$CFG
dtype=$DTYPE
causal=$CAUSAL
workload=$WORKLOAD
forced=$FORCED
last=$LAST
EOF
pass() {  # name, program array name, rocprofv3 options...
  local name=$1 prog=$2; shift 2
  local -n p=$prog
  local cmd=(python3 "$ROCPROFV3" "$@" --output-format csv -d "$OUT/$name" -o "$name" -- "${p[@]}")
  echo "cd /tmp && ${FORCED}${cmd[*]}" >> "$META"
  echo "[profile.sh] $(date +%T) pass $name ${FORCED}" >&2
  (cd /tmp && timeout -k 10 -s KILL 120 "${cmd[@]}" > "$OUT/$name.log" 2>&1)
}
pass trace TRACE_PROG --kernel-trace --stats
pass fetch PMC_PROG --pmc FETCH_SIZE
pass write PMC_PROG --pmc WRITE_SIZE
pass sq PMC_PROG --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS \
  SQ_INSTS_VALU_TRANS_F32 SQ_VALU_MFMA_COEXEC_CYCLES SQ_WAVES SQ_INSTS_SALU GRBM_GUI_ACTIVE
pass stall PMC_PROG --pmc SQ_WAVE_CYCLES SQ_BUSY_CU_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY \
  SQ_ACTIVE_INST_ANY SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE
pass lds PMC_PROG --pmc SQ_INSTS_LDS_LOAD_BANDWIDTH SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE \
  GRBM_GUI_ACTIVE
python3 "$HERE/prof_summary.py" "$OUT" > "$OUT/summary.md"
echo "[profile.sh] $(date +%T) done $OUT" >&2

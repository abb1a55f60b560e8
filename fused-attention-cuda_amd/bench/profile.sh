#!/usr/bin/env bash
# profile.sh -- rocprofv3 capture of one stage on the torch-free fa_bench (the MI355X counterpart
# of ref:scripts/profile.sh, which runs Nsight Compute on the reference's fa_bench).
#
#   usage: profile.sh <stage> <cfg> <dtype> <outdir> [causal]
#   e.g.   profile.sh 5 C64 fp16 gpurun_out/prof_s5_C64
#
# Passes, each its own rocprofv3 run under its own time limit (counters never share a run with a
# trace domain, and each counter pass stays within the per-block counter limits: FETCH_SIZE and
# WRITE_SIZE in separate passes, at most 8 SQ counters per pass):
#   trace  --kernel-trace --stats: per-kernel average duration (<outdir>/trace/*_kernel_stats.csv)
#   fetch  --pmc FETCH_SIZE   (KiB read from HBM per dispatch)
#   write  --pmc WRITE_SIZE   (KiB written to HBM per dispatch)
#   sq     --pmc MFMA busy/instruction counts/VALU-MFMA co-execution
#   lds    --pmc LDS bandwidth and bank conflicts
# then prof_summary.py turns the CSVs into <outdir>/summary.md. The program under rocprofv3 is
# fa_bench itself (no wrapper: the profiler library initialises the GPU before the program runs).
set -euo pipefail
STAGE=${1:?usage: profile.sh <stage> <cfg> <dtype> <outdir> [causal]}
CFG=${2:?cfg}; DTYPE=${3:?dtype}; OUT=${4:?outdir}; CAUSAL=${5:-0}
HERE=$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)
BENCH=$HERE/fa_bench
[ -x "$BENCH" ] || { echo "profile.sh: $BENCH is not built (python fused-attention-cuda_amd/build.py)"; exit 1; }
mkdir -p "$OUT"
OUT=$(cd "$OUT" && pwd)
export TMPDIR=/tmp
# Provenance for the CSV row, resolved here: fa_bench itself starts no other program.
FA_COMMIT=${FA_COMMIT:-$(git -C "$HERE" rev-parse --short HEAD 2>/dev/null || echo unknown)}
FA_ROCPROF_VERSION=${FA_ROCPROF_VERSION:-$(rocprofv3 --version 2>/dev/null | head -1 || true)}
export FA_COMMIT FA_ROCPROF_VERSION
ARGS=(--stage "$STAGE" --cfg "$CFG" --dtype "$DTYPE" --causal "$CAUSAL" --iters 20 --warmup 3)
META=$OUT/commands.txt
: > "$META"
pass() {  # name, rocprofv3 options...
  local name=$1; shift
  local cmd=(rocprofv3 "$@" --output-format csv -d "$OUT/$name" -o "$name" -- "$BENCH" "${ARGS[@]}")
  echo "${cmd[*]}" >> "$META"
  echo "[profile.sh] pass $name"
  (cd /tmp && timeout -k 10 -s KILL 120 "${cmd[@]}" > "$OUT/$name.log" 2>&1)
}
pass trace --kernel-trace --stats
pass fetch --pmc FETCH_SIZE
pass write --pmc WRITE_SIZE
pass sq --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS \
  SQ_INSTS_VALU_TRANS_F32 SQ_VALU_MFMA_COEXEC_CYCLES GRBM_GUI_ACTIVE
pass lds --pmc SQ_INSTS_LDS_LOAD_BANDWIDTH SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_WAIT_INST_LDS \
  GRBM_GUI_ACTIVE
python3 "$HERE/prof_summary.py" "$OUT" --stage "$STAGE" --cfg "$CFG" --dtype "$DTYPE" \
  --causal "$CAUSAL" > "$OUT/summary.md"
cat "$OUT/summary.md"

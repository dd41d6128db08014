#!/usr/bin/env bash
# rocprofv3 counter report of the attention kernel, run on the standalone driver (dev/fa_dev),
# so only the kernel and a few copies are in the trace.
#
#   dev/counters.sh [name] [B H N D causal [variant]]     default: cfg4 1 16 16384 128 0 opt
#   OUT=out/counters/x dev/counters.sh cfg2c 4 16 4096 128 1
#   FA_DEV_ARGS="--std 0.5 --boost-keys 0.01:8" dev/counters.sh cfg5 16 32 2048 64 1
#       (FA_DEV_ARGS: extra fa_dev input options, e.g. the many-heads config's inputs)
#
# Writes OUT (default out/counters/<name>): one rocprofv3 directory per pass and
# summary.md, made by dev/counters.py. Passes (rocprofv3 collects each counter set in one run
# of its own; a set stays within 8 SQ, 4 TCC and 2 GRBM counters):
#   trace   kernel trace + per-kernel stats (durations)
#   pmcA    MFMA busy cycles, instruction mix (VALU, MFMA, LDS), LDS bank conflicts, GRBM active
#   pmcB    MFMA/VALU co-execution, waits on LDS and on anything, active-instruction cycles,
#           transcendental count
#   fetch   FETCH_SIZE (HBM/MALL reads, KiB per dispatch)
#   write   WRITE_SIZE (writes, KiB per dispatch)
# Each pass runs under `timeout -s KILL`, and the script stops at the first pass that fails.
# Counterpart of the reference's profile/ncu.sh:43-58 (Nsight Compute sections on fa_dev).
set -euo pipefail
here=$(cd "$(dirname "$0")" && pwd)
NAME=${1:-cfg4}
shift || true
ARGS=("$@")
if [[ ${#ARGS[@]} -eq 0 ]]; then ARGS=(1 16 16384 128 0); fi
VARIANT=opt
if [[ ${#ARGS[@]} -ge 6 ]]; then VARIANT=${ARGS[5]}; ARGS=("${ARGS[@]:0:5}"); fi
BIN="$here/fa_dev"
if [[ ! -x $BIN ]]; then
    echo "build the driver first: python3 $here/../fa_build.py --only dev" >&2
    exit 2
fi
OUT=${OUT:-out/counters/$NAME}
mkdir -p "$OUT"
export TMPDIR=${TMPDIR:-/tmp}
# 1 checked launch, warmup launches for WARMUP_MS (default 100 ms: the clock ramps), 3 timed
read -r -a EXTRA <<< "${FA_DEV_ARGS:-}"
RUN=("$BIN" "${ARGS[@]}" 3 "$VARIANT" --warmup-ms "${WARMUP_MS:-100}" "${EXTRA[@]}")

pass() {
    local name=$1
    shift
    echo "== pass $name" >&2
    timeout -s KILL "${PASS_TIMEOUT:-120}" rocprofv3 "$@" --output-format csv -d "$OUT/$name" \
        -o run -- "${RUN[@]}" > "$OUT/$name.log" 2>&1 || {
        echo "pass $name failed; see $OUT/$name.log" >&2
        tail -n 20 "$OUT/$name.log" >&2
        exit 1
    }
    tail -n 2 "$OUT/$name.log" >&2
}

pass trace --kernel-trace --stats
pass pmcA --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU \
    SQ_INSTS_MFMA SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE
pass pmcB --pmc SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS SQ_WAIT_INST_ANY \
    SQ_VALU_MFMA_COEXEC_CYCLES SQ_INSTS_VALU_TRANS_F32 SQ_ACTIVE_INST_ANY SQ_WAIT_ANY
pass fetch --pmc FETCH_SIZE
pass write --pmc WRITE_SIZE

python3 "$here/counters.py" "$OUT" --shape "${ARGS[@]}" --variant "$VARIANT" \
    --command "${FA_DEV_ARGS:+FA_DEV_ARGS=\"$FA_DEV_ARGS\" }dev/counters.sh $NAME ${ARGS[*]} $VARIANT" > "$OUT/summary.md"
echo "summary: $OUT/summary.md" >&2
cat "$OUT/summary.md"

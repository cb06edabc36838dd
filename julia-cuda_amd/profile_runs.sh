#!/bin/bash
# The profiler runs behind profiles/ (per-step kernels only: no cooperative launch runs under
# rocprofv3). Usage, from the repository root on the GPU box:
#     bash julia-cuda_amd/profile_runs.sh OUT [parts]
# parts (default all): trace (bench.py's timed runs under --kernel-trace: the rocprofv3 duration
# of every HIP-event figure in the bench line), traffic (FETCH_SIZE / WRITE_SIZE passes of the
# 293-token roofline kernels, calibrated by the library's copy kernel), forward (kernel
# statistics of the 293-token forward pass, per-step path). Writes raw output under OUT and the
# summaries bench.py reads under OUT/profiles_new (copy them to profiles/).
set -o pipefail
R=$(cd "$(dirname "$0")/.." && pwd)
OUT=$(cd "$1" && pwd) || exit 2
PARTS=${2:-trace,traffic,forward}
NEW=$OUT/profiles_new
mkdir -p $NEW
cd /tmp && export TMPDIR=/tmp
has() { [[ ",$PARTS," == *",$1,"* ]]; }
if has trace; then
    echo "profile: bench.py --section kernels,fused_gemm under --kernel-trace" >&2
    timeout -k 10 600 rocprofv3 --kernel-trace --stats -f csv -d $OUT/bk -o bk -- \
        python3 $R/bench.py --section kernels,fused_gemm --path per-step \
        --trace-labels $OUT/labels.json > $OUT/bk.log 2>&1 || exit $?
    python3 $R/julia-cuda_amd/kernel_trace.py $OUT/bk $OUT/labels.json \
        --out $NEW/bench_kernels_rocprof.json > $NEW/bench_kernels_rocprof.table || exit $?
fi
if has traffic; then
    for step in qkv wo wi wo_mlp; do
        for c in FETCH_SIZE WRITE_SIZE; do
            echo "profile: $c of $step at 293 tokens" >&2
            timeout -s KILL 120 rocprofv3 --pmc $c -f csv -d $OUT/pmc_${step}_$c -o pmc -- \
                python3 $R/julia-cuda_amd/kernel_bench.py --step $step --tokens 293 --iters 200 \
                --copy-mb 64 > $OUT/pmc_${step}_$c.log 2>&1 || exit $?
        done
    done
fi
if has forward; then
    echo "profile: the 293-token forward pass, per-step kernels" >&2
    timeout -k 10 300 rocprofv3 --kernel-trace --stats -f csv -d $OUT/fwd -o fwd -- \
        python3 $R/bench.py --quick --path per-step --steps 200 --warmup 20 > $OUT/fwd.log 2>&1 || exit $?
fi
echo "profile: done" >&2

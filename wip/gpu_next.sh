#!/bin/bash
# GPU checks of the branch, run from the worktree copy on the box (cd _work/wt first).
# Each step bounded; stops at the first failure.
set -o pipefail
mkdir -p ../../gpurun_out
export TMPDIR=/tmp
step() { echo "== $*"; }
step "focused tests" && timeout -k 10 900 python3 -u -m pytest -x -v --timeout 300 --timeout-method thread \
    tests/test_gpu_dot2.py tests/test_gpu_wgrad_pipelined.py tests/test_gpu_two_stream.py \
    tests/test_gpu_trib_empty_chunk.py tests/test_gpu_event.py > ../../gpurun_out/next_tests.log 2>&1 && \
step "16-slot kernels" && timeout -k 10 600 python3 -u bench.py --mode kernels --slots 16 > ../../gpurun_out/next_k16.jsonl 2> ../../gpurun_out/next_k16.err && \
step "two streams" && timeout -k 10 600 python3 -u bench.py --streams 2 --no-extra --no-cpu-baseline > ../../gpurun_out/next_s2.json 2> ../../gpurun_out/next_s2.err && \
step "one stream" && timeout -k 10 600 python3 -u bench.py --streams 1 --no-extra --no-cpu-baseline > ../../gpurun_out/next_s1.json 2> ../../gpurun_out/next_s1.err && \
step "one stream, overlapped finalize" && timeout -k 10 600 python3 -u bench.py --overlap-finalize --no-extra --no-cpu-baseline > ../../gpurun_out/next_s1o.json 2> ../../gpurun_out/next_s1o.err
rc=$?; tail -5 ../../gpurun_out/next_tests.log; exit $rc

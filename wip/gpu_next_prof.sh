#!/bin/bash
# rocprof summaries of the branch's kernels (run from the worktree copy on the box).
set -o pipefail
R=$PWD; O=$R/../../gpurun_out
cd /tmp && export TMPDIR=/tmp
timeout -k 10 600 rocprofv3 --kernel-trace --stats --output-format csv -d $O/prof_k16 -o k16 -- \
    python3 $R/bench.py --mode kernels --slots 16 > $O/prof_k16.out 2>&1 && \
timeout -k 10 600 rocprofv3 --kernel-trace --stats --output-format csv -d $O/prof_k4 -o k4 -- \
    python3 $R/bench.py --mode kernels --slots 4 > $O/prof_k4.out 2>&1 && \
timeout -k 10 600 rocprofv3 --kernel-trace --stats --output-format csv -d $O/prof_s2 -o s2 -- \
    python3 $R/bench.py --streams 2 --steps 3 --warmup 1 --no-cpu-baseline --no-extra > $O/prof_s2.out 2>&1
rc=$?; tail -3 $O/prof_s2.out; exit $rc

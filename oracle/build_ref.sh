#!/usr/bin/env bash
# Builds the reference's own CPU-side programs from their sources where they lie
# under the reference checkout, into oracle/_ref/.  These binaries are checkers
# (golden-vector and fixture generators, and the cpu_cli baseline); nothing of the
# reference's source is written into this repository: the one slice that is not a
# whole translation unit (the host functions of the fastscan unit test) is piped to
# the compiler on stdin.
#
#   oracle/build_ref.sh [REFERENCE_DIR]     (default /root/reference)
#
# Programs built (all with g++ -O3 -std=c++20, no -march, so no FMA contraction):
#   cpu_cli          src/cpu_cli.cpp           (reference CPU search CLI, JSON on stdin)
#   build_graph      src/build_graph.cpp       (Vamana builder, OpenMP)
#   build_rabitq     src/build_rabitq.cpp      (RaBitQ codebook builder, OpenMP)
#   replicate_queries src/replicate_queries.cpp (fvecs/ivecs tiler)
#   ref_fastscan     unittest/test_fastscan.cu:54-145 host functions + oracle/ref_fastscan_main.inc
set -euo pipefail
REF="${1:-/root/reference}"
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
OUT="$HERE/_ref"
if [ ! -d "$REF/src" ]; then
    echo "build_ref: reference not found at $REF (skipping)" >&2
    exit 0
fi
mkdir -p "$OUT"
CXX="${CXX:-g++}"
FLAGS=(-O3 -std=c++20 -I "$REF/include" -I "$REF/3rd")

pids=()
"$CXX" "${FLAGS[@]}" "$REF/src/cpu_cli.cpp" -o "$OUT/cpu_cli" & pids+=($!)
"$CXX" "${FLAGS[@]}" -fopenmp "$REF/src/build_graph.cpp" -o "$OUT/build_graph" & pids+=($!)
"$CXX" "${FLAGS[@]}" -fopenmp "$REF/src/build_rabitq.cpp" -o "$OUT/build_rabitq" & pids+=($!)
"$CXX" "${FLAGS[@]}" "$REF/src/replicate_queries.cpp" -o "$OUT/replicate_queries" & pids+=($!)

# The fastscan host restatement lives in a CUDA test file; only lines 54-145
# (cpu_padded_dim .. cpu_estimate) are plain C++.  Check the slice boundaries by
# content so a changed reference fails loudly instead of compiling the wrong lines.
SRC="$REF/unittest/test_fastscan.cu"
first="$(sed -n '54p' "$SRC")"
last_fn="$(sed -n '135p' "$SRC")"
if [ "$first" != "static int cpu_padded_dim(int dim)" ] || [ "$last_fn" != "static float cpu_estimate(" ]; then
    echo "build_ref: unexpected content in $SRC:54/135; refusing to build ref_fastscan" >&2
    exit 1
fi
{ cat "$HERE/ref_fastscan_prelude.inc"; sed -n '54,145p' "$SRC"; cat "$HERE/ref_fastscan_main.inc"; } \
    | "$CXX" -O3 -std=c++20 -x c++ - -o "$OUT/ref_fastscan" & pids+=($!)
rc=0
for p in "${pids[@]}"; do wait "$p" || rc=1; done
if [ "$rc" != 0 ]; then echo "build_ref: a reference build failed" >&2; exit 1; fi
echo "build_ref: built $(ls "$OUT" | tr '\n' ' ')"

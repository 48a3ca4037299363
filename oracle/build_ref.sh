#!/bin/sh
# Builds the parts of the reference that compile from their own sources without ggml into
# oracle/_ref/: its header-only sampling / RNG / delay-pattern code behind a C shim, and its
# own sampling_test and pattern_test. Everything else in the reference needs the ggml
# submodule, which is not vendored. Needs /root/reference; outputs stay in oracle/_ref/.
set -e
REF=${REF:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT="$HERE/_ref"
if [ ! -f "$REF/src/mg/sampling.h" ]; then
    echo "reference sources not found at $REF; skipping oracle/_ref" >&2
    exit 0
fi
mkdir -p "$OUT"
CXX=${CXX:-g++}
FLAGS="-std=c++17 -O2 -ffp-contract=off -I$REF/src"
$CXX $FLAGS -shared -fPIC -o "$OUT/libref_host.so" "$HERE/ref_shim.cpp"
$CXX $FLAGS -o "$OUT/sampling_test" "$REF/tests/sampling_test.cpp"
$CXX $FLAGS -o "$OUT/pattern_test" "$REF/tests/pattern_test.cpp"
echo "built $OUT"

#!/bin/bash
# Builds the oracle (test infrastructure): the C + OpenMP restatement of the
# reference's seera_cpp GEMM/conv functions, as oracle/liboracle_seera.so.
#
# The reference's own seera_cpp (engine/src/*.cpp) is NOT built: it includes
# <cblas.h> and links -lopenblas from a system path (build_engine.py:51-52),
# neither of which exists in this image, so oracle/_ref stays empty.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
gcc -O3 -march=x86-64-v2 -fopenmp -fPIC -shared -std=c11 -Wall -Wextra \
    -o "$here/liboracle_seera.so.tmp" "$here/seera_cpp_oracle.c" -ldl
mv -f "$here/liboracle_seera.so.tmp" "$here/liboracle_seera.so"

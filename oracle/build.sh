#!/usr/bin/env bash
# Builds the CPU oracle (test infrastructure) into oracle/build/liboracle.so.
# -ffp-contract=off / no fast-math: every f32/f64 operation stays as written.
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
mkdir -p "$here/build"
gcc -O3 -std=gnu11 -fPIC -shared -ffp-contract=off -fno-fast-math -fopenmp \
    -Wall -Wextra -Wno-unused-parameter \
    "$here/oracle.c" -o "$here/build/liboracle.so.tmp" -lm
mv -f "$here/build/liboracle.so.tmp" "$here/build/liboracle.so"

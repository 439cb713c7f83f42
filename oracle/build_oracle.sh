#!/bin/sh
# Build the CPU oracle (test infrastructure) into oracle/liboracle.so.
# -ffp-contract=off + explicit fmaf: the C source's operation order is the
# arithmetic that runs; -march=x86-64-v3 makes fmaf/rintf single instructions.
set -e
cd "$(dirname "$0")"
CC=${CC:-gcc}
$CC -O2 -march=x86-64-v3 -ffp-contract=off -fno-fast-math -fno-math-errno -fopenmp -fPIC -shared -std=gnu11 \
    -Wall -Wextra -o liboracle.so.tmp kc_oracle.c -lm
mv liboracle.so.tmp liboracle.so

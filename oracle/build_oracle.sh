#!/bin/sh
# Build the CPU oracle (test infrastructure) into oracle/liboracle.so.
# -ffp-contract=off + explicit fmaf: the C source's operation order is the
# arithmetic that runs; -march=x86-64-v3 makes fmaf/rintf single instructions.
# SANITIZE=1 builds it with AddressSanitizer and UBSan (every finding fatal);
# run the tests with the sanitizer runtimes preloaded, e.g.
#   LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)" \
#   ASAN_OPTIONS=detect_leaks=0 python -m pytest tests/test_oracle_*.py
# and rebuild without SANITIZE afterwards.
set -e
cd "$(dirname "$0")"
CC=${CC:-gcc}
EXTRA=""
if [ "${SANITIZE:-0}" = "1" ]; then
    EXTRA="-g -fsanitize=address,undefined -fno-sanitize-recover=all -fno-omit-frame-pointer"
fi
$CC -O2 -march=x86-64-v3 -ffp-contract=off -fno-fast-math -fno-math-errno -fopenmp -fPIC -shared -std=gnu11 \
    -Wall -Wextra $EXTRA -o liboracle.so.tmp kc_oracle.c -lm
mv liboracle.so.tmp liboracle.so

#!/bin/bash
# Builds the C part of the CPU oracle (test infrastructure, not the product).
# -ffp-contract=off keeps every a*b+c as two IEEE binary32 operations, which
# the HIP kernels' shared GELU/exp sequence relies on for bit-identical values.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
gcc -O2 -fPIC -shared -ffp-contract=off -fno-fast-math -std=c11 -mfma \
    -o "$here/liboracle.so.tmp" "$here/fvsr_oracle.c" -lm
mv -f "$here/liboracle.so.tmp" "$here/liboracle.so"

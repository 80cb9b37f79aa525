#!/bin/sh
# Builds the CPU oracle (test infrastructure only) into oracle/libdsa_oracle.so.
# -ffp-contract=off keeps the indexer score's rounding order (no fused
# multiply-add); x86-64 SSE arithmetic has no excess precision.
set -e
here="$(cd "$(dirname "$0")" && pwd)"
gcc -O2 -fPIC -shared -fopenmp -ffp-contract=off -fno-fast-math \
    -o "$here/libdsa_oracle.so.tmp" "$here/dsa_oracle.c" -lm
mv -f "$here/libdsa_oracle.so.tmp" "$here/libdsa_oracle.so"

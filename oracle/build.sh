#!/usr/bin/env bash
# Builds the CPU oracle (test infrastructure only) into oracle/librsllm_oracle.so.
#
# -O3 -ffp-contract=off and no -ffast-math / -march: the reference is Rust,
# whose float code is never contracted into FMAs nor reassociated, built for
# the default x86-64 target.
#
# The reference itself (Rust, cargo workspace) cannot be built here: there is
# no cargo/rustc in the image, so oracle/_ref stays empty.
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
gcc -O3 -ffp-contract=off -fno-fast-math -std=c11 -Wall -Wextra -fPIC -shared -pthread \
    "$here/rsllm_oracle.c" -o "$here/librsllm_oracle.so.tmp" -lm
mv -f "$here/librsllm_oracle.so.tmp" "$here/librsllm_oracle.so"

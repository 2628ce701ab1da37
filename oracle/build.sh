#!/usr/bin/env bash
# Builds the oracle's C restatement (test infrastructure) into oracle/_build/.
# The reference itself is pure Python/torch: there is no C/C++ reference
# source to compile, so oracle/_ref/ is never produced.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
mkdir -p "$here/_build"
gcc -O2 -fPIC -shared -std=c11 -Wall -Wextra \
    -o "$here/_build/libmt19937_ref.so" "$here/mt19937_ref.c"

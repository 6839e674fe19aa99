#!/bin/bash
# Runs the CPU test suite against the AddressSanitizer + UndefinedBehaviorSanitizer build of the C oracle
# (test infrastructure: the oracle is the checker, not the product).  The interpreter is not instrumented,
# so the sanitizer runtime is preloaded; leak checking is off (the interpreter's own allocations).
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
make -C "$HERE" sanitize
export PDM_ORACLE_LIB="$HERE/_build/liboracle_asan.so"
export LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
cd "$HERE/.."
exec python -m pytest tests -q -x -m "not gpu" -p no:cacheprovider "$@"

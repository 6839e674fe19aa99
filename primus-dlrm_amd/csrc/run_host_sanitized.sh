#!/bin/bash
# Runs the C ABI tests (argument checks, struct layouts, exported symbols: host code, no GPU work) against
# the host-side AddressSanitizer + UndefinedBehaviorSanitizer build of libpdm.so.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
make -C "$HERE" -j8 sanitize-host
RT=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)
export PDM_LIB="$HERE/_build/san/libpdm.so"
export LD_PRELOAD="$RT"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
cd "$HERE/../.."
exec python -m pytest tests/test_abi.py -q -x -p no:cacheprovider "$@"

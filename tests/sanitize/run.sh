#!/bin/bash
# Runs the host-code CPU tests (safetensors pages, the header fuzz, the oracle) against the
# AddressSanitizer + UndefinedBehaviorSanitizer builds of Makefile next to this script.  CPU
# only: the GPU tests and the HIP library's kernels are not part of it.
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
REPO="$(cd "$HERE/../.." && pwd)"
make -s -C "$HERE"
ASAN_RT="$(gcc -print-file-name=libasan.so)"
UBSAN_RT="$(gcc -print-file-name=libubsan.so)"
export ASTRO_MOE_HOST_LIB="$HERE/_build/libastro_moe_host_asan.so"
export ASTRO_ORACLE_LIB="$HERE/_build/liboracle_moe_asan.so"
# the interpreter and torch are not instrumented: no leak report at exit, no new/free pairing
# checks across them; any error in the instrumented code aborts the run
export ASAN_OPTIONS="detect_leaks=0:alloc_dealloc_mismatch=0:abort_on_error=1:halt_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
cd "$REPO"
# the verification GEMV's argument checks live beside its kernels, outside the host-only build
LD_PRELOAD="$ASAN_RT:$UBSAN_RT" python -m pytest -q -p no:cacheprovider -m "not gpu" \
  --deselect tests/test_oracle_verify.py::test_abi_rejects_like_the_reference \
  --deselect tests/test_oracle_verify.py::test_abi_rejects_float32_activations \
  tests/test_pages_host.py tests/test_pages_fuzz.py tests/test_oracle_*.py "$@"

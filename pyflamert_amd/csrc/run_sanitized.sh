#!/bin/bash
# Builds the host runtime with AddressSanitizer + UBSan and runs the
# runtime's CPU tests (the .pfm loader on valid, corrupt and hostile files,
# graph validation, the quantization rewrite) against it.  CPU only: the
# sanitizers instrument the g++-built host code; the kernel library is the
# ordinary build.  Python itself is not instrumented, so the ASan runtime is
# preloaded and leak checking (of the interpreter's own allocations) is off.
# The test that loads our files with the compiled reference is left out: the
# reference's Tensor asks aligned_alloc for 64-byte alignment with sizes that
# are not multiples of 64, which ASan reports inside the reference library.
set -euo pipefail
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
ROOT="$(cd "$HERE/../.." && pwd)"
make -s -C "$HERE" -j8 all sanitize
ASAN_LIB="$(g++ -print-file-name=libasan.so)"
UBSAN_LIB="$(g++ -print-file-name=libubsan.so)"
cd "$ROOT"
LD_PRELOAD="$ASAN_LIB $UBSAN_LIB" \
ASAN_OPTIONS=detect_leaks=0:abort_on_error=1 \
UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1 \
PFR_RUNTIME_LIB="$ROOT/pyflamert_amd/lib/libpyflamert_san.so" \
    python -m pytest tests/test_runtime_cpu.py -q -p no:cacheprovider \
        --deselect tests/test_runtime_cpu.py::test_reference_loader_runs_our_files "$@"

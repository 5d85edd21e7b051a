#!/bin/bash
# Builds the parts of the reference that compile from their own C sources into
# oracle/_ref/ (test infrastructure: only tests/ load them, as the checker).
#
#   oracle/_ref/libqot_session.so   FPGA_Project/software/qmap_prompt_demo/qot_session.c
#                                   (the host session loop; qmap_one_token_runtime.h is
#                                   header-only and its MMIO runner is never called: the
#                                   tests inject their own runner)
#   oracle/_ref/test_session_host   the reference's own host test of it, run once here to
#                                   validate the build
#
# Usage: oracle/build_ref.sh [REFERENCE_ROOT]   (default /root/reference)
# Reads the reference sources where they lie and copies none of them.
set -euo pipefail
REF=${1:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT="$HERE/_ref"
SW="$REF/FPGA_Project/software"
if [ ! -f "$SW/qmap_prompt_demo/qot_session.c" ]; then
  echo "reference sources not found under $REF; nothing built" >&2
  exit 0
fi
mkdir -p "$OUT"
CFLAGS="-O2 -std=c11 -Wall -Wno-unused-function -I$SW/qmap_one_token_runtime -I$SW/qmap_prompt_demo"
gcc $CFLAGS -shared -fPIC "$SW/qmap_prompt_demo/qot_session.c" -o "$OUT/libqot_session.so"
gcc $CFLAGS "$SW/qmap_prompt_demo/test_session_host.c" "$SW/qmap_prompt_demo/qot_session.c" -o "$OUT/test_session_host"
"$OUT/test_session_host" > "$OUT/test_session_host.out"
tail -1 "$OUT/test_session_host.out"

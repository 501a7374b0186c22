#!/bin/bash
# Regenerates tests/golden/staging_trace.txt: tests/golden/staging_trace.cpp linked
# against LeanStream's own WeightManager and O_DIRECT engine (built with its
# STREAM_TESTING read hook). Needs the reference checkout (default /root/reference);
# builds only into oracle/_ref/.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
make -s -C "$root/oracle" ref-staging REF="${REF:-/root/reference}"
"$root/oracle/_ref/staging_trace_ref" > "$here/staging_trace.txt"
echo "wrote $here/staging_trace.txt ($(wc -l < "$here/staging_trace.txt") lines)"

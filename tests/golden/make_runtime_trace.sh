#!/bin/bash
# Regenerates tests/golden/runtime_trace.txt from LeanStream's own runtime sources.
# Needs the reference checkout (default /root/reference); builds only into oracle/_ref/.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
make -s -C "$root/oracle" ref-trace REF="${REF:-/root/reference}"
"$root/oracle/_ref/runtime_trace_ref" > "$here/runtime_trace.txt"
echo "wrote $here/runtime_trace.txt ($(wc -l < "$here/runtime_trace.txt") lines)"

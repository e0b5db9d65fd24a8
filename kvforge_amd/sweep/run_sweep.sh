#!/bin/bash
# Plans every shape under kvforge_amd/sweep/shapes with `kvf plan --all` and
# times every candidate on this GPU with kvf_sweep.
#
#   kvforge_amd/sweep/run_sweep.sh OUT_DIR [SHAPE ...] [-- kvf_sweep options]
#
# Writes OUT_DIR/plans/<shape>/plans.csv and OUT_DIR/sweep.csv. Run from any
# directory; machine paths in the shapes are relative to the repository root.
set -euo pipefail
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
OUT=$(mkdir -p "${1:?usage: run_sweep.sh OUT_DIR [SHAPE ...] [-- options]}" && cd "$1" && pwd)
shift
shapes=()
while [ $# -gt 0 ] && [ "$1" != "--" ]; do shapes+=("$1"); shift; done
[ "${1:-}" = "--" ] && shift
[ ${#shapes[@]} -eq 0 ] && for s in "$HERE"/shapes/*.kv; do shapes+=("$(basename "$s" .kv)"); done
list=""
for b in "${shapes[@]}"; do
  (cd "$ROOT" && kvforge_amd/bin/kvf plan "kvforge_amd/sweep/shapes/$b.kv" --all --out "$OUT/plans/$b" > /dev/null)
  list="$list${list:+,}$OUT/plans/$b/plans.csv"
  echo "planned $b: $(($(wc -l < "$OUT/plans/$b/plans.csv") - 1)) candidates"
done
"$ROOT/kvforge_amd/bin/kvf_sweep" --plans "$list" --out "$OUT/sweep.csv" "$@"

#!/usr/bin/env bash
# Regenerates philox_kat.json:
#  * "random123": the published Random123 known-answer vectors for
#    philox4x32-10 (kat_vectors, Salmon et al. SC'11 distribution);
#  * "rocrand": words drawn from rocRAND's philox4x32_10_engine(seed,
#    subsequence=stream, offset) -- an independent implementation of the same
#    (seed, stream, offset) -> word mapping the oracle and the HIP kernels use.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
tmp="$(mktemp -d)"
trap 'rm -rf "$tmp"' EXIT
hipcc -x hip --offload-arch=gfx950 -I/opt/rocm/include -O1 \
  "$here/rocrand_philox_words.cpp" -o "$tmp/words" 2>/dev/null
python3 - "$tmp/words" > "$here/philox_kat.json" <<'PY'
import json, subprocess, sys
exe = sys.argv[1]
cases = [(0, 0, 0, 8), (1, 0, 0, 8), (12345, 7, 1001, 9), (2**40 + 3, 2, 2**33 + 1, 5),
         (0xDEADBEEF, 0xFFFFFFFF, 3, 6)]
roc = []
for seed, stream, off, n in cases:
    out = subprocess.run([exe, str(seed), str(stream), str(off), str(n)], check=True,
                         capture_output=True, text=True).stdout.split()
    roc.append({"seed": seed, "stream": stream, "offset": off, "words": [int(x) for x in out]})
r123 = [
    {"ctr": ["00000000"] * 4, "key": ["00000000"] * 2,
     "out": ["6627e8d5", "e169c58d", "bc57ac4c", "9b00dbd8"]},
    {"ctr": ["ffffffff"] * 4, "key": ["ffffffff"] * 2,
     "out": ["408f276d", "41c83b0e", "a20bc7c6", "6d5451fd"]},
    {"ctr": ["243f6a88", "85a308d3", "13198a2e", "03707344"], "key": ["a4093822", "299f31d0"],
     "out": ["d16cfe09", "94fdcceb", "5001e420", "24126ea1"]},
]
json.dump({"random123": r123, "rocrand": roc}, sys.stdout, indent=1)
PY
echo "wrote $here/philox_kat.json"

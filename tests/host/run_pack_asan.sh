#!/bin/bash
# Builds the GGUF parser (pixal3d.cpp_amd/csrc/pack.cpp) for the host with
# AddressSanitizer and runs it over mutated copies of the golden packs
# (byte overwrites in the header and tensor table, truncations, splices,
# extreme 64-bit counts).  Any out-of-bounds access or leak aborts the run.
# Usage: tests/host/run_pack_asan.sh [count]   (CPU only)
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/../.." && pwd)
OUT=$(mktemp -d)
trap 'rm -rf "$OUT"' EXIT
COUNT=${1:-3000}
python3 - "$ROOT" "$OUT" "$COUNT" <<'PY'
import pathlib, random, sys
root, out, count = pathlib.Path(sys.argv[1]), pathlib.Path(sys.argv[2]), int(sys.argv[3])
sys.path.insert(0, str(root / "oracle"))
import pack_oracle as G
rng = random.Random(7)
bases = []
for stem in ("pack_flow_f16", "pack_decoder_f16", "pack_flow_bf16"):
    p = root / "tests" / "golden" / f"{stem}.gguf"
    bases.append((p.read_bytes(), G.load_pack_info(p).data_offset))
extremes = [(2**63 - 1).to_bytes(8, "little"), (2**64 - 1).to_bytes(8, "little"),
            (1 << 40).to_bytes(8, "little"), bytes(8)]
for i in range(count):
    data, head = rng.choice(bases)
    data = bytearray(data)
    for _ in range(rng.randint(1, 4)):
        lim = min(head, len(data))
        if lim < 8:
            break
        kind = rng.choice(["byte", "byte", "byte", "truncate", "splice", "u64"])
        if kind == "byte":
            data[rng.randrange(lim)] = rng.randrange(256)
        elif kind == "u64":
            at = rng.randrange(lim - 7)
            data[at:at + 8] = rng.choice(extremes + [rng.randrange(1 << 32).to_bytes(8, "little")])
        elif kind == "truncate":
            del data[rng.randrange(len(data)):]
        else:
            at = rng.randrange(lim + 1)
            data[at:at] = bytes(rng.randrange(256) for _ in range(rng.randint(1, 24)))
    (out / f"m{i:05d}.gguf").write_bytes(bytes(data))
PY
SRC=$ROOT/pixal3d.cpp_amd/csrc
/opt/rocm/bin/hipcc -O1 -g -std=c++17 -I"$ROOT/include" -I"$SRC" -Xarch_host -fsanitize=address \
    -fno-omit-frame-pointer -o "$OUT/driver" "$ROOT/tests/host/pack_asan_driver.cpp" \
    "$SRC/pack.cpp" "$SRC/capi.cpp"
ASAN_OPTIONS=detect_leaks=1:abort_on_error=1 "$OUT/driver" "$OUT"/m*.gguf

#!/bin/bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of the CPU test
# infrastructure and the library's host code (no GPU needed):
#   * the oracle (oracle/refcpu.cpp) under the CPU oracle tests;
#   * the geometry, offset and LoRA-grid checks (tests/native/*_check.cpp);
#   * the split planners and C ABI host code (attn_fwd.hip, attn_bwd.hip,
#     attn_capi.cpp host halves) under tests/native/plan_check.cpp.
# Device code is built without sanitizers.  Outputs go to $OUT (default
# /tmp/mft_sanitize).  Usage: bash tests/native/sanitize.sh
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/../.." && pwd)
OUT=${OUT:-/tmp/mft_sanitize}
mkdir -p "$OUT/obj"
HIPCC=/opt/rocm/bin/hipcc
CLANG=/opt/rocm/llvm/bin/clang++
SAN_HOST="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined"
INC="-I $ROOT/include -I $ROOT/mobilefinetuner_amd/csrc"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1 UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1

echo "[sanitize] oracle under the CPU oracle tests"
g++ -O1 -g -std=c++17 -fPIC -ffp-contract=off -fsanitize=address,undefined -fno-omit-frame-pointer -shared \
    -o "$OUT/librefcpu.so" "$ROOT/oracle/refcpu.cpp"
LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)" OUT="$OUT" python3 - <<PY
import sys, os
sys.path.insert(0, "$ROOT")
from oracle import oracle as O
O.LIB_PATH = os.path.join(os.environ["OUT"], "librefcpu.so")
import pytest
sys.exit(pytest.main(["-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                      "$ROOT/tests/test_oracle.py", "$ROOT/tests/test_lm_loss_oracle.py",
                      "$ROOT/tests/test_lora_oracle.py", "$ROOT/tests/test_prologue_oracle.py"]))
PY

for t in geometry_check offsets_check lora_grid_check; do
    echo "[sanitize] $t"
    $HIPCC -x hip --offload-arch=gfx950 --cuda-host-only -O1 -g -std=c++17 $SAN_HOST $INC \
        "$ROOT/tests/native/$t.cpp" -o "$OUT/$t"
    "$OUT/$t"
done

echo "[sanitize] split planners + C ABI host code"
for f in attn_fwd.hip attn_bwd.hip attn_capi.cpp; do
    $HIPCC -x hip --offload-arch=gfx950 -O1 -g -std=c++17 -fPIC -Xclang -target-feature -Xclang -packed-fp32-ops \
        $SAN_HOST $INC -c "$ROOT/mobilefinetuner_amd/csrc/$f" -o "$OUT/obj/$f.o"
done
$HIPCC -x hip --offload-arch=gfx950 --cuda-host-only -O1 -g -std=c++17 $SAN_HOST $INC \
    -c "$ROOT/tests/native/plan_check.cpp" -o "$OUT/obj/plan_check.o"
OTHER=$(ls "$ROOT"/mobilefinetuner_amd/_build/*.o | grep -v -e '/attn_fwd.hip.o' -e '/attn_bwd.hip.o' \
        -e '/attn_capi.cpp.o' | grep -F -f <(ls "$ROOT"/mobilefinetuner_amd/csrc | sed 's/$/.o/'))
$CLANG --hip-link --offload-arch=gfx950 -fsanitize=address,undefined -fno-gpu-sanitize "$OUT"/obj/*.o $OTHER \
    -L/opt/rocm/lib -lamdhip64 -lrocblas -Wl,-rpath,/opt/rocm/lib -o "$OUT/plan_check"
HIP_VISIBLE_DEVICES= "$OUT/plan_check"
echo "[sanitize] all clean"

#!/bin/sh
# integrate_go.sh — points a go-nngpu checkout (module github.com/tsawler/gometal) at this
# library instead of its Objective-C / Metal backend. Only cgo directives, the bridge header
# and one line of fused-operations.go change; no other Go code is touched.
#
#   usage: integrate_go.sh <go-nngpu checkout> [<this repository>]
#
# 1. internal/cgo/metal_bridge.h becomes include/gonngpu.h, which declares every function the
#    Go packages call through cgo with the reference prototype (Part 1 and Part 3), so the
#    `#include "../../internal/cgo/metal_bridge.h"` lines stay as they are.
# 2. The Objective-C sources and the Metal shader file of internal/cgo are removed (go build
#    would compile the .m files; the library replaces them).
# 3. In every file with a cgo preamble, the macOS link line (-framework ...) becomes a link
#    against libgonngpu.so, and the Objective-C compile flags are dropped.
# 4. FusedLinearActivation.Forward sends ActivationType ReLU for a nil activation instead of
#    OpReLU (6, which the library reads as the ActivationType Swish).
# Then `go build ./...` in the checkout needs libgonngpu.so built (make -C go-nngpu_amd).
set -eu
dst=$1
src=${2:-$(cd "$(dirname "$0")/.." && pwd)}
lib="$src/go-nngpu_amd/lib"
[ -f "$src/include/gonngpu.h" ] || { echo "integrate_go.sh: $src/include/gonngpu.h not found" >&2; exit 1; }
[ -f "$dst/internal/cgo/metal_bridge.h" ] || { echo "integrate_go.sh: $dst is not a go-nngpu checkout" >&2; exit 1; }
cd "$dst"
cp "$src/include/gonngpu.h" internal/cgo/metal_bridge.h
rm -f internal/cgo/*.m internal/cgo/default.metal
files=$(grep -rl --include='*.go' 'import "C"' internal gpu tensor)
# shellcheck disable=SC2086
sed -i -E \
  -e "s|#cgo (darwin )?LDFLAGS: .*-framework.*|#cgo LDFLAGS: -L$lib -Wl,-rpath,$lib -lgonngpu|" \
  -e '/#cgo (darwin )?CFLAGS: .*objective-c/d' \
  $files
sed -i 's|activationType := C.int(OpReLU) // Default to ReLU|activationType := C.int(ReLU) // Default to ReLU (ActivationType 0)|' \
  gpu/matrix/fused-operations.go
grep -q 'activationType := C.int(ReLU)' gpu/matrix/fused-operations.go ||
  { echo "integrate_go.sh: the nil-activation line of fused-operations.go was not found" >&2; exit 1; }
echo "integrate_go.sh: $(echo "$files" | wc -w) cgo files now link $lib/libgonngpu.so"

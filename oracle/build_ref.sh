#!/bin/sh
# Builds oracle/_ref/libref_sampler.so from the reference's header-only sampler where it lies in the reference tree
# (test infrastructure; nothing is copied).  Skipped when the reference tree is absent.
set -e
REF=${SEEDPLANE_REFERENCE:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
[ -f "$REF/native/vulkan_decode/sampler.hpp" ] || { echo "reference sampler not found under $REF: skipped"; exit 0; }
mkdir -p "$HERE/_ref"
g++ -O2 -std=c++17 -shared -fPIC -I"$REF/native/vulkan_decode" "$HERE/ref_sampler_shim.cpp" -o "$HERE/_ref/libref_sampler.so"
echo "$HERE/_ref/libref_sampler.so"

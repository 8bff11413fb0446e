#!/bin/bash
# Builds the C++ mapper self-test (test infrastructure: links the oracle).
set -e
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(dirname "$(dirname "$HERE")")"
mkdir -p "$HERE/bin"
g++ -O1 -std=c++17 -Wall -I"$ROOT/include" -I"$ROOT/micronaut3-bug_amd/host" -I"$ROOT/oracle" \
    "$HERE/mapper_selftest.cpp" "$ROOT/oracle/liboracle.so" "$ROOT/micronaut3-bug_amd/libpetjson.so" \
    -Wl,--allow-shlib-undefined \
    -Wl,-rpath,"\$ORIGIN/../../../oracle" -Wl,-rpath,"\$ORIGIN/../../../micronaut3-bug_amd" \
    -o "$HERE/bin/mapper_selftest"

#!/bin/sh
# Builds the oracle (test infrastructure): oracle/liboracle.so from glt_oracle.c.
set -e
cd "$(dirname "$0")"
gcc -O3 -march=x86-64-v2 -fopenmp -fPIC -shared -std=c11 -Wall -o liboracle.so.tmp glt_oracle.c -lm
mv liboracle.so.tmp liboracle.so

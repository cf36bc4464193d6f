"""Build recipe of the oracle's C restatement (test infrastructure).

Compiles ``oracle/moe_route_ref.c`` with gcc into ``oracle/_build/liboracle_route.so``. No
fast-math and no FMA contraction, so the fp32 operations are exactly the ones written in the
source.

The reference itself has no native code on this path (its device arithmetic lives in the
external, un-vendored ``ttnn`` package and the HF model code is Hub remote code), so there is no
``oracle/_ref`` build.
"""
from __future__ import annotations

import os
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(ORACLE_DIR, "_build")
ROUTE_SRC = os.path.join(ORACLE_DIR, "moe_route_ref.c")
ROUTE_LIB = os.path.join(BUILD_DIR, "liboracle_route.so")


def build() -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = ROUTE_LIB + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", ROUTE_SRC, "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    os.replace(tmp, ROUTE_LIB)
    return ROUTE_LIB


if __name__ == "__main__":
    print(build())

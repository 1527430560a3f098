"""Build recipe of the oracle (test infrastructure): oracle.cpp -> oracle/liboracle.so.

The reference itself is Rust (crates/hardshell, crates/taco-coder) and this image has no Rust
toolchain, so there is no oracle/_ref build; the C++ restatement is pinned by the reference's
golden vectors instead (tests/test_oracle.py).
"""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-pthread",
        "-mavx2", "-ffp-contract=off", "-fno-fast-math",
        os.path.join(HERE, "oracle.cpp"), "-o", LIB + ".tmp",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

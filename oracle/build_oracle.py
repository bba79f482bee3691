"""Build recipe of the CPU oracle (liboracle.so) -- test infrastructure only."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build() -> str:
    out = os.path.join(HERE, "liboracle.so")
    tmp = out + ".tmp"
    # oracle.c: the restatement of the reference's arithmetic; cpu_q8k.c: the
    # CPU baseline (candle's Q8_K dot-product path), AVX2 selected at run time
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-shared", "-fPIC",
           os.path.join(HERE, "oracle.c"), os.path.join(HERE, "cpu_q8k.c"), "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())

"""Builds the C restatement of the oracle (oracle/attn_ref.c) into oracle/libattn_oracle.so.

Test infrastructure only. The reference itself is not built here: its kernels are CUDA (no nvcc
in this image) and its oracle is Python, which is read, not run; so there is no oracle/_ref.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "attn_ref.c"
OUTPUT = HERE / "libattn_oracle.so"


def build() -> Path:
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-std=c11", "-fopenmp", "-fPIC", "-shared", str(SOURCE), "-o", str(tmp), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(f"built {build()}")

"""ORACLE — TEST INFRASTRUCTURE ONLY.  Builds oracle/liboracle.so from accept.c and
filter.c with gcc (strict IEEE binary32: no fast-math, no implicit multiply-add contraction)."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SO = HERE / "liboracle.so"


def build() -> Path:
    tmp = SO.with_suffix(".so.tmp")
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fPIC",
                    "-shared", "-o", str(tmp), str(HERE / "accept.c"), str(HERE / "filter.c"), "-lm"], check=True)
    tmp.replace(SO)
    return SO


if __name__ == "__main__":
    print(build())

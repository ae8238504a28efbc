"""Compiles libtorchure_amd.so for gfx950 with hipcc (no torch build machinery).

Flags: -O3, C++17, position-independent shared object, and the packed-fp32
target feature switched off (``-Xclang -target-feature -Xclang -packed-fp32-ops``)
so that no v_pk_{add,mul,fma}_f32 instructions are emitted.
"""

from __future__ import annotations

import os
import shutil
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_HERE)
SOURCES = [os.path.join(_HERE, "csrc", "tm_optim.hip"), os.path.join(_HERE, "csrc", "tm_ce.hip")]
INCLUDE = os.path.join(ROOT, "include")
OUTPUT = os.path.join(_HERE, "libtorchure_amd.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def command(output: str = OUTPUT, extra: list[str] | None = None) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}",
        *(extra or []),
        "-o", output,
        *SOURCES,
    ]


def build(verbose: bool = False) -> str:
    """Always recompiles; writes to a temporary name and renames into place."""
    tmp = OUTPUT + ".tmp"
    res = subprocess.run(command(tmp), capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr:
        print(res.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))

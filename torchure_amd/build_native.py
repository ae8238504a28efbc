"""Compiles the package's two native libraries (no torch build machinery):

- libtorchure_amd.so: the gfx950 kernels and the C ABI, with hipcc. Flags: -O3, C++17,
  position-independent shared object, and the packed-fp32 target feature switched off
  (``-Xclang -target-feature -Xclang -packed-fp32-ops``) so that no v_pk_{add,mul,fma}_f32
  instructions are emitted.
- _tm_host.<ext>.so: host-side list primitives (CPU only) as a Python extension, with g++
  against torch's headers and libraries.

Both are compiled in parallel.
"""

from __future__ import annotations

import os
import shutil
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_HERE)
SOURCES = [os.path.join(_HERE, "csrc", f) for f in ("tm_optim.hip", "tm_ce.hip", "tm_ce_gemm.hip")]
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


HOST_SOURCE = os.path.join(_HERE, "csrc", "tm_host.cpp")


def host_output() -> str:
    import sysconfig

    return os.path.join(_HERE, "_tm_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def host_command(output: str) -> list[str]:
    import sysconfig

    import torch

    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return [
        shutil.which("g++") or "g++", "-O2", "-std=c++17", "-shared", "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_tm_host", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-I{tdir}/include", f"-I{tdir}/include/torch/csrc/api/include",
        f"-I{sysconfig.get_paths()['include']}",
        HOST_SOURCE,
        f"-L{tdir}/lib", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{tdir}/lib",
        "-o", output,
    ]


def _start(cmd: list[str]) -> subprocess.Popen:
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def build(verbose: bool = False) -> str:
    """Always recompiles both libraries; each is written to a temporary name and renamed
    into place. Returns the kernel library's path."""
    jobs = []
    for out, cmd_of, what in ((OUTPUT, command, "hipcc"), (host_output(), host_command, "g++")):
        tmp = out + ".tmp"
        jobs.append((out, tmp, what, _start(cmd_of(tmp))))
    errors = []
    for out, tmp, what, proc in jobs:
        stdout, stderr = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"{what} failed:\n{stdout}\n{stderr}")
            continue
        if verbose and stderr:
            print(stderr)
        os.replace(tmp, out)
    if errors:
        raise RuntimeError("\n".join(errors))
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))

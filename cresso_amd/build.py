"""Build libcresso_hip.so in-tree with hipcc for gfx950.

    python -m cresso_amd.build            # or: python cresso_amd/build.py

Every *.hip file under cresso_amd/csrc/ goes into one shared library next to
this file.  Packed-FP32 instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libcresso_hip.so"
ARCH = os.environ.get("CRESSO_HIP_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources():
    return sorted(CSRC.glob("*.hip"))


HOST_SRC = CSRC / "host_batch.cpp"


def host_ext_path() -> Path:
    import sysconfig

    return HERE / ("_hostbatch" + sysconfig.get_config_var("EXT_SUFFIX"))


def host_cmd() -> list:
    """g++ line of the host bookkeeping extension (a torch C++ extension, CPU only)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce

    inc = [f"-I{d}" for d in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    libdir = ce.library_paths()[0]
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    tmp = host_ext_path().with_suffix(".tmp")
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w", str(HOST_SRC), "-o", str(tmp), *inc,
            "-DTORCH_EXTENSION_NAME=_hostbatch", "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{libdir}"]


def build(verbose: bool = False, jobs: int = 8) -> Path:
    # the host extension (slowest compile: torch headers) starts first, in parallel
    hcmd = host_cmd()
    if verbose:
        print(" ".join(hcmd), flush=True)
    hproc = subprocess.Popen(hcmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    srcs = sources()
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    common = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-I", str(HERE.parent / "include")]
    procs = []
    objs = []
    for src in srcs:
        obj = objdir / (src.stem + ".o")
        objs.append(obj)
        cmd = [hipcc(), *common, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    while procs:
        _wait(procs.pop(0))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if out.returncode != 0:
        raise RuntimeError("link failed:\n" + out.stdout.decode(errors="replace"))
    os.replace(tmp, LIB)
    hout, _ = hproc.communicate()
    if hproc.returncode != 0:
        raise RuntimeError("g++ failed on host_batch.cpp:\n" + hout.decode(errors="replace"))
    os.replace(host_ext_path().with_suffix(".tmp"), host_ext_path())
    return LIB


def _wait(item):
    src, proc = item
    out, _ = proc.communicate()
    text = out.decode(errors="replace")
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{text}")
    noise = [l for l in text.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noise:
        print(f"[{src.name}]\n" + "\n".join(noise), file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

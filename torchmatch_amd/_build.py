"""In-tree build of the native parts (gfx950 only).

Produces, next to this file:

* ``lib/libtorchmatch_amd.so`` -- the C-ABI library (``include/torchmatch_amd.h``):
  the HIP kernels in ``csrc/*.hip``, compiled by ``hipcc --offload-arch=gfx950``;
* ``_C.so`` -- torch dispatcher registrations (``csrc/torch_ops.cpp``) linked
  against the C-ABI library; loaded with ``torch.ops.load_library``;
* ``bench_probes.so`` at the repository root -- the microbenchmarks
  ``bench.py`` prices the JV kernels against (``bench_probes.hip``: LDS read
  bandwidth, wave-wide argmin latency); measurement support for the
  benchmark, not part of the package or the C ABI.

``python torchmatch_amd/_build.py`` runs it; ``__graft_entry__.build()`` calls
:func:`build` too.  hipcc cross-compiles, so no GPU is needed.
"""

from __future__ import annotations

import os
import shlex
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB_DIR = PKG / "lib"
CABI_SO = LIB_DIR / "libtorchmatch_amd.so"
OPS_SO = PKG / "_C.so"
PROBE_SRC = PKG.parent / "bench_probes.hip"
PROBE_SO = PKG.parent / "bench_probes.so"

HIP_SOURCES = ["jv_batch.hip", "jv_large.hip", "jv_unpack.hip", "sinkhorn.hip", "sinkhorn64.hip"]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 ops (the host pass
# warns that it does not know the feature; harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout)
        sys.stderr.write(res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {cmd[0]} ... {cmd[-1]}")


def build_cabi(verbose: bool = True) -> Path:
    """Compile the HIP kernels + C ABI into lib/libtorchmatch_amd.so."""
    LIB_DIR.mkdir(exist_ok=True)
    objs = []
    for src in HIP_SOURCES:
        obj = LIB_DIR / (Path(src).stem + ".o")
        _run(["hipcc", *HIPCC_FLAGS, "-I", str(INCLUDE), "-c", str(CSRC / src), "-o", str(obj)],
             verbose)
        objs.append(str(obj))
    tmp = CABI_SO.with_suffix(".so.tmp")
    _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs,
          f"-Wl,-rpath,{ROCM / 'lib'}"], verbose)
    os.replace(tmp, CABI_SO)
    for o in objs:
        Path(o).unlink(missing_ok=True)
    return CABI_SO


def build_probe(verbose: bool = True) -> Path:
    """Compile the benchmark's microbenchmarks into bench_probes.so."""
    tmp = PROBE_SO.with_suffix(".so.tmp")
    _run(["hipcc", *HIPCC_FLAGS, "-I", str(PKG.parent), "-shared", "-o", str(tmp),
          str(PROBE_SRC), f"-Wl,-rpath,{ROCM / 'lib'}"], verbose)
    os.replace(tmp, PROBE_SO)
    return PROBE_SO


def build_ops(verbose: bool = True) -> Path:
    """Compile the torch op registrations into _C.so."""
    import torch
    from torch.utils import cpp_extension as ce

    includes = ce.include_paths(device_type="cuda")
    libdirs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-Wno-unused-parameter",
        *[f"-I{p}" for p in includes],
        f"-I{INCLUDE}",
        f"-I{sysconfig.get_paths()['include']}",
        str(CSRC / "torch_ops.cpp"),
        "-o", str(OPS_SO.with_suffix(".so.tmp")),
        *[f"-L{p}" for p in libdirs],
        f"-L{LIB_DIR}",
        "-ltorchmatch_amd", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN/lib",
    ]
    _run(cmd, verbose)
    os.replace(OPS_SO.with_suffix(".so.tmp"), OPS_SO)
    return OPS_SO


def build(verbose: bool = True) -> None:
    build_cabi(verbose)
    build_ops(verbose)
    build_probe(verbose)


if __name__ == "__main__":
    build(verbose=True)

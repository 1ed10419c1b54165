"""Build recipe for the native parts of the package (explicit compiler lines, in-tree output).

Products, all written under ``domesticated_torch_mlu_ops_amd/_lib/``:

* ``libtmo_hip.so``  -- the gfx950 HIP kernels behind the plain C ABI of ``include/tmo_hip.h``.
* ``_tmo_torch.so``  -- the thin PyTorch-ROCm extension: ``tmo::torch_api`` (the prototypes of
  ``include/torch_mlu_ops.h``) plus the ``torch_mlu_ops::*`` schema registrations; it links
  ``libtmo_hip.so`` and calls only the C ABI.

The CPU oracle (test infrastructure) is built separately by ``oracle/Makefile``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
INCLUDE = REPO_DIR / "include"
OBJ_DIR = LIB_DIR / "obj"

HIP_LIB = LIB_DIR / "libtmo_hip.so"
TORCH_EXT = LIB_DIR / "_tmo_torch.so"

HIP_SOURCES = ["quant_paged.hip", "reshape_paged.hip", "dequant_paged.hip", "fused_rope.hip",
               "linear_cache.hip", "decode_attn.hip",
               "scaled_quantize.hip", "abi_info.hip"]

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# gfx950 only.  -ffp-contract=off keeps every fp32 multiply/add separately rounded (the int8
# codes must be bit-identical to IEEE arithmetic); packed fp32 VALU ops are disabled.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _atomic_link(cmd_prefix: list[str], out: Path, cmd_suffix: list[str], verbose: bool) -> None:
    tmp = out.with_name(out.name + ".tmp")
    _run(cmd_prefix + ["-o", str(tmp)] + cmd_suffix, verbose)
    os.replace(tmp, out)


def build_hip_lib(verbose: bool = False, jobs: int = 8) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = OBJ_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    _atomic_link([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"], HIP_LIB,
                 [str(o) for o in objs], verbose)
    return HIP_LIB


def _torch_paths():
    import torch
    from torch.utils.cpp_extension import include_paths, library_paths
    return include_paths(), library_paths(), bool(torch._C._GLIBCXX_USE_CXX11_ABI)


def build_torch_ext(verbose: bool = False) -> Path:
    incs, libs, cxx11 = _torch_paths()
    py_inc = sysconfig.get_paths()["include"]
    cxx = shutil.which("g++") or "g++"
    cmd = [cxx, "-shared", "-fPIC", "-O2", "-std=c++17",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(cxx11)}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-DTORCH_EXTENSION_NAME=_tmo_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in incs], f"-I{py_inc}", f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
           str(CSRC / "torch_api.cpp")]
    suffix = [*[f"-L{p}" for p in libs], f"-L{LIB_DIR}",
              "-ltmo_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
              "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{p}" for p in libs]]
    _atomic_link(cmd, TORCH_EXT, suffix, verbose)
    return TORCH_EXT


def build_all(verbose: bool = False) -> None:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    build_hip_lib(verbose)
    build_torch_ext(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)

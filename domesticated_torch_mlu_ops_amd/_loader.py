"""Loads the native libraries of the package (built in-tree by ``_build.py``).

There is no fallback: if ``_lib/_tmo_torch.so`` (and the ``libtmo_hip.so`` it links) is
missing, importing the package raises ImportError.  The ops have no CPU kernels either, so a
call with CPU tensors fails in the dispatcher instead of silently computing elsewhere.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_DIR = Path(__file__).resolve().parent / "_lib"
HIP_LIB_PATH = LIB_DIR / "libtmo_hip.so"
TORCH_EXT_PATH = LIB_DIR / "_tmo_torch.so"

_loaded = False


def native_paths() -> tuple[Path, Path]:
    return HIP_LIB_PATH, TORCH_EXT_PATH


def load_native() -> None:
    """Load ``_tmo_torch.so`` into torch (registers the ``torch_mlu_ops::*`` ops)."""
    global _loaded
    if _loaded:
        return
    missing = [p for p in (HIP_LIB_PATH, TORCH_EXT_PATH) if not p.exists()]
    if missing:
        raise ImportError(
            "domesticated_torch_mlu_ops_amd: native library not built: "
            + ", ".join(str(p) for p in missing)
            + "  (run `python domesticated_torch_mlu_ops_amd/_build.py` or "
            "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root)")
    torch.ops.load_library(str(TORCH_EXT_PATH))
    _loaded = True


def c_abi() -> ctypes.CDLL:
    """The plain C ABI (include/tmo_hip.h) as a ctypes library, loaded after torch so the
    process keeps a single HIP runtime."""
    if not HIP_LIB_PATH.exists():
        raise ImportError(f"domesticated_torch_mlu_ops_amd: {HIP_LIB_PATH} not built")
    return ctypes.CDLL(str(HIP_LIB_PATH))

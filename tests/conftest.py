"""Test configuration: the ``gpu`` marker, repository imports, and in-tree builds.

GPU tests (``-m gpu``) need an MI355X; everything else runs on the CPU.  The native
libraries are built in-tree when they are missing (``__graft_entry__.build()`` rebuilds them
unconditionally; a changed source needs that call before pytest).
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

import torch  # noqa: E402  (first: the native libraries share torch's HIP runtime)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    import __graft_entry__
    recipe = __graft_entry__._builder()  # by file path: the package import needs the libraries
    if not (recipe.HIP_LIB.exists() and recipe.TORCH_EXT.exists()):
        recipe.build_all()
    import oracle
    if not oracle.LIB_PATH.exists():
        oracle.build()


_ensure_built()


@pytest.fixture(scope="session")
def tmo():
    import domesticated_torch_mlu_ops_amd as m
    return m


@pytest.fixture(scope="session")
def ref():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)

"""MI355X (gfx950) build of torch_mlu_ops' quantized paged-KV-cache path.

Drop-in for ``torch_mlu_ops.{reshape_paged_cache, quant_to_paged_cache,
dequant_from_paged_cache, moe_quantize, scaled_quantize}`` (plus the
``per_token_smooth_quantize`` alias): the same Python signatures, the same
``torch.ops.torch_mlu_ops.*`` op names, fake kernels for tracing, and the
``tmo::torch_api`` C++ prototypes, over hand-written HIP kernels behind the C ABI of
``include/tmo_hip.h``.  Importing the package loads the native libraries; there is no
CPU or pure-PyTorch fallback.
"""
import torch  # noqa: F401  (torch first: the native libraries share its HIP runtime)

from ._loader import load_native as _load_native

_load_native()

from ._ops import *  # noqa: E402,F401,F403
from ._ops import __all__ as _ops_all  # noqa: E402
from . import abstract  # noqa: E402,F401  (registers the fake kernels)

__version__ = "0.1.0"
__all__ = list(_ops_all)

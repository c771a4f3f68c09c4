"""Drop-in import name of the reference package ``rtdl_num_embeddings_cuda``.

Re-exports :mod:`piecewiselinearembeddings_optimized_amd` so that code written
against the reference (``from rtdl_num_embeddings_cuda import
CudaPiecewiseLinearEmbeddings``, ``torch.ops.rtdl_num_embeddings_cuda.*``,
``rtdl_num_embeddings_cuda._C``) runs unchanged.
"""

import sys as _sys

import piecewiselinearembeddings_optimized_amd as _impl
from piecewiselinearembeddings_optimized_amd import _C as _C  # noqa: F401
from piecewiselinearembeddings_optimized_amd import _meta as _meta  # noqa: F401
from piecewiselinearembeddings_optimized_amd import _autograd as _autograd  # noqa: F401
from piecewiselinearembeddings_optimized_amd.module import CudaPiecewiseLinearEmbeddings

_sys.modules[__name__ + "._C"] = _C
_sys.modules[__name__ + "._meta"] = _meta
_sys.modules[__name__ + "._autograd"] = _autograd
_sys.modules[__name__ + ".module"] = _impl.module

__all__ = [
    "CudaPiecewiseLinearEmbeddings",
]

__version__ = _impl.__version__

"""MI355X-native fused piecewise-linear embeddings (PLE).

Drop-in for the reference package ``rtdl_num_embeddings_cuda`` (also
importable under that name): the same ``torch.ops.rtdl_num_embeddings_cuda``
operators, FakeTensor and autograd registrations, and the
``CudaPiecewiseLinearEmbeddings`` module, running hand-written HIP kernels for
gfx950 (``csrc/ple_forward.hip``, ``csrc/ple_backward.hip``) behind the C ABI
of ``include/ple_hip.h`` (``csrc/ple_capi.hip``).

Import order follows the reference (``__init__.py:3-7`` there): the native
registrations first, then the fake kernels, then autograd, then the module.
"""

import sys as _sys

__version__ = "0.2.0.dev0"


def _running_build() -> bool:
    """True under ``python -m piecewiselinearembeddings_optimized_amd._build``:
    Python imports this package before it runs the build script, when the
    native modules may not exist yet."""
    argv = list(getattr(_sys, "orig_argv", ()))
    return "-m" in argv and argv[argv.index("-m") + 1:argv.index("-m") + 2] == [__name__ + "._build"]


if not _running_build():
    import torch  # noqa: F401  (loads the HIP runtime the extension links against)

    from . import _C as _C  # noqa: F401
    from . import _meta as _meta  # noqa: F401
    from . import _autograd as _autograd  # noqa: F401
    from .module import CudaPiecewiseLinearEmbeddings, CudaPiecewiseLinearEncoding
    from .bins import bin_tables, compute_bins

__all__ = [
    "CudaPiecewiseLinearEmbeddings",
    "CudaPiecewiseLinearEncoding",
    "bin_tables",
    "compute_bins",
]

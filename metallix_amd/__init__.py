"""metallix_amd: MI355X-native token sampler for metallix.

The product is libmx_sampler.so (HIP kernels for gfx950 behind the C ABI in
include/mx_sampler.h).  This package loads it with ctypes and offers a thin
host binding used by tests and the benchmark; device memory and streams come
from PyTorch.  There is no CPU fallback: every entry point fails loudly when
the built library or a GPU is missing.
"""
from .sampler import (  # noqa: F401
    LIB_PATH,
    MXS_BF16,
    MXS_F32,
    ROW_STATUS,
    Sampler,
    SamplerError,
    load_library,
)

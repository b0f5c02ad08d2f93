"""rac_amd — MI355X (gfx950) implementation of the RAC rotation-accumulate
hot path: CORDIC matmul, hyperbolic-CORDIC exp/softmax/SiLU, circular-CORDIC
RoPE, CORDIC-vectoring rsqrt norms.

  rac_amd/librac_amd.so   the kernels and their C ABI (include/rac.h,
                          include/rac_ext.h), built by rac_amd/csrc/Makefile
  rac_amd.ext             tensor-level ops (the rac_cuda_ext surface)
  rac_amd.rac_torch       nn.Module surface (RACLinear, RACLlamaBlock, ...)
"""
from ._lib import LIB_PATH, RACError, load, release_cached_memory

__version__ = "1.0.0"
__all__ = ["LIB_PATH", "RACError", "load", "release_cached_memory", "__version__"]

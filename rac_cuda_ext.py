"""``rac_cuda_ext``: the reference extension module's import name.

The reference's Python layer imports its compiled extension as
``rac_cuda_ext`` (rac_torch/rac_torch.py:59-151; module defined at
rac_torch/rac_torch_bind.cpp:223-258).  This module gives that name to
``rac_amd.ext``, which keeps the reference's op names, keyword arguments,
defaults and ``MODE_*`` constants and adds the row, elementwise, attention,
Q8_0 and RAC-DSP ops under new names.  Code written against the reference
extension runs unchanged: ``import rac_cuda_ext`` then e.g.
``rac_cuda_ext.linear_forward(x, w, torch.empty(0), iters=16, mode=1)``.

Every name is the object from ``rac_amd.ext`` itself, so the process-wide
knobs (``set_cordic_iters``, ``set_cordic_mode``) are shared by both names.
"""
from rac_amd import ext as _ext

__all__ = list(_ext.__all__)
globals().update({_name: getattr(_ext, _name) for _name in __all__})

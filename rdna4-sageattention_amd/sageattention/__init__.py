"""The `sageattention` package name for MI355X (gfx950): installs in place of SageAttention 2.2 and exports the same
seven entry points (reference: src/sageattention/__init__.py:6-13), all running on cdna4_sage's kernels.

    from sageattention import sageattn
"""
from .core import sageattn, sageattn_varlen
from .core import sageattn_qk_int8_pv_fp16_triton
from .core import sageattn_qk_int8_pv_fp16_cuda
from .core import sageattn_qk_int8_pv_fp8_cuda
from .core import sageattn_qk_int8_pv_fp8_cuda_sm90
from .core import sageattn_qk_int8_pv_gfx12_native

__version__ = "2.2.0+cdna4.0.1.0"

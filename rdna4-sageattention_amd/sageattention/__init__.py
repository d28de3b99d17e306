"""SageAttention 2.2 drop-in for AMD MI355X (gfx950), backed by cdna4_sage.

Same import paths and functions as SageAttention 2.2 (reference: src/sageattention/__init__.py:1-13):
    from sageattention import sageattn
"""
from .core import sageattn, sageattn_varlen
from .core import sageattn_qk_int8_pv_fp16_triton
from .core import sageattn_qk_int8_pv_fp16_cuda
from .core import sageattn_qk_int8_pv_fp8_cuda
from .core import sageattn_qk_int8_pv_fp8_cuda_sm90
from .core import sageattn_qk_int8_pv_gfx12_native

__version__ = "2.2.0+cdna4.0.1.0"

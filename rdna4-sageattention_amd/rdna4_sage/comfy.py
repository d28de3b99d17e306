"""ComfyUI backend under the reference's import and registry name (src/rdna4_sage/comfy.py:1-40):

    import rdna4_sage.comfy
    rdna4_sage.comfy.register()   # registers "rdna4_sage", backed by the gfx950 kernels
"""
from cdna4_sage.comfy import attention_cdna4_sage as attention_rdna4_sage
from cdna4_sage.comfy import register as _register


def register(name="rdna4_sage"):
    return _register(name)

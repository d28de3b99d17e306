"""ctypes binding of libsage_capi.so (the C ABI declared in include/sage_capi.h).

Replaces the reference's driver-API FFI (src/rdna4_sage/_hip.py:1-73): instead of packing kernarg blocks into a
shared ctypes buffer per kernel and calling hipModuleLaunchKernel, each launch is a typed C call with arguments
passed by value, so concurrent callers cannot clobber each other's arguments.  torch is imported before the library
is opened, so the library binds to the HIP runtime instance torch already loaded (same soname) and shares its device
context and streams, which is the reason the reference looks the runtime up in /proc/self/maps (_hip.py:11-28).
"""
from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "libsage_capi.so"

SAGE_OK, SAGE_ERR_INVALID, SAGE_ERR_UNSUPPORTED, SAGE_ERR_HIP = 0, 1, 2, 3
DTYPE_BF16, DTYPE_F16, DTYPE_BOOL = 0, 1, 2
ABI_VERSION = 6

_lib = None
_lock = threading.Lock()

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

SIGNATURES = {
    "sage_abi_version": ([], _I),
    "sage_last_error": ([], ctypes.c_char_p),
    "sage_kv_pad": ([_I], _I),
    "sage_layout_dim": ([_I], _I),
    "sage_manifest_json": ([], ctypes.c_char_p),
    "sage_quant_q": ([_P, _L, _L, _L, _I, _I, _I, _I, _I, _F, _P, _P, _P], _I),
    "sage_v_amax": ([_P, _L, _L, _L, _I, _I, _I, _I, _I, _P, _P], _I),
    "sage_quant_kv": ([_P, _L, _L, _L, _P, _L, _L, _L, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P], _I),
    "sage_attn_plan": ([_I, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "sage_attn_fwd": ([_P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _L, _P], _I),
    "sage_forward_workspace": ([_I, _I, _I, _I, _I, _I, _I, _P], _I),
    "sage_lse_fwd": ([_P, _L, _L, _L, _P, _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P], _I),
    "sage_forward": ([_P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L,
                      _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _L, _P], _I),
    "sage_varlen_layout": ([_I, _I, _I, _I, _I, _P, _P], _I),
    "sage_forward_varlen": ([_P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _P,
                             _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _L, _P], _I),
    "sage_mask_workspace": ([_I, _I, _I, _I, _I, _I, _I, _I, _L, _L, _L, _P], _I),
    "sage_forward_masked": ([_P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L,
                             _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _I, _L, _L, _L,
                             _P, _P, _P, _P, _P, _P, _P, _L, _P], _I),
    "sage_forward_noalloc": ([_P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L, _P, _L, _L, _L,
                              _I, _I, _I, _I, _I, _I, _I, _I, _F, _P], _I),
}


class SageError(RuntimeError):
    """A libsage_capi call returned an error code."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"cdna4_sage: {fn} failed (code {code}): {message}")
        self.code = code


def lib():
    """Open libsage_capi.so once (thread-safe).  Raises RuntimeError when the library has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(f"cdna4_sage: {LIB_PATH} is missing; build it with "
                                       "`python rdna4-sageattention_amd/build_kernels.py` (hipcc --offload-arch=gfx950)")
                h = ctypes.CDLL(str(LIB_PATH))
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(h, name)
                    fn.argtypes = args
                    fn.restype = res
                if h.sage_abi_version() != ABI_VERSION:
                    raise RuntimeError(f"cdna4_sage: library ABI {h.sage_abi_version()} != expected {ABI_VERSION}")
                _lib = h
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != SAGE_OK:
        raise SageError(name, rc, lib().sage_last_error().decode(errors="replace"))


def kv_pad(skv: int) -> int:
    return int(lib().sage_kv_pad(int(skv)))


def layout_dim(head_dim: int) -> int:
    """Channels of the Q8 / K8 / V8T / VS layouts for this head_dim (128 for 96, else head_dim)."""
    return int(lib().sage_layout_dim(int(head_dim)))


@functools.lru_cache(maxsize=4096)
def attn_plan(device_index: int, B: int, H: int, Sq: int, Skv: int, D: int, causal: bool):
    """(n_full, chunks, workspace_bytes) of sage_attn_fwd for this shape on device `device_index`."""
    n_full, chunks, ws = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    with torch.cuda.device(device_index):
        call("sage_attn_plan", B, H, Sq, Skv, D, int(causal), ctypes.byref(n_full), ctypes.byref(chunks),
             ctypes.byref(ws))
    return n_full.value, chunks.value, ws.value


@functools.lru_cache(maxsize=4096)
def forward_workspace(device_index: int, B: int, H: int, Hkv: int, Sq: int, Skv: int, D: int, causal: bool) -> int:
    """Workspace bytes of sage_forward for this shape on device `device_index`."""
    ws = ctypes.c_int64()
    with torch.cuda.device(device_index):
        call("sage_forward_workspace", B, H, Hkv, Sq, Skv, D, int(causal), ctypes.byref(ws))
    return ws.value


@functools.lru_cache(maxsize=4096)
def mask_workspace(device_index: int, B: int, H: int, Hkv: int, Sq: int, Skv: int, D: int, causal: bool,
                   mask_dtype: int, msb: int, msh: int, msq: int) -> int:
    """Workspace bytes of sage_forward_masked for this shape, mask dtype and mask strides on `device_index`."""
    ws = ctypes.c_int64()
    with torch.cuda.device(device_index):
        call("sage_mask_workspace", B, H, Hkv, Sq, Skv, D, int(causal), mask_dtype, msb, msh, msq, ctypes.byref(ws))
    return ws.value


@functools.lru_cache(maxsize=4096)
def varlen_layout(batch: int, H: int, Hkv: int, total_q: int, total_k: int):
    """(kv_rows, workspace_bytes) of sage_forward_varlen: padded packed key rows per kv head and the bytes of its
    table workspace (host arithmetic only)."""
    rows, ws = ctypes.c_int(), ctypes.c_int64()
    call("sage_varlen_layout", batch, H, Hkv, total_q, total_k, ctypes.byref(rows), ctypes.byref(ws))
    return rows.value, ws.value

"""Ahead-of-time build of the gfx950 kernels: hipcc -> cdna4_sage/libsage_capi.so (+ cdna4_sage/manifest.json).

Replaces the reference's offline kernel build (kernel_build/build_kernels.py:117-142, which ran FlyDSL and Triton
and wrote one code object per variant plus kernels/manifest.json).  Here every variant (layouts of 64 / 128 / 256
channels for head dims 64, 96, 128, 256 x bf16/f16 x causal/non-causal x dense/varlen) is compiled by hipcc into one
shared library; the manifest is the library's own description
(``sage_manifest_json``), written next to it so the Python side can read the supported shapes without loading it.

usage: python rdna4-sageattention_amd/build_kernels.py
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent       # rdna4-sageattention_amd/
PKG = ROOT / "cdna4_sage"

CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB = PKG / "libsage_capi.so"
MANIFEST = PKG / "manifest.json"
ARCH = "gfx950"
SOURCES = ("sage_capi.hip", "sage_quant.hip", "sage_attn.hip", "sage_lse.hip", "sage_varlen.hip", "sage_mask.hip")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",               # the kernels' fused multiply-adds are all explicit
    "-fno-gpu-flush-denormals-to-zero",
    "-mcode-object-version=5",
    # no packed-fp32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libsage_capi.so)")


def build(verbose: bool = False) -> Path:
    """Compile every kernel variant for gfx950 into libsage_capi.so and refresh manifest.json."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is harmless
    noise = [ln for ln in (res.stderr or "").splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    os.replace(tmp, LIB)
    # the manifest comes from the library itself, queried in a child process (no GPU or torch needed)
    probe = ("import ctypes,sys; l=ctypes.CDLL(sys.argv[1]); l.sage_manifest_json.restype=ctypes.c_char_p; "
             "print(l.sage_manifest_json().decode())")
    out = subprocess.run([sys.executable, "-c", probe, str(LIB)], capture_output=True, text=True, check=True).stdout
    manifest = json.loads(out)
    manifest["library"] = LIB.name
    manifest["build_flags"] = HIP_FLAGS
    MANIFEST.write_text(json.dumps(manifest, indent=1) + "\n")
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))

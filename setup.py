"""Wheel of the MI355X (gfx950) SageAttention path.

Same distribution name as SageAttention (reference: pyproject.toml:8-22), so the wheel substitutes a SageAttention
install.  It ships three packages from rdna4-sageattention_amd/: `sageattention` (SageAttention 2.2 API),
`cdna4_sage` (the gfx950 kernels: libsage_capi.so built by hipcc, its manifest, the ComfyUI backend) and `rdna4_sage`
(the reference's import name).  build_py compiles the library first (rdna4-sageattention_amd/build_kernels.py);
CDNA4_SAGE_PREBUILT=1 packages the library already in the tree instead.  The library is loaded through ctypes, so the
wheel is tagged for the platform and not for a Python ABI.

    pip wheel --no-deps --no-build-isolation .
"""
import importlib.util
import os
from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.command.install import install
from setuptools.dist import Distribution

try:
    from wheel.bdist_wheel import bdist_wheel
except ImportError:  # wheel missing: sdists and in-place installs still work
    bdist_wheel = None

ROOT = Path(__file__).resolve().parent
PKG_ROOT = "rdna4-sageattention_amd"


class BuildPyWithKernels(build_py):
    def run(self):
        lib = ROOT / PKG_ROOT / "cdna4_sage" / "libsage_capi.so"
        if os.environ.get("CDNA4_SAGE_PREBUILT") == "1":
            if not lib.exists():
                raise RuntimeError(f"CDNA4_SAGE_PREBUILT=1 but {lib} has not been built")
        else:
            spec = importlib.util.spec_from_file_location("sage_build_kernels", ROOT / PKG_ROOT / "build_kernels.py")
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            mod.build(verbose=True)
        super().run()


class BinaryDistribution(Distribution):
    """The packages carry a native library: platform-specific build and install directories."""

    def has_ext_modules(self):
        return True


class InstallPlatlib(install):
    """Install the packages as platform-specific (the wheel root, not .data/purelib): they carry libsage_capi.so."""

    def finalize_options(self):
        super().finalize_options()
        self.install_lib = self.install_platlib


cmdclass = {"build_py": BuildPyWithKernels, "install": InstallPlatlib}
if bdist_wheel is not None:
    class PlatformWheel(bdist_wheel):
        def get_tag(self):
            return "py3", "none", super().get_tag()[2]

    cmdclass["bdist_wheel"] = PlatformWheel

setup(
    name="sageattention",
    version="2.2.0+cdna4.0.1.0",
    description="SageAttention 2.2 drop-in for AMD MI355X (gfx950, CDNA4): hand-written HIP int8/fp8 attention kernels",
    keywords=["attention", "sageattention", "cdna4", "gfx950", "mi355x", "rocm", "comfyui"],
    license="Apache-2.0",
    python_requires=">=3.10",
    # torch must be a ROCm build: the library binds to the HIP runtime torch loads
    install_requires=["torch>=2.10"],
    package_dir={"": PKG_ROOT},
    packages=["sageattention", "cdna4_sage", "rdna4_sage"],
    package_data={"cdna4_sage": ["libsage_capi.so", "manifest.json"]},
    cmdclass=cmdclass,
    distclass=BinaryDistribution,
)

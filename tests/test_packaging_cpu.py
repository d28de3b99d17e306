"""The wheel (setup.py; reference: pyproject.toml:8-22): distribution `sageattention`, the three packages, the
gfx950 library built in the tree and its manifest, a platform tag; the unpacked wheel imports and loads its own
library."""
import glob
import os
import shutil
import subprocess
import sys
import zipfile
from pathlib import Path

import pytest

from cdna4_sage import _capi

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "rdna4-sageattention_amd" / "cdna4_sage" / "libsage_capi.so"


@pytest.fixture(scope="module")
def wheel(tmp_path_factory):
    if not LIB.exists():
        pytest.skip("libsage_capi.so not built")
    tmp = tmp_path_factory.mktemp("wheel")
    src = tmp / "src"
    src.mkdir()
    for f in ("setup.py", "pyproject.toml"):
        shutil.copy(ROOT / f, src / f)
    shutil.copytree(ROOT / "rdna4-sageattention_amd", src / "rdna4-sageattention_amd",
                    ignore=shutil.ignore_patterns("__pycache__", "csrc"))
    env = dict(os.environ, CDNA4_SAGE_PREBUILT="1")
    subprocess.run([sys.executable, "-m", "pip", "wheel", "--no-deps", "--no-build-isolation", "--no-index", "-q",
                    "-w", str(tmp / "dist"), str(src)], check=True, env=env, cwd=tmp, timeout=600)
    (whl,) = glob.glob(str(tmp / "dist" / "*.whl"))
    return Path(whl)


def test_wheel_contents(wheel):
    assert wheel.name.startswith("sageattention-2.2.0+cdna4") and wheel.name.endswith("-py3-none-linux_x86_64.whl")
    names = set(zipfile.ZipFile(wheel).namelist())
    for n in ("sageattention/__init__.py", "sageattention/core.py", "cdna4_sage/__init__.py", "cdna4_sage/_capi.py",
              "cdna4_sage/libsage_capi.so", "cdna4_sage/manifest.json", "cdna4_sage/comfy.py",
              "rdna4_sage/__init__.py", "rdna4_sage/ops.py", "rdna4_sage/comfy.py"):
        assert n in names, n
    assert not any(n.startswith(("oracle/", "tests/")) or "/csrc/" in n for n in names)
    meta = zipfile.ZipFile(wheel).read(next(n for n in names if n.endswith("METADATA"))).decode()
    assert "Name: sageattention" in meta and "Requires-Dist: torch" in meta


def test_unpacked_wheel_imports_its_own_library(wheel, tmp_path):
    zipfile.ZipFile(wheel).extractall(tmp_path)
    code = ("import sageattention, cdna4_sage, rdna4_sage; from cdna4_sage import _capi; "
            "print(_capi.lib().sage_abi_version(), cdna4_sage.HEAD_DIMS, _capi.LIB_PATH)")
    env = dict(os.environ, PYTHONPATH=str(tmp_path))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, cwd=tmp_path,
                         timeout=300, check=True).stdout.strip()
    abi, *rest = out.split(" ", 1)
    assert int(abi) == _capi.ABI_VERSION and "(64, 96, 128, 256)" in rest[0]
    assert str(tmp_path) in rest[0]

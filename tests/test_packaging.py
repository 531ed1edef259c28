"""CPU tests of the packaging: the distribution keeps the reference's name and `gpu` marker
(pyproject.toml:6,22), drops Triton, and its wheel carries the HIP library the loader opens."""

import configparser
import os
import shutil
import subprocess
import sys
import zipfile

import pytest
import tomli

from sol_attn_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _setup_cfg():
    cfg = configparser.ConfigParser()
    cfg.read(os.path.join(ROOT, "setup.cfg"))
    return cfg


def test_distribution_metadata():
    cfg = _setup_cfg()
    assert cfg["metadata"]["name"] == "sol-attn-amd"
    requires = cfg["options"]["install_requires"].split()
    assert any(r.startswith("torch") for r in requires)
    assert not any("triton" in r for r in requires)
    assert cfg["options"]["packages"].strip() == "sol_attn_amd"
    # The library shipped as package data is the one the loader opens.
    assert cfg["options.package_data"]["sol_attn_amd"].strip() == os.path.basename(_native.LIB_PATH)
    with open(os.path.join(ROOT, "pyproject.toml"), "rb") as f:
        pyproject = tomli.load(f)
    markers = pyproject["tool"]["pytest"]["ini_options"]["markers"]
    assert any(m.startswith("gpu:") for m in markers)


def test_wheel_carries_the_library_and_loads_it(tmp_path):
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so is not built")
    src = tmp_path / "src"
    src.mkdir()
    for name in ("pyproject.toml", "setup.cfg", "setup.py", "README.md"):
        shutil.copy(os.path.join(ROOT, name), src / name)
    shutil.copytree(os.path.join(ROOT, "solattn-amd_amd", "sol_attn_amd"),
                    src / "solattn-amd_amd" / "sol_attn_amd",
                    ignore=shutil.ignore_patterns("__pycache__", "_build"))
    env = dict(os.environ, SOL_ATTN_AMD_PREBUILT="1")
    res = subprocess.run([sys.executable, "-m", "pip", "wheel", "--no-deps", "--no-build-isolation",
                          "-w", str(tmp_path / "dist"), str(src)],
                         capture_output=True, text=True, timeout=300, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    wheels = list((tmp_path / "dist").glob("*.whl"))
    assert len(wheels) == 1
    assert wheels[0].name.startswith("sol_attn_amd-0.1.0-py3-none-linux_")
    with zipfile.ZipFile(wheels[0]) as z:
        names = set(z.namelist())
        assert "sol_attn_amd/libsol_attn_amd.so" in names
        assert {"sol_attn_amd/__init__.py", "sol_attn_amd/_native.py", "sol_attn_amd/attention.py",
                "sol_attn_amd/indexed.py"} <= names
        z.extractall(tmp_path / "site")
    # Imported from the unpacked wheel, the package opens its own copy of the library.
    probe = ("import os, sol_attn_amd; from sol_attn_amd import _native; "
             "assert _native.LIB_PATH.startswith(os.environ['SITE']); "
             "lib = _native.library(); print(lib.sol_abi_version())")
    res = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True, timeout=300,
                         cwd=str(tmp_path), env=dict(os.environ, SITE=str(tmp_path / "site"),
                                                     PYTHONPATH=str(tmp_path / "site")))
    assert res.returncode == 0, res.stdout + res.stderr
    assert int(res.stdout.split()[-1]) == _native.ABI_VERSION

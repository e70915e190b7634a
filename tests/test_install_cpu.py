"""The two installable distributions (CPU only).

fable_attn (flash-attention-rdna2_amd/setup.cfg: the package with the built C-ABI library) and
the name-only flash_attn distribution (flash-attention-rdna2_amd/compat/setup.cfg) install
offline with pip into a temporary target. A fresh interpreter that sees only that target then
finds the distributions' metadata (importlib.metadata, which transformers queries to decide
whether flash-attention is available: the reason the reference ships the second distribution,
README.md:133-142, compat/pyproject.toml:6-10), and `import flash_attn` / `flash_attn_interface`
resolve to the installed fable_attn.
"""
import json
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-attention-rdna2_amd")
LIB = os.path.join(PKG, "fable_attn", "libfable_attn_hip.so")

_PROBE = r"""
import importlib.metadata as md, json, sys
import fable_attn, flash_attn, flash_attn_interface
from flash_attn import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from flash_attn.flash_attn_interface import flash_attn_combine
from flash_attn_interface import get_scheduler_metadata
res = {"v_flash_attn": md.version("flash_attn"), "v_fable_attn": md.version("fable_attn"),
       "api_version": fable_attn.FLASH_ATTN_API_VERSION, "mod_version": flash_attn.__version__,
       "files": [fable_attn.__file__, flash_attn.__file__, flash_attn_interface.__file__],
       "same_func": flash_attn_func is fable_attn.flash_attn_func,
       "requires": md.requires("flash_attn")}
try:
    from transformers.utils.import_utils import _is_package_available
    res["transformers"] = list(_is_package_available("flash_attn", return_version=True))
except ImportError:
    res["transformers"] = None
print(json.dumps(res))
"""


def _copy_src(dst):
    """The two distribution trees without build leftovers (pip builds in the source tree)."""
    ign = shutil.ignore_patterns("__pycache__", "_build", "build", "*.egg-info", "*.tmp")
    fab = os.path.join(dst, "fable_src")
    os.makedirs(fab)
    for name in ("fable_attn", "setup.py", "setup.cfg", "pyproject.toml", "build.py"):
        src = os.path.join(PKG, name)
        (shutil.copytree if os.path.isdir(src) else shutil.copy2)(src, os.path.join(fab, name),
                                                                   **({"ignore": ign} if os.path.isdir(src) else {}))
    comp = os.path.join(dst, "compat_src")
    shutil.copytree(os.path.join(PKG, "compat"), comp, ignore=ign)
    return fab, comp


@pytest.mark.skipif(not os.path.exists(LIB), reason="the C-ABI library is not built")
def test_offline_install_exposes_metadata(tmp_path):
    fab, comp = _copy_src(str(tmp_path))
    site = str(tmp_path / "site")
    r = subprocess.run([sys.executable, "-m", "pip", "install", "--no-build-isolation", "--no-deps",
                        "--no-index", "--disable-pip-version-check", "--target", site, fab, comp],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert os.path.exists(os.path.join(site, "fable_attn", "libfable_attn_hip.so"))
    env = dict(os.environ, PYTHONPATH=site)
    p = subprocess.run([sys.executable, "-c", _PROBE], capture_output=True, text=True, env=env,
                       cwd=str(tmp_path), timeout=300)
    assert p.returncode == 0, p.stdout + p.stderr
    res = json.loads(p.stdout.strip().splitlines()[-1])
    assert res["v_flash_attn"] == res["api_version"] == res["mod_version"]
    assert res["v_flash_attn"].startswith("2.8.3+fable.")
    assert res["v_fable_attn"] == res["api_version"].rsplit(".mi355x.", 1)[1]
    for f in res["files"]:
        assert os.path.realpath(f).startswith(os.path.realpath(site)), f
    assert res["same_func"]
    assert [r.replace("-", "_") for r in res["requires"]] == ["fable_attn"]
    if res["transformers"] is not None:
        assert res["transformers"] == [True, res["api_version"]]


def test_compat_version_matches_the_package():
    """compat/setup.cfg states the flash_attn version statically; it must be the version the
    package announces (fable_attn.FLASH_ATTN_API_VERSION), built from fable_attn.__version__."""
    import configparser
    import re
    cfg = configparser.ConfigParser()
    cfg.read(os.path.join(PKG, "compat", "setup.cfg"))
    init = open(os.path.join(PKG, "fable_attn", "__init__.py")).read()
    own = re.search(r'^__version__ = "([^"]+)"', init, re.M).group(1)
    prefix = re.search(r'^FLASH_ATTN_API_VERSION = "([^"]+)" \+ __version__', init, re.M).group(1)
    assert cfg["metadata"]["version"] == prefix + own

"""Package smoke tests that need no GPU (the reference's tests/test_import.py): every Python file of the package,
the oracle, the tests and the entry points byte-compiles; the package imports; every module of the package is
named in the package's module map; every module imports on a machine without a GPU."""
import glob
import importlib
import os
import py_compile
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mace-million_amd", "mace_onegpu")
PY_FILES = sorted(glob.glob(os.path.join(ROOT, "mace-million_amd", "**", "*.py"), recursive=True)
                  + glob.glob(os.path.join(ROOT, "oracle", "**", "*.py"), recursive=True)
                  + glob.glob(os.path.join(ROOT, "tests", "**", "*.py"), recursive=True)
                  + [os.path.join(ROOT, f) for f in ("bench.py", "__graft_entry__.py")])
MODULES = sorted(os.path.basename(p)[:-3] for p in glob.glob(os.path.join(PKG, "*.py"))
                 if not os.path.basename(p).startswith("__"))


@pytest.mark.parametrize("path", PY_FILES, ids=lambda p: os.path.relpath(p, ROOT))
def test_py_compile(path, tmp_path):
    py_compile.compile(path, doraise=True, cfile=str(tmp_path / "out.pyc"))


def test_package_imports():
    import mace_onegpu

    assert mace_onegpu.__version__


def test_every_module_is_listed():
    """The module map of the package docstring names every module (and no module that does not exist)."""
    import mace_onegpu

    listed = set()
    for line in mace_onegpu.__doc__.splitlines():
        m = re.match(r"\s{2}(\w+(?:,\s*\w+)*)\s{2,}", line)
        if m:
            listed.update(n.strip() for n in m.group(1).split(","))
    assert listed == set(MODULES), (sorted(set(MODULES) - listed), sorted(listed - set(MODULES)))


@pytest.mark.parametrize("name", MODULES)
def test_module_imports(name):
    importlib.import_module(f"mace_onegpu.{name}")

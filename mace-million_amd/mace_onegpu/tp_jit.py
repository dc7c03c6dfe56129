"""Explicit-weight channelwise TP kernels for path tables that the library does not carry, built on first use.

The reference's FusedConvTP evaluates any channelwise path table: cuEquivariance builds its SegmentedPolynomial from
the irreps at run time (fused_edge_conv.py:43-68), as conv_spline generates its Triton kernels for a table
(conv_spline.py:38-181).  The library here carries the tables of o3.COMPILED_TP_TABLES.  For any other table
(spherical harmonics up to l = 3) this module generates the same straight-line kernels (codegen.tpw_source) and
builds them with the library's own compiler flags into a small shared library next to it, lib/jit/tpw_j<key>.so
(key: a hash of the table; MM_TP_JIT_DIR names another directory), the first time the table is used; later calls
and processes load the built file.  A file built from other sources (another generator, common.h or api.cpp) is
rebuilt.  Building takes about 5 s and needs hipcc; build.py builds the tables of o3.PREBUILT_JIT_TP_TABLES ahead.
"""
import ctypes
import hashlib
import importlib.util
import os
import shutil
import subprocess
import tempfile
import threading

from . import codegen
from ._lib import I, L, P, _Fn

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))     # mace-million_amd/
CSRC = os.path.join(PKG, "csrc")
# where the run-time libraries live: next to the library, or MM_TP_JIT_DIR (e.g. for a read-only install)
JIT_DIR = os.environ.get("MM_TP_JIT_DIR") or os.path.join(PKG, "lib", "jit")

# argument types of mm_tpw_<name>_fwd / _bwd (include/mace_million_amd.h)
SIG_FWD = [P, I, P, P, P, L, P, L, P, L, P, L, P]
SIG_BWD = [P, I, P, P, P, L, P, L, P, L, P, L, P, L, P, L, P, L, P]

_loaded = {}
_lock = threading.Lock()


def table_key(table):
    """12 hex digits identifying a path table (sizes, paths and every term with its coefficient)."""
    rep = repr((table["nX"], table["nW"], table["nO"], table["nY"], table["paths"], table["terms"]))
    return hashlib.sha256(rep.encode()).hexdigest()[:12]


def _build_module():
    spec = importlib.util.spec_from_file_location("_mm_build", os.path.join(PKG, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _source(table, name, flags):
    """The generated source, stamped with the hashes of what else goes into the build."""
    stamp = hashlib.sha256()
    for f in ("common.h", "api.cpp"):
        with open(os.path.join(CSRC, f), "rb") as fh:
            stamp.update(fh.read())
    stamp.update(" ".join(flags).encode())
    return f"// built with common.h / api.cpp / flags {stamp.hexdigest()[:16]}\n" + codegen.tpw_source(table, name)


def paths(table):
    """(kernel name, source path, library path) of a table's JIT build."""
    name = "j" + table_key(table)
    return name, os.path.join(JIT_DIR, f"tpw_{name}.hip"), os.path.join(JIT_DIR, f"tpw_{name}.so")


def _is_current(hip, so, src):
    if not (os.path.exists(so) and os.path.exists(hip)):
        return False
    with open(hip) as fh:
        return fh.read() == src


def is_current(table):
    """True when the table's library exists and was built from the sources and flags of this tree."""
    mod = _build_module()
    name, hip, so = paths(table)
    return _is_current(hip, so, _source(table, name, list(mod.FLAGS)))


def build(table, force=False):
    """Builds the table's library unless an up-to-date one exists (or always, with force); returns its path."""
    mod = _build_module()
    flags = list(mod.FLAGS)
    name, hip, so = paths(table)
    src = _source(table, name, flags)
    if not force and _is_current(hip, so, src):
        return so
    if not os.path.exists(mod.HIPCC):
        raise RuntimeError(f"the channelwise TP table {name} has no kernels built yet and building them needs hipcc "
                           f"({mod.HIPCC} is missing; set HIPCC)")
    os.makedirs(JIT_DIR, exist_ok=True)
    tmp = tempfile.mkdtemp(prefix=f".{name}.", dir=JIT_DIR)
    try:
        t_hip, t_so = os.path.join(tmp, os.path.basename(hip)), os.path.join(tmp, os.path.basename(so))
        with open(t_hip, "w") as fh:
            fh.write(src)
        # the generated source includes "../common.h" (its place in csrc/gen/): found through -I csrc/gen
        cmd = [mod.HIPCC] + flags + ["-shared", "-I", os.path.join(CSRC, "gen"), t_hip,
                                     os.path.join(CSRC, "api.cpp"), "-o", t_so]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"building the channelwise TP kernels of table {name} failed: {' '.join(cmd)}\n"
                               f"{r.stdout}\n{r.stderr}")
        os.replace(t_so, so)          # the library first: a matching source then always names a built library
        os.replace(t_hip, hip)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return so


def kernels(table):
    """(forward, backward) entry points of the table's kernels, with the arguments of mm_tpw_l1_fwd / _bwd; built
    first when needed."""
    key = table_key(table)
    with _lock:
        if key not in _loaded:
            name, _, _ = paths(table)
            so = ctypes.CDLL(build(table))
            so.mm_last_error.restype = ctypes.c_char_p
            so.mm_last_error.argtypes = []

            def err(so=so):
                return so.mm_last_error().decode()

            fns = []
            for kind, sig in (("fwd", SIG_FWD), ("bwd", SIG_BWD)):
                f = getattr(so, f"mm_tpw_{name}_{kind}")
                f.argtypes, f.restype = sig, ctypes.c_int
                fns.append(_Fn(f"mm_tpw_{name}_{kind}", f, err))
            _loaded[key] = (so, fns[0], fns[1])
    return _loaded[key][1], _loaded[key][2]

"""ctypes wrapper of the plain-C neighbour-build restatement (nlist.c) -- TEST INFRASTRUCTURE ONLY.

build() compiles liboracle_nlist.so next to the source with gcc (-O2 -ffp-contract=off -fopenmp); it is called by
__graft_entry__.build() and, when the library is missing, by load().
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "nlist.c")
LIB = os.path.join(HERE, "liboracle_nlist.so")
_lib = None


def build():
    cmd = ["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared", SRC,
           "-o", LIB + ".tmp", "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
            build()
        _lib = ctypes.CDLL(LIB)
        P, L, D = ctypes.c_void_p, ctypes.c_long, ctypes.c_double
        _lib.onl_sort.argtypes = [L, P, P, D, P, P, P, P]
        _lib.onl_neighbors.argtypes = [L, P, P, P, P, D, P, P, P, P, P]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def neighbor_list(pos, box, r_max):
    """(perm int64 [N], pos_sorted [N,3], NN int32 [N], rowptr int64 [N+1], send int32 [E]) in the reference's
    order (receiver_chunk_mace.py:82-165)."""
    lib = load()
    pos = np.ascontiguousarray(pos, dtype=np.float64)
    box = np.ascontiguousarray(box, dtype=np.float64).reshape(3)
    N = len(pos)
    ncell = np.zeros(3, dtype=np.int64)
    perm = np.zeros(N, dtype=np.int64)
    ps = np.zeros((N, 3), dtype=np.float64)
    cell = np.zeros((N, 3), dtype=np.int64)
    if lib.onl_sort(N, _p(pos), _p(box), float(r_max), _p(ncell), _p(perm), _p(ps), _p(cell)) != 0:
        raise MemoryError("onl_sort")
    nc = int(np.prod(ncell))
    cs, cc = np.zeros(nc, np.int64), np.zeros(nc, np.int64)
    NN = np.zeros(N, dtype=np.int32)
    rowptr = np.zeros(N + 1, dtype=np.int64)
    lib.onl_neighbors(N, _p(ps), _p(cell), _p(box), _p(ncell), float(r_max), _p(cs), _p(cc), _p(NN), None, None)
    rowptr[1:] = np.cumsum(NN)
    send = np.zeros(max(int(rowptr[-1]), 1), dtype=np.int32)
    lib.onl_neighbors(N, _p(ps), _p(cell), _p(box), _p(ncell), float(r_max), _p(cs), _p(cc), _p(NN), _p(rowptr),
                      _p(send))
    return perm, ps, NN, rowptr, send[: int(rowptr[-1])]

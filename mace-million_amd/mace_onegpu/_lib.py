"""ctypes binding of the C-ABI library libmace_million_amd.so (declared in include/mace_million_amd.h).

The library is built in-tree by mace-million_amd/build.py.  There is no fallback: importing a compute entry point
without the library raises, so a GPU run can never silently take another path.  Every call checks the returned
status and raises RuntimeError with mm_last_error() on failure.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(HERE), "lib", "libmace_million_amd.so")
ABI_VERSION = 7     # mm_version() of the library this binding's buffer layouts are written for

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_long
F = ctypes.c_float
D = ctypes.c_double
SZ = ctypes.c_size_t

# name -> argument types (the last argument of every compute entry point is the hipStream_t)
SIGNATURES = {
    "mm_version": [],
    "mm_build_info": [P, P, P],
    "mm_last_error": [],
    # neighbour list
    "mm_nl_workspace_bytes": [L, P],
    "mm_nl_prepare": [P, L, P, P, P, P, P, P, P, P],
    "mm_nl_sort": [P, P, P, P, L, P, SZ, P],
    "mm_nl_gather": [P, L, P, P, P, P, P, P, P],
    "mm_nl_cell_ranges": [P, L, P, P, P, P],
    "mm_nl_count": [P, P, L, P, P, P, P, D, I, P, P],
    "mm_nl_scan": [P, P, L, P, SZ, P],
    "mm_nl_scan_noalloc": [P, P, L, P],
    "mm_nl_fill": [P, P, L, P, P, P, P, D, I, P, P, P],
    "mm_nl_filter_count": [P, L, P, P, P, D, P, P, P],
    "mm_nl_filter_fill": [P, L, P, P, P, D, P, P, P, I, P],
    "mm_nl_reverse": [P, P, L, L, P, P],
    # geometry
    "mm_edge_geom_rij": [I, P, P, P, I, P, P, I, P, P, I, F, I, I, F, F, I, P, P, P, P, P, P],
    "mm_edge_geom_pos": [I, P, P, P, P, I, P, P, P, I, P, P, I, F, I, I, F, F, I, P, P, P, P, P, P],
    # layer-1 ACE kernels
    "mm_ace1_fwd": [P, I, P, P, P, I, I, P, P, P],
    "mm_ace1_bwd": [P, I, P, P, P, I, I, P, F, P, P],
    "mm_spline_coeffs_flat": [P, I, I, D, D, I, P, P],
    "mm_edge_grad": [I, P, P, L, I, P, P, P, P, P, I, P],
    # convolutions (generated)
    "mm_conv1_fwd": [P, I, P, P, P, I, P, I, I, P, P, P],
    "mm_conv2_fwd": [P, I, P, P, P, I, P, I, I, P, P, P],
    "mm_conv1_bwd": [P, I, P, P, P, I, P, I, I, F, P, P, L, P, P],
    "mm_conv2_bwd": [P, I, P, P, P, I, P, I, I, F, P, P, L, P, P],
    "mm_conv2_bwd_det": [P, I, P, P, P, I, P, I, I, F, P, P, L, P, P],
    "mm_conv0123_fwd": [P, I, P, P, P, I, P, I, I, P, P, P],
    "mm_conv0123_bwd": [P, I, P, P, P, I, P, I, I, F, P, P, L, P, P],
    "mm_gather_rows_csr": [P, P, P, L, I, P, L, I, P],
    # explicit-weight channelwise TP (generated; FusedConvTP)
    **{f"mm_tpw_{n}_fwd": [P, I, P, P, P, L, P, L, P, L, P, L, P] for n in ("l1", "l2", "l0123")},
    **{f"mm_tpw_{n}_bwd": [P, I, P, P, P, L, P, L, P, L, P, L, P, L, P, L, P, L, P] for n in ("l1", "l2", "l0123")},
    # symmetric contraction (generated)
    "mm_symc1_fwd": [I, P, L, P, P, P, L, P],
    "mm_symc2_fwd": [I, P, L, P, P, P, L, P],
    "mm_symc1_bwd": [I, P, L, P, P, P, L, P, L, P, P, P],
    "mm_symc2_bwd": [I, P, L, P, P, P, L, P, L, P, P, P],
    # node level
    "mm_linear": [P, L, P, P, L, P, P, P, I, P, P, L, I, I, I, I, I, P, P, P, P, I, P],
    "mm_fill_f32": [P, L, F, P],
    "mm_fill_f64": [P, L, D, P],
    "mm_fill_i32": [P, L, I, P],
    "mm_species_lists": [P, I, I, P, L, P, P],
    "mm_readout1": [I, P, L, P, F, P, P, L, P, L, I, P],
    "mm_readout2": [I, P, L, P, P, I, F, F, P, P, L, P],
    "mm_ghost_forward": [P, P, I, I, I, P, P],
    "mm_ghost_reverse": [P, P, I, I, P, P, P],
    "mm_pair_forces_to_atoms": [I, P, P, P, P, P, P],
    "mm_pair_forces_skin": [L, P, P, P, P, P, P],
    "mm_chunk_forces": [I, I, P, P, P, P, P, P, P],
    "mm_chunk_edge_index": [L, P, P, P, I, P, P, P],
    # tables
    "mm_radial_mlp_f64": [I, P, P, P, P, P, I, I, I, D, I, D, P, P],
    "mm_spline_coeffs": [P, I, I, D, D, I, I, P, P],
}

_lib = None


class _Fn:
    """A C-ABI entry point: device tensors passed as pointers, a nonzero status raised with the message of the
    library's mm_last_error() (err; the main library's by default)."""

    def __init__(self, name, fn, err=None):
        self.name, self.fn, self.err = name, fn, err

    def __call__(self, *args):
        conv = []
        for k, a in enumerate(args):
            if isinstance(a, torch.Tensor):
                # tensors are device buffers; the HOST arrays of the ABI are passed as ctypes objects
                if a.device.type != "cuda":
                    raise TypeError(f"{self.name}: argument {k} is a {a.device.type} tensor; the kernels take "
                                    "device memory")
                conv.append(ctypes.c_void_p(a.data_ptr()))
            elif a is None:
                conv.append(ctypes.c_void_p(0))
            else:
                conv.append(a)
        rc = self.fn(*conv)
        if rc != 0:
            raise RuntimeError(f"{self.name} failed ({rc}): {(self.err or last_error)()}")
        return rc


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"MI355X kernel library not built: {LIB_PATH} is missing "
                               "(run python mace-million_amd/build.py)")
        so = ctypes.CDLL(LIB_PATH)
        for name, argt in SIGNATURES.items():
            f = getattr(so, name)
            f.argtypes = argt
            f.restype = ctypes.c_char_p if name == "mm_last_error" else ctypes.c_int
        if so.mm_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has argument conventions version {so.mm_version()}, this binding needs "
                               f"{ABI_VERSION}: rebuild it (python mace-million_amd/build.py)")
        _lib = so
    return _lib


def last_error():
    return lib().mm_last_error().decode()


def fn(name):
    return _Fn(name, getattr(lib(), name))


class _Namespace:
    def __getattr__(self, name):
        f = fn(name)
        setattr(self, name, f)
        return f


K = _Namespace()


def stream():
    """Handle of the current torch stream (HIP stream) for the kernels."""
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

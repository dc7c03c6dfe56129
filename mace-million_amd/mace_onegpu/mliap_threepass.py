"""LAMMPS ML-IAP ("pair_style mliap unified <file.pt> 0") wrapper of the three-pass MACE evaluation on MI355X.

Same class, module path, constructor, attributes and compute_forces(data) contract as the reference's
mace_onegpu/mliap_threepass.py (ThreePassMLIAP, :155-622):
    pass A  receiver chunks of local atoms:  h1 = layer1 (no grad)                       -> H1[local]
            forward_exchange(H1)                                                        -> H1 on ghosts
    pass B  chunks: E2 = layer-2 energy;  dE2/drij -> pair forces,  dE2/dh1 -> G1[local + ghost]
            reverse_exchange(G1)                                                        -> ghost terms on owners
    pass C  chunks: layer 1 again with gradient; loss = scale R1 + G1 . h1; d/drij -> pair forces
H1, G1, the per-pair arrays and (MACE3P_CACHE_L1=1, the default) pass A's layer-1 message and density of every
local atom (8 KiB per atom, so that pass C does not recompute layer 1) persist; every other wide intermediate lives
in one chunk's workspace.  The arithmetic runs in the HIP kernels of libmace_million_amd.so
(fast_layers.FastLayers); with MACE3P_GRAPHS=1 the passes of full chunks are captured once as HIP graphs and
replayed per chunk (chunk_graphs.ChunkGraphExec).
"""
import json
import os
import time

import torch

from . import chunk_graphs, fast_layers
from .receiver_chunk_mace import chunk_topology, make_chunk

try:
    from lammps.mliap.mliap_unified_abc import MLIAPUnified
except ImportError:  # pragma: no cover - LAMMPS is not part of this build
    class MLIAPUnified:
        def __init__(self):
            pass

CHEMICAL_SYMBOLS = [
    "X", "H", "He", "Li", "Be", "B", "C", "N", "O", "F", "Ne", "Na", "Mg", "Al", "Si", "P", "S", "Cl", "Ar", "K",
    "Ca", "Sc", "Ti", "V", "Cr", "Mn", "Fe", "Co", "Ni", "Cu", "Zn", "Ga", "Ge", "As", "Se", "Br", "Kr", "Rb", "Sr",
    "Y", "Zr", "Nb", "Mo", "Tc", "Ru", "Rh", "Pd", "Ag", "Cd", "In", "Sn", "Sb", "Te", "I", "Xe", "Cs", "Ba", "La",
    "Ce", "Pr", "Nd", "Pm", "Sm", "Eu", "Gd", "Tb", "Dy", "Ho", "Er", "Tm", "Yb", "Lu", "Hf", "Ta", "W", "Re", "Os",
    "Ir", "Pt", "Au", "Hg", "Tl", "Pb", "Bi", "Po", "At", "Rn", "Fr", "Ra", "Ac"]

_RUNTIME = ("_fl", "_dev", "_cols", "_e0", "_loc", "_flag", "_log", "_D1", "_gx", "_use_graphs", "_fmax_abort",
            "_t_end", "_peak", "_topo", "_cache_l1", "_l1cache")

_INT_MAX = 2 ** 31 - 1


def _exchange(fn, src, dst, D):
    """LAMMPS' ML-IAP comm buffers are sized with 32-bit ints (ntotal * D): split the feature columns so that every
    call stays below 2^31 elements (mliap_threepass.py:40-55)."""
    nt = src.shape[0]
    if nt * D < _INT_MAX:
        fn(src, dst, D)
        return
    w = D
    while nt * w >= _INT_MAX and w > 1:
        w //= 2
    for c in range(0, D, w):
        cw = min(w, D - c)
        s = src[:, c:c + cw].contiguous()
        d = torch.empty_like(s)
        fn(s, d, cw)
        dst[:, c:c + cw] = d


class ThreePassMLIAP(MLIAPUnified):
    def __init__(self, model, chunk=16384, spline_grid=512, node_bucket=8192, e_align=65536, rebuild_config=None):
        super().__init__()
        self.model = model
        self.element_types = [CHEMICAL_SYMBOLS[int(z)] for z in model.atomic_numbers]
        self.num_species = len(self.element_types)
        self.rcutfac = 0.5 * float(model.r_max)
        self.ndescriptors = 1
        self.nparams = 1
        self.chunk = int(chunk)
        self.spline_grid = int(spline_grid)
        self.node_bucket = int(node_bucket)
        self.e_align = int(e_align)
        self.dtype = next(model.parameters()).dtype
        self.step = 0
        # rebuild recipe (class, constructor kwargs, state_dict): the file then stores no module object and the
        # model is constructed again on the first force call (mliap_threepass.py:172-202)
        self._rebuild = None
        if rebuild_config is not None:
            self._rebuild = (type(model), dict(rebuild_config),
                             {k: v.detach().cpu() for k, v in model.state_dict().items()})

    # runtime objects (device tables, kernels' constants, graphs) are rebuilt after unpickling
    def __getstate__(self):
        d = self.__dict__.copy()
        for k in _RUNTIME:
            d.pop(k, None)
        if d.get("_rebuild") is not None:
            d.pop("model", None)
        return d

    def _rebuild_model(self):
        cls, cfg, sd = self._rebuild
        m = cls(**cfg)
        m.load_state_dict(sd, strict=True)
        return m.to(self.dtype)

    # ------------------------------------------------------------------ setup
    def _setup(self, elems):
        dev = elems.device if elems.is_cuda else torch.device("cuda")
        self._dev = dev
        if getattr(self, "model", None) is None:
            self.model = self._rebuild_model()
        if os.environ.get("MACE3P_CHUNK"):
            self.chunk = int(os.environ["MACE3P_CHUNK"])
        self.model = self.model.to(dev).eval()
        for p in self.model.parameters():
            p.requires_grad_(False)
        cols = sorted(int(c) for c in torch.unique(elems).tolist())
        self._cols = cols
        # MACE3P_ACE_L1=1 (default): layer 1 in the exact density-projection form (csrc/ace.hip)
        ace = os.environ.get("MACE3P_ACE_L1", "1") == "1"
        self._fl = fast_layers.FastLayers(self.model, cols, spline_grid=self.spline_grid, device=dev, ace_layer1=ace)
        self.scale, self.shift = self._fl.scale, self._fl.shift
        self._e0 = self._fl.e0
        self._loc = None
        self._flag = None
        self._D1 = 4 * self.model.spec.C
        self._fmax_abort = float(os.environ.get("MACE3P_FMAX_ABORT", "100.0"))
        # MACE3P_CACHE_L1=1 (default): pass A keeps the layer-1 message and density of every local atom
        # (8 KiB per atom) and pass C reuses them instead of recomputing layer 1
        self._cache_l1 = os.environ.get("MACE3P_CACHE_L1", "1") == "1"
        self._l1cache = None
        self._use_graphs = os.environ.get("MACE3P_GRAPHS", "0") == "1"
        self._gx = None
        self._peak = 0.0
        path = os.environ.get("MACE3P_LOG")
        self._log = open(path, "a", buffering=1) if path else None

    def _prepare_graphs(self, graphs, nt):
        """A captured executor that fits every full chunk of this call (recaptured when a capacity is exceeded);
        None without full chunks (mliap_threepass.py:390-431)."""
        full = [g for g in graphs if g.nC == self.chunk]
        if not full:
            return None
        n_max = max(g.n_nodes for g in full)
        e_max = max(g.nE for g in full)
        gx = self._gx
        if gx is None or gx.cache_layer1 != self._cache_l1 or not gx.fits(n_max, e_max, nt):
            self._gx = gx = None
            torch.cuda.empty_cache()
            margin = float(os.environ.get("MACE3P_CAP_MARGIN", "1.25"))
            n_cap, e_cap, nt_cap = chunk_graphs.capacities(n_max, e_max, nt, self.e_align, margin)
            gx = chunk_graphs.ChunkGraphExec(self._fl, self.chunk, n_cap, e_cap, nt_cap, "rij", self._cache_l1,
                                             exchange=True)
            self._gx = gx
            self.n_captures = getattr(self, "n_captures", 0) + 1
            if self._log is not None:
                self._log.write(json.dumps(dict(capture=dict(n_cap=n_cap, e_cap=e_cap, nt_cap=nt_cap))) + "\n")
        gx.begin(graphs)
        return gx

    def _topology_all(self, bounds, rp_cpu, pi, pj, nl, nt):
        """{(a, b): (nodes int32, local sender index int32 [nE])} for every receiver chunk, identical to
        ThreePassMLIAP._topology chunk by chunk (mliap_threepass.py:288-310, :344-388)."""
        dev = self._dev
        if self._loc is None or self._loc.numel() < nt:
            self._loc = torch.full((max(nt, 1),), -1, dtype=torch.int32, device=dev)
            self._flag = torch.zeros(max(nt, 1), dtype=torch.bool, device=dev)
        out = {}
        for a, b in bounds:
            e0, e1 = int(rp_cpu[a]), int(rp_cpu[b])
            out[(a, b)] = chunk_topology(a, b, e0, e1, pj, self._loc, self._flag)
        return out

    # ------------------------------------------------------------------ LAMMPS entry point
    def compute_forces(self, data):
        nl, nt, P = int(data.nlocal), int(data.ntotal), int(data.npairs)
        if nl == 0 or P <= 1:
            return
        t_start = time.perf_counter()
        # int32 neighbour-slot guard of the LAMMPS/Kokkos neighbour list (mliap_threepass.py:450-461)
        skin = float(os.environ.get("MACE3P_SKIN", "2.0"))
        rmax = 2.0 * self.rcutfac
        est_slots = P * ((rmax + skin) / rmax) ** 3
        if est_slots > 0.95 * 2 ** 31 and os.environ.get("MACE3P_ALLOW_HUGE", "0") != "1":
            raise RuntimeError(f"ThreePassMLIAP guard: nlocal={nl:,}, pairs={P:,} -> estimated LAMMPS neighbour slots "
                               f"{est_slots:.3e} is close to the 2^31 int32 limit of the Kokkos neighbour list "
                               f"(skin {skin} A). Use fewer atoms per GPU, a smaller skin, or more GPUs.")
        elems = torch.as_tensor(data.elems).long()
        if not hasattr(self, "_fl") or not set(torch.unique(elems).tolist()) <= set(self._cols):
            self._setup(elems)
        self.step += 1
        dev, fl, D1 = self._dev, self._fl, self._D1
        elems = elems.to(dev)
        pi = torch.as_tensor(data.pair_i).to(dev).int()
        pj = torch.as_tensor(data.pair_j).to(dev).int()
        rij = torch.as_tensor(data.rij).to(dev).double()
        order = None
        if not bool((pi[1:] >= pi[:-1]).all()):
            order = torch.argsort(pi, stable=True)
            pi, pj, rij = pi[order], pj[order], rij[order]
        pi, pj, rij = pi.contiguous(), pj.contiguous(), rij.contiguous()
        rp = torch.searchsorted(pi, torch.arange(nl + 1, device=dev, dtype=pi.dtype))
        rp_cpu = rp.cpu().numpy()
        C = self.chunk
        bounds = [(a, min(a + C, nl)) for a in range(0, nl, C)]
        node_spec_all = fl.col2s[elems]
        t = {}
        t0 = time.perf_counter()
        topo = self._topology_all(bounds, rp_cpu, pi, pj, nl, nt)
        graphs = []
        for a, b in bounds:
            e0, e1 = int(rp_cpu[a]), int(rp_cpu[b])
            g = make_chunk(a, b, e0, e1, topo[(a, b)][0], topo[(a, b)][1], rp, node_spec_all)
            g.rij, g.pair_i = rij[e0:e1], pi[e0:e1]
            graphs.append(g)
        gx = self._prepare_graphs(graphs, nt) if self._use_graphs else None
        torch.cuda.synchronize()
        t["A_topology"] = time.perf_counter() - t0
        PF = torch.zeros(P, 3, dtype=torch.float32, device=dev)
        # ---------------- pass A
        t0 = time.perf_counter()
        cache = None
        if gx is not None:      # the executor's static buffers: its graphs read and write them in place
            H1, eat = gx.H1[:nt], gx.eat[:nl]
            H1.zero_()
            cache = gx.cache()
        else:
            H1 = torch.zeros(nt, D1, dtype=torch.float32, device=dev)
            eat = torch.zeros(nl, dtype=torch.float64, device=dev)
            if self._cache_l1:
                if self._l1cache is None or self._l1cache["rho"].numel() < nl:
                    self._l1cache = fl.layer1_cache(nl)
                cache = self._l1cache
        for g in graphs:
            if gx is not None and g.nC == C:
                gx.pass_a(g)
            else:
                fl.pass_a(g, H1, cache)
        H1x = gx.H1x[:nt] if gx is not None else torch.empty_like(H1)
        _exchange(data.forward_exchange, H1, H1x, D1)
        del H1
        torch.cuda.synchronize()
        t["A"] = time.perf_counter() - t0
        # ---------------- pass B
        t0 = time.perf_counter()
        if gx is not None:
            G1 = gx.G1[:nt]
            G1.zero_()
            eat.zero_()
        else:
            G1 = torch.zeros_like(H1x)
        for g in graphs:
            if gx is not None and g.nC == C:
                gx.pass_b(g)
            else:
                fl.pass_b(g, H1x, G1, PF, eat)
        H1c = H1x if cache is not None else None       # pass C reads h1 from H1x only with the layer-1 cache
        del H1x
        G1r = gx.G1r[:nt] if gx is not None else torch.empty_like(G1)
        _exchange(data.reverse_exchange, G1, G1r, D1)
        del G1
        torch.cuda.synchronize()
        t["B"] = time.perf_counter() - t0
        # ---------------- pass C
        t0 = time.perf_counter()
        for g in graphs:
            if gx is not None and g.nC == C:
                gx.pass_c(g)
            elif cache is None:
                fl.pass_c(g, G1r, PF, eat)
            else:
                fl.pass_c(g, G1r, PF, eat, H1c, cache)
        if gx is not None:
            gx.finish(graphs, PF)
        del G1r, H1c
        torch.cuda.synchronize()
        t["C"] = time.perf_counter() - t0
        eat = eat + self._e0[elems[:nl]] + self.shift
        PF = PF.double()
        if order is not None:
            out = torch.empty_like(PF)
            out[order] = PF
            PF = out
        # non-finite / absurd output guard (mliap_threepass.py:595-601)
        fmax = float(PF.abs().max()) if PF.numel() else 0.0
        if not (bool(torch.isfinite(eat).all()) and fmax == fmax and fmax < self._fmax_abort):
            raise RuntimeError(f"ThreePassMLIAP guard: non-finite or absurd output at call {self.step} "
                               f"(max |pair force| = {fmax:.3e} eV/A, limit {self._fmax_abort:g}); aborting before LAMMPS "
                               f"integrates it. The model is probably extrapolating (check the trajectory / training data).")
        torch.as_tensor(data.eatoms).copy_(eat)
        data.energy = float(eat.sum())
        data.update_pair_forces_gpu(PF)
        self.last_timings = t
        if self._log is not None:
            self._log.write(json.dumps(dict(step=self.step, nlocal=nl, ntotal=nt, npairs=P, chunks=len(bounds),
                                            sorted_pairs=order is None, t_total=time.perf_counter() - t_start,
                                            **t)) + "\n")

    def compute_descriptors(self, data):
        pass

    def compute_gradients(self, data):
        pass

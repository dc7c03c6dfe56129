"""Standalone receiver-chunked three-pass evaluator and its neighbour list (no LAMMPS).

Mirrors mace_onegpu/receiver_chunk_mace.py of the reference:
  * System (receiver_chunk_mace.py:91-165): positions wrapped and sorted in Morton order of cells, cell-list
    neighbour list -- here built by the HIP kernels of csrc/nlist.hip (bit-exact with the reference), stored as a
    CSR (rowptr int64 [N+1], senders int32 [E]) in the sorted index space;
  * chunk topology (LocalGraph, receiver_chunk_mace.py:169-215, and ThreePassMLIAP._topology,
    mliap_threepass.py:288-310): receivers of the chunk first, then the outside senders in ascending order;
  * ReceiverChunkMACE.compute (receiver_chunk_mace.py:278-386): passes A, B, C over receiver chunks; edge vectors
    are the fp64 minimum images of the sorted positions; forces F = -dE/dx in fp64.
"""
import ctypes
import os
import time

import numpy as np
import torch

from ._lib import K, stream


def host_f64(vals):
    return ctypes.cast((ctypes.c_double * len(vals))(*[float(v) for v in vals]), ctypes.c_void_p)


def host_i32(vals):
    return ctypes.cast((ctypes.c_int * len(vals))(*[int(v) for v in vals]), ctypes.c_void_p)


class System:
    """Positions sorted in Morton order of cells; perm maps sorted -> original index.  pos [N, 3] fp64,
    box [3], spidx [N] model element index; r_cut = cutoff of the neighbour list (r_max, or r_max + skin)."""

    def __init__(self, pos, box, spidx, r_max, device="cuda"):
        dev = torch.device(device)
        self.device = dev
        self.box = np.asarray(box, dtype=np.float64).reshape(3)
        if not (self.box > 2 * r_max).all():
            raise ValueError("minimum image needs box > 2 r_max in every direction")
        self.r_max = float(r_max)
        pos = torch.as_tensor(pos, dtype=torch.float64).to(dev).contiguous()
        spidx = torch.as_tensor(spidx).to(dev).to(torch.int32).contiguous()
        N = pos.shape[0]
        self.N = N
        self.ncell = np.maximum(np.floor(self.box / r_max).astype(np.int64), 1)
        cs = self.box / self.ncell.astype(np.float64)
        self._box_h, self._nc_h, self._cs_h = host_f64(self.box), host_i32(self.ncell), host_f64(cs)
        pos_w = torch.empty_like(pos)
        cell = torch.empty(N, 3, dtype=torch.int32, device=dev)
        key = torch.empty(N, dtype=torch.int64, device=dev)
        idx = torch.empty(N, dtype=torch.int64, device=dev)
        K.mm_nl_prepare(pos, N, self._box_h, self._nc_h, self._cs_h, pos_w, cell, key, idx, stream())
        nbytes = ctypes.c_size_t(0)
        K.mm_nl_workspace_bytes(N + 1, ctypes.byref(nbytes))
        self._ws = torch.empty(int(nbytes.value), dtype=torch.uint8, device=dev)
        key_s = torch.empty_like(key)
        perm = torch.empty_like(idx)
        K.mm_nl_sort(key, key_s, idx, perm, N, self._ws, self._ws.numel(), stream())
        self.perm = perm
        self.pos = torch.empty_like(pos)
        self.cell = torch.empty_like(cell)
        self.spidx = torch.empty_like(spidx)
        K.mm_nl_gather(perm, N, pos_w, cell, spidx, self.pos, self.cell, self.spidx, stream())
        del pos_w, cell, key, idx, key_s

    def min_image(self, v):
        box = torch.as_tensor(self.box, dtype=v.dtype, device=v.device)
        return v - box * torch.round(v / box)

    def build_neighbors(self, r_cut=None):
        """CSR neighbour list within r_cut (default r_max) in the reference's candidate order.  The cell grid
        is the one of r_max (as System.__init__ fixes it), so r_cut must not exceed r_max unless the System was
        created with r_max = r_cut."""
        r_cut = self.r_max if r_cut is None else float(r_cut)
        if r_cut > self.r_max:
            raise ValueError("r_cut larger than the cell size of this System")
        dev, N = self.device, self.N
        nc = self.ncell
        ncells = int(np.prod(nc))
        brute = int((nc < 3).any())
        start = torch.empty(ncells, dtype=torch.int32, device=dev)
        count = torch.empty(ncells, dtype=torch.int32, device=dev)
        K.mm_nl_cell_ranges(self.cell, N, self._nc_h, start, count, stream())
        NN = torch.empty(N, dtype=torch.int32, device=dev)
        r2 = r_cut ** 2
        K.mm_nl_count(self.pos, self.cell, N, self._box_h, self._nc_h, start, count, r2, brute, NN, stream())
        rowptr = torch.empty(N + 1, dtype=torch.int64, device=dev)
        K.mm_nl_scan(NN, rowptr, N, self._ws, self._ws.numel(), stream())
        E = int(rowptr[-1])
        send = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
        K.mm_nl_fill(self.pos, self.cell, N, self._box_h, self._nc_h, start, count, r2, brute, rowptr, send,
                     stream())
        self.NN, self.rowptr, self.send = NN, rowptr, send[:E]
        self.MN = int(NN.max()) if N else 0
        return self.MN


class ChunkGraph:
    """Topology and inputs of one receiver chunk [a, b) whose edges are [e0, e1) of the receiver-sorted pairs."""
    rij = None
    pair_i = None
    pos = None
    box_host = None
    recv_local = None
    E_dev = None   # device int32 [1]: the edge count the edge kernels read (graph replays); None: nE
    N_dev = None   # device int32 [1]: the node count of the node-level linears (graph replays); None: n_nodes


def chunk_topology(a, b, e0, e1, pj, loc, flag):
    """Receivers a..b-1 first, then the senders outside [a, b) in ascending order; int32 local sender index per
    edge.  Restates ThreePassMLIAP._topology (mliap_threepass.py:288-310); loc (int32, -1) and flag (bool, False)
    are scratch arrays over all atoms and are restored before returning."""
    dev = pj.device
    nC = b - a
    send_g = pj[e0:e1].long()
    loc[a:b] = torch.arange(nC, device=dev, dtype=loc.dtype)
    flag[send_g] = True
    flag[a:b] = False
    new = torch.nonzero(flag).squeeze(1)
    flag[new] = False
    loc[new] = torch.arange(nC, nC + new.numel(), device=dev, dtype=loc.dtype)
    nodes = torch.cat([torch.arange(a, b, device=dev, dtype=torch.int32), new.to(torch.int32)])
    ls = loc[send_g].contiguous()
    loc[nodes.long()] = -1
    return nodes, ls


def check_chunk(g, n_atoms, n_species=None):
    """Host-side range check of one chunk's index arrays before its kernels dereference them (opt-in:
    MACE3P_CHECK=1 in ThreePassMLIAP, check=True in ReceiverChunkMACE; a few device-to-host reads per chunk).
    Raises ValueError naming the array: the receiver CSR (monotone, from 0 to nE), local senders in
    [0, n_nodes), node rows in [0, n_atoms) with the receivers a..b-1 first, species in [0, n_species), and the
    receiver of every edge inside the chunk."""
    def span(t):
        t = t.reshape(-1)
        return (int(t.min()), int(t.max())) if t.numel() else (0, -1)
    nC, nE, n = g.nC, g.nE, g.n_nodes
    rp = g.rowptr
    if rp.numel() != nC + 1:
        raise ValueError(f"chunk [{g.a}, {g.b}): rowptr has {rp.numel()} entries, expected {nC + 1}")
    if int(rp[0]) != 0 or int(rp[-1]) != nE or (nC > 0 and bool((rp[1:] < rp[:-1]).any())):
        raise ValueError(f"chunk [{g.a}, {g.b}): rowptr is not a monotone CSR from 0 to nE = {nE}")
    lo, hi = span(g.ls[:nE])
    if g.ls.numel() < nE or lo < 0 or hi >= n:
        raise ValueError(f"chunk [{g.a}, {g.b}): local senders span [{lo}, {hi}], outside [0, {n})")
    lo, hi = span(g.nodes)
    if g.nodes.numel() != n or lo < 0 or hi >= n_atoms:
        raise ValueError(f"chunk [{g.a}, {g.b}): node rows span [{lo}, {hi}], outside [0, {n_atoms})")
    if not torch.equal(g.nodes[:nC].long().cpu(), torch.arange(g.a, g.b)):
        raise ValueError(f"chunk [{g.a}, {g.b}): the first nodes are not the receivers a..b-1")
    lo, hi = span(g.node_spec)
    if g.node_spec.numel() != n or lo < 0 or (n_species is not None and hi >= n_species):
        raise ValueError(f"chunk [{g.a}, {g.b}): node species span [{lo}, {hi}] (species not in the model's "
                         f"present columns?)")
    if g.rij is not None:
        if g.rij.shape[0] < nE or g.pair_i.numel() < nE:
            raise ValueError(f"chunk [{g.a}, {g.b}): fewer pair vectors or receivers than edges")
        recv = g.pair_i[:nE].long() - g.a
    else:
        recv = g.recv_local[:nE].long()
    lo, hi = span(recv)
    if lo < 0 or hi >= nC:
        raise ValueError(f"chunk [{g.a}, {g.b}): edge receivers span [{lo}, {hi}] (chunk-local), outside [0, {nC})")


def make_chunk(a, b, e0, e1, nodes, ls, rowptr_full, node_spec_all):
    g = ChunkGraph()
    g.a, g.b, g.e0, g.e1 = a, b, e0, e1
    g.nC, g.nE = b - a, e1 - e0
    g.nodes = nodes.contiguous()
    g.n_nodes = nodes.numel()
    g.ls = ls
    g.rowptr = (rowptr_full[a:b + 1] - e0).to(torch.int32).contiguous()
    g.node_spec = node_spec_all[g.nodes.long()].contiguous()
    return g


class ReceiverChunkMACE:
    """Three-pass energy + forces of a System with the MI355X kernels (fp32 arithmetic, fp64 energies and forces)."""

    def __init__(self, model, chunk=16384, spline_grid=512, device="cuda", cache_layer1=True, use_graphs=False,
                 e_align=65536, ace_layer1=True, check=None, deterministic=None, low_memory=False):
        self.model, self.chunk, self.spline_grid = model, int(chunk), int(spline_grid)
        # low_memory: the reference's own memory layout (receiver_chunk_mace.py:278-386): each chunk's topology is
        # built when a pass reaches it and dropped after it, and each chunk's pair forces are added to F at once
        # (mm_chunk_forces), so what stays resident per atom is the positions, the pair list, H1, G1 and F.  No
        # HIP graphs and no layer-1 cache in this mode; compute() returns PF = None.
        self.low_memory = bool(low_memory)
        if self.low_memory and use_graphs:
            raise ValueError("low_memory evaluates chunks eagerly (no HIP graphs)")
        # host-side range check of every chunk's index arrays before its kernels run (check_chunk)
        self.check = (os.environ.get("MACE3P_CHECK", "0") == "1") if check is None else bool(check)
        # bitwise-repeatable evaluations (the sender-feature gradient summed in a fixed order, FastLayers)
        self.deterministic = ((os.environ.get("MACE3P_DETERMINISTIC", "0") == "1") if deterministic is None
                              else bool(deterministic))
        self.ace_layer1 = bool(ace_layer1)       # layer 1 in the exact density-projection form (csrc/ace.hip)
        self.dev = torch.device(device)
        self.fl = None
        self.H1 = self.G1 = None          # H1 and G1 of the last call (kept for inspection until the next one)
        self.D1 = 4 * model.spec.C
        # keep pass A's layer-1 message and density (8 KiB per atom) so that pass C does not recompute them
        self.cache_layer1 = bool(cache_layer1) and not self.low_memory
        self._cache = None
        # full chunks replayed from HIP graphs (chunk_graphs.ChunkGraphExec), recaptured when a capacity is exceeded
        self.use_graphs, self.e_align = bool(use_graphs), int(e_align)
        self._gx = None
        self.n_captures = 0

    def _layers(self, sysm):
        from .fast_layers import FastLayers
        key = (sysm.spidx.data_ptr(), sysm.spidx.numel(), sysm.spidx._version)
        if self.fl is not None and getattr(self, "_cols_key", None) == key:
            return self.fl          # same species array as the last call: no device-to-host read
        cols = sorted(int(c) for c in torch.unique(sysm.spidx.long()).tolist())
        if self.fl is None or self.fl.cols != cols:
            self.fl = FastLayers(self.model, cols, self.spline_grid, device=self.dev, ace_layer1=self.ace_layer1,
                                 deterministic=self.deterministic)
        self._cols_key = key
        return self.fl

    def graphs(self, sysm):
        """Topologies of all chunks (a pair list that builds its own chunks -- the MD driver's -- is asked for
        them)."""
        fl = self._layers(sysm)
        if getattr(sysm, "chunk_graphs", None) is not None:
            return sysm.chunk_graphs(self.chunk, fl.col2s)
        return list(self._chunk_iter(sysm, fl))

    def _chunk_iter(self, sysm, fl, rp_cpu=None):
        """The chunks of a System one at a time (topology built when the chunk is reached)."""
        dev, N = self.dev, sysm.N
        rp = sysm.rowptr
        rp_cpu = rp.cpu().numpy() if rp_cpu is None else rp_cpu
        loc = torch.full((N,), -1, dtype=torch.int32, device=dev)
        flag = torch.zeros(N, dtype=torch.bool, device=dev)
        node_spec_all = fl.col2s[sysm.spidx.long()]
        box_h = host_f64(sysm.box)
        for a in range(0, N, self.chunk):
            b = min(a + self.chunk, N)
            e0, e1 = int(rp_cpu[a]), int(rp_cpu[b])
            nodes, ls = chunk_topology(a, b, e0, e1, sysm.send, loc, flag)
            g = make_chunk(a, b, e0, e1, nodes, ls, rp, node_spec_all)
            g.pos, g.box_host = sysm.pos, box_h
            g.recv_local = torch.repeat_interleave(torch.arange(b - a, device=dev, dtype=torch.int32),
                                                   sysm.NN[a:b].long(), output_size=e1 - e0)
            yield g

    def _checked(self, graphs, sysm, fl):
        if self.check:
            for g in graphs:
                check_chunk(g, sysm.N, fl.S)
        return graphs

    def _graph_exec(self, fl, sysm, graphs):
        """The HIP-graph executor of this call's full chunks, their topology loaded (a new executor -- new
        captures -- when the box changes or a capacity is exceeded); None without full chunks."""
        from . import chunk_graphs
        full = [g for g in graphs if g.nC == self.chunk]
        if not full:
            return None
        n_max = max(g.n_nodes for g in full)
        e_max = max(g.nE for g in full)
        box = tuple(float(b) for b in sysm.box)
        gx = self._gx
        if gx is None or gx.box != box or not gx.fits(n_max, e_max, sysm.N):
            self._gx = gx = None
            torch.cuda.empty_cache()
            # the chunks' nodes and edges change as atoms move (25 % headroom); the atom count of a System does not
            n_cap, e_cap, nt_cap = chunk_graphs.capacities(n_max, e_max, sysm.N, self.e_align, nt_margin=1.0)
            gx = chunk_graphs.ChunkGraphExec(fl, self.chunk, n_cap, e_cap, nt_cap, "pos", self.cache_layer1,
                                             box_host=host_f64(box))
            gx.box = box
            self._gx = gx
            self.n_captures += 1
        gx.set_positions(sysm.pos)
        gx.begin(graphs)
        return gx

    def _idle_exec(self, sysm):
        """The graph executor of an earlier call, for its static H1 / G1 / layer-1 cache rows, when they hold this
        system (same box, at most nt_cap atoms, the same layer-1 cache setting); else None."""
        gx = self._gx
        if gx is None or gx.box != tuple(float(b) for b in sysm.box) or sysm.N > gx.nt_cap:
            return None
        if gx.cache_layer1 != self.cache_layer1:
            return None
        return gx

    def _compute_low_memory(self, sysm, timings):
        """The three passes with each chunk's topology rebuilt when a pass reaches it and its pair forces added to
        F at once (low_memory); returns (E, eat, F, None)."""
        fl = self._layers(sysm)
        dev, N = self.dev, sysm.N
        self.H1 = self.G1 = None          # the previous call's rows go before this call allocates its own
        rp_cpu = sysm.rowptr.cpu().numpy()
        sync = torch.cuda.synchronize if timings is not None else (lambda: None)
        t, t0 = {}, time.perf_counter()
        H1 = torch.empty(N, self.D1, dtype=torch.float32, device=dev)
        for g in self._checked_iter(sysm, fl, rp_cpu):
            fl.pass_a(g, H1)
        sync()
        t["A"], t0 = time.perf_counter() - t0, time.perf_counter()
        G1 = torch.zeros_like(H1)
        eat = torch.zeros(N, dtype=torch.float64, device=dev)
        F = torch.zeros(N, 3, dtype=torch.float64, device=dev)
        for g in self._checked_iter(sysm, fl, rp_cpu):
            fl.pass_b(g, H1, G1, None, eat, forces=F)
        sync()
        t["B"], t0 = time.perf_counter() - t0, time.perf_counter()
        for g in self._checked_iter(sysm, fl, rp_cpu):
            fl.pass_c(g, G1, None, eat, forces=F)
        sync()
        t["C"] = time.perf_counter() - t0
        eat += fl.e0[sysm.spidx.long()] + fl.shift
        if timings is not None:
            timings.update(t)
        self.H1, self.G1 = H1, G1
        return float(eat.sum()), eat, F, None

    def _checked_iter(self, sysm, fl, rp_cpu):
        for g in self._chunk_iter(sysm, fl, rp_cpu):
            if self.check:
                check_chunk(g, sysm.N, fl.S)
            yield g

    def compute(self, sysm, graphs=None, timings=None):
        """Returns (E float, eat fp64 [N], F fp64 [N, 3], PF fp32 [E, 3]) in the sorted index space (PF None with
        low_memory)."""
        if self.low_memory:
            if graphs is not None or getattr(sysm, "chunk_graphs", None) is not None:
                raise ValueError("low_memory builds its chunks from a System's neighbour list")
            return self._compute_low_memory(sysm, timings)
        self.H1 = self.G1 = None          # the previous call's rows go before this call allocates its own
        fl = self._layers(sysm)
        dev, N = self.dev, sysm.N
        graphs = self._checked(graphs if graphs is not None else self.graphs(sysm), sysm, fl)
        E = sum(g.nE for g in graphs)
        t = {}
        sync = torch.cuda.synchronize if timings is not None else (lambda: None)   # pass timings only on request
        sync()
        t0 = time.perf_counter()
        gx = self._graph_exec(fl, sysm, graphs) if self.use_graphs else None
        # without graphs for this call, an executor of an earlier call whose static rows hold this system lends
        # them, instead of a second set of H1, G1 and layer-1 cache rows
        bx = gx if gx is not None else self._idle_exec(sysm)
        if bx is not None and bx.ws is not None:
            # the executor's workspace (sized for its capacities) serves the eager chunks too: a partial chunk,
            # or every chunk of a call without graphs, instead of a second workspace
            fl.ws = bx.ws
        nC = self.chunk
        cache = None
        # pass A writes every column of every receiver's h1 row, and pass B stores every pair force of its chunk
        # before pass C adds to it: neither buffer is cleared first (G1 and eat are accumulated into and are)
        if bx is not None:      # the executor's static buffers: its graphs read and write them in place
            H1, G1, eat = bx.H1x[:N], bx.G1[:N], bx.eat[:N]
            cache = bx.cache()
        else:
            H1 = torch.empty(N, self.D1, dtype=torch.float32, device=dev)
            if self.cache_layer1:
                if self._cache is None or self._cache["rho"].numel() < N:
                    self._cache = fl.layer1_cache(N)
                cache = self._cache
        for g in graphs:
            if gx is not None and g.nC == nC:
                gx.pass_a(g)
            else:
                fl.pass_a(g, H1, cache)
        sync()
        t["A"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        if bx is not None:
            G1.zero_()
            eat.zero_()
        else:
            G1 = torch.zeros_like(H1)
            eat = torch.zeros(N, dtype=torch.float64, device=dev)
        PF = torch.empty(max(E, 1), 3, dtype=torch.float32, device=dev)
        for g in graphs:
            if gx is not None and g.nC == nC:
                gx.pass_b(g)
            else:
                fl.pass_b(g, H1, G1, PF, eat)
        sync()
        t["B"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        for g in graphs:
            if gx is not None and g.nC == nC:
                gx.pass_c(g)
            else:
                fl.pass_c(g, G1, PF, eat, H1, cache)
        if gx is not None:
            gx.finish(graphs, PF)
        sync()
        t["C"] = time.perf_counter() - t0
        eat = eat + fl.e0[sysm.spidx.long()] + fl.shift
        F = pair_to_atom_forces(sysm, PF, graphs)
        if timings is not None:
            timings.update(t)
        self.H1, self.G1 = H1, G1
        return float(eat.sum()), eat, F, PF[:E]


INT32_MAX = 2 ** 31 - 1


def pair_to_atom_forces(sysm, PF, graphs=None):
    """F_i = -sum_{e: recv=i} PF_e + sum_{e: send=i} PF_e (v_e = x_recv - x_send), deterministic CSR sums.  Up to
    2^31 - 1 pairs through one sender sort of the whole list (kept on the System); beyond that, chunk by chunk
    through each chunk's own sender CSR (mm_chunk_forces; a sort of more than 2^31 - 1 keys is not available)."""
    if getattr(sysm, "atom_forces_fn", None) is not None:     # MD pair list filtered from a skin list
        return sysm.atom_forces_fn(PF)
    dev, N = sysm.device, sysm.N
    if sysm.send.numel() > INT32_MAX:
        if graphs is None:
            raise ValueError("more than 2^31 - 1 pairs: per-atom forces need the chunk topologies")
        from .fast_layers import sender_csr
        F = torch.zeros(N, 3, dtype=torch.float64, device=dev)
        for g in graphs:
            srp, sperm = sender_csr(g)
            K.mm_chunk_forces(g.n_nodes, g.nC, g.rowptr, srp, sperm, g.nodes, PF[g.e0:g.e1], F, stream())
        return F
    if not hasattr(sysm, "_s_perm") or sysm._s_perm_E != sysm.send.numel():
        s_perm = torch.argsort(sysm.send.long(), stable=True)
        cnt = torch.bincount(sysm.send.long(), minlength=N)
        s_rowptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        s_rowptr[1:] = torch.cumsum(cnt, 0)
        sysm._s_perm, sysm._s_rowptr, sysm._s_perm_E = s_perm, s_rowptr, sysm.send.numel()
    F = torch.empty(N, 3, dtype=torch.float64, device=dev)
    K.mm_pair_forces_to_atoms(N, sysm.rowptr, sysm._s_rowptr, sysm._s_perm, PF, F, stream())
    return F


def _sync():
    torch.cuda.synchronize()


def _in_input_order(sysm, t):
    """Rows of a sorted-index-space tensor in the input atom order (sysm.perm: sorted -> input index)."""
    out = torch.empty_like(t)
    out[sysm.perm.long()] = t
    return out


def main(argv=None):
    """Command line of the standalone evaluator (the reference's receiver_chunk_mace.main, :422-518): energy and
    forces of one structure, with the neighbour-list and evaluation times, peak device memory and, optionally, the
    replica check (every atom of a periodic replica against its image in the base cell, evaluated alone) and a
    JSON record.

        python -m mace_onegpu.receiver_chunk_mace --water 343000 --chunk 131072 --repeat 3 --graphs
        python -m mace_onegpu.receiver_chunk_mace --base cell.xyz --rep 4 4 4 --check-replica --json out.json
    """
    import argparse
    import json

    from . import systems
    from .model import from_arg

    ap = argparse.ArgumentParser(prog="python -m mace_onegpu.receiver_chunk_mace", description=main.__doc__.split(
        "\n\n")[0])
    ap.add_argument("--model", default="seed:0", help='"seed:N" (random-init weights) or a weights file '
                                                      "(.safetensors or a weights-only torch state_dict)")
    systems.add_structure_args(ap)
    ap.add_argument("--chunk", type=int, default=131072, help="receivers per chunk")
    ap.add_argument("--repeat", type=int, default=1, help="evaluations of the same structure")
    ap.add_argument("--graphs", action="store_true", help="replay full chunks from HIP graphs")
    ap.add_argument("--low-memory", action="store_true", help="the reference's memory layout (per-pass topologies)")
    ap.add_argument("--deterministic", action="store_true", help="bitwise-repeatable sender-feature gradient")
    ap.add_argument("--check-replica", action="store_true", help="with --rep: every atom against its base image")
    ap.add_argument("--json", default=None, help="write the results here")
    a = ap.parse_args(argv)
    if a.check_replica and tuple(a.rep) == (1, 1, 1):
        ap.error("--check-replica needs --rep with more than one copy")
    if not torch.cuda.is_available():
        raise SystemExit("the evaluator runs on the GPU; no GPU is visible")
    model = from_arg(a.model)
    r_max = float(model.spec.r_max)
    pos, box, Z, base = systems.structure_from_args(a)
    N = len(pos)
    print(f"N={N:,} box={np.round(box, 3).tolist()} chunk={a.chunk} graphs={a.graphs} low_memory={a.low_memory} "
          f"model={a.model}", flush=True)
    t0 = time.perf_counter()
    s = System(pos, box, np.asarray(Z) - 1, r_max, "cuda")
    s.build_neighbors()
    _sync()
    n_pairs = int(s.rowptr[-1])
    res = dict(N=N, pairs=n_pairs, chunk=a.chunk, graphs=a.graphs, low_memory=a.low_memory, model=a.model,
               t_neighbours=time.perf_counter() - t0, runs=[])
    print(f"neighbour list: {n_pairs:,} pairs ({n_pairs / N:.2f} per atom), {res['t_neighbours']:.2f} s", flush=True)
    ev = ReceiverChunkMACE(model, chunk=a.chunk, device="cuda", use_graphs=a.graphs, low_memory=a.low_memory,
                           deterministic=True if a.deterministic else None)
    E = eat = F = None
    for rep in range(a.repeat):
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        E, eat, F, _ = ev.compute(s)
        _sync()
        tt = time.perf_counter() - t0
        peak = torch.cuda.max_memory_allocated() / 1e9
        res["runs"].append(dict(energy=E, t_total=tt, atom_step_per_s=N / tt, peak_gb=peak))
        print(f"[rep {rep}] E={E:.6f} eV  t={tt:.3f} s ({N / tt:.3e} atom-step/s)  peak={peak:.2f} GB", flush=True)
    if a.check_replica:
        pb, bb, zb = base
        nb = len(pb)
        sb = System(pb, bb, np.asarray(zb) - 1, r_max, "cuda")
        sb.build_neighbors()
        Eb, eb, Fb, _ = ReceiverChunkMACE(model, chunk=a.chunk, device="cuda").compute(sb)
        Fb, eb = _in_input_order(sb, Fb), _in_input_order(sb, eb)
        Fo, eo = _in_input_order(s, F), _in_input_order(s, eat)
        img = torch.arange(N, device=Fo.device) % nb
        dF = float((Fo - Fb[img]).abs().max())
        de = float((eo - eb[img]).abs().max())
        res["replica_check"] = dict(base_atoms=nb, max_dF=dF, max_de=de, dE_per_atom=E / N - Eb / nb,
                                    max_F=float(Fb.abs().max()))
        print(f"REPLICA CHECK against the {nb}-atom base cell, every one of {N:,} atoms: max|dF|={dF:.3e} eV/A  "
              f"max|de_i|={de:.3e} eV  E/N - E_base/N_base = {E / N - Eb / nb:+.3e} eV/atom", flush=True)
    if a.json:
        with open(a.json, "w") as fh:
            json.dump(res, fh, indent=1)
    return res


if __name__ == "__main__":
    main()

"""HIP-graph execution of full receiver chunks (MACE3P_GRAPHS=1 / use_graphs=True), the MI355X counterpart of the
reference's _GraphExec / _prepare_graphs (mliap_threepass.py:58-152, 390-431).

Every FULL chunk (nC == chunk) of a call gets a slot: static topology buffers of fixed capacity (n_cap chunk
nodes, e_cap chunk edges) and its own three captured graphs, one per pass (A, B, C).  The passes of a chunk read
and write the executor's shared static buffers in place:

* H1 (pass A output; with a ghost exchange, H1x is its exchanged copy, otherwise H1x is the output itself);
* G1 (pass B scatter target) and G1r (the reverse-exchanged G1 that pass C reads, or G1 itself);
* the layer-1 cache (M, rho) and the per-atom energies eat.

So the only per-call traffic is one load of every chunk's topology into its slot and one copy of each chunk's
pair forces out of it: the edge offsets of a chunk change between calls.  All slots share one workspace: the
graphs are replayed one after another on the current stream.

The arithmetic is the eager path's (FastLayers.pass_a/b/c run on a static ChunkGraph), so the results agree with
the eager path up to the order of the fp32 atomic additions of the sender-feature gradient.

Padding:
* The captured launches are sized for the capacities, but the per-edge kernels (geometry, pair-force assembly)
  read the chunk's edge count from its CSR end (rowptr[nC], device memory) and the node-level linears the node
  count from the slot's device counter: a replay does the loaded chunk's own work.
* Edges beyond a chunk's nE are outside every receiver's CSR range, so no convolution reads them. They hold
  harmless inputs: in the LAMMPS path rij = (1.5 r_max, 0, 0) with receiver 0; in the standalone path the sender is
  a pad node.
* Nodes beyond the chunk's n_nodes point at a sink row (index nt_cap) of the static H1x / G1 / position
  buffers. H1x[sink] = 0, and a G1 scatter of pad rows would land in G1[sink], never in a real atom's row.
* The per-species receiver lists are loaded with the topology (built once per chunk object, outside the graphs).

Partial chunks run eagerly on the same buffers.  Buffers are cleared inside graphs with fill kernels only.
"""
import torch

from ._lib import K, stream
from .receiver_chunk_mace import ChunkGraph

C = 128


def _align(x, a):
    return ((int(x) + a - 1) // a) * a


def capacities(n_max, e_max, nt, e_align=65536, margin=1.25, nt_margin=None):
    """(n_cap, e_cap, nt_cap) with the reference's headroom (mliap_threepass.py:418-421).  nt_margin (default:
    margin) is the headroom of the atom rows: LAMMPS' ghost count changes between calls, a standalone system's
    atom count does not."""
    ntm = margin if nt_margin is None else nt_margin
    return _align(int(n_max * margin) + 2, 1024), _align(int(e_max * margin), e_align), int(nt * ntm) + 1024


class _Slot:
    """Static topology of one full chunk and its three captured passes."""

    def __init__(self, ex, j):
        dev, fl = ex.fl.dev, ex.fl
        i32 = dict(dtype=torch.int32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        nC, n_cap, e_cap = ex.C, ex.n_cap, ex.e_cap
        self.j = j
        self.a, self.b = j * nC, (j + 1) * nC
        self.rowptr = torch.zeros(nC + 1, **i32)
        self.ls = torch.zeros(e_cap, **i32)
        self.nodes = torch.full((n_cap,), ex.sink, **i32)
        self.node_spec = torch.zeros(n_cap, **i32)
        if ex.mode == "rij":
            self.rij = torch.zeros(e_cap, 3, dtype=torch.float64, device=dev)
            self.pair_i = torch.full((e_cap,), self.a, **i32)     # global receiver index (the kernel subtracts a)
        else:
            self.recv_local = torch.zeros(e_cap, **i32)
        self.lists = torch.zeros(fl.S * nC, **i32)
        self.list_counts = torch.zeros(fl.S, **i32)
        self.PF = torch.zeros(e_cap, 3, **f32)
        self.n_nodes_dev = torch.zeros(1, **i32)   # the loaded chunk's node count (its edge count is rowptr[nC])
        if getattr(fl, "deterministic", False):   # the sender CSR of the deterministic dL/dX sum, real edges only
            self.sender_rowptr = torch.zeros(n_cap + 1, **i32)
            self.sender_perm = torch.zeros(e_cap, **i32)
        self.graphs = None
        self.node_src, self.node_key, self.loaded = None, None, False
        self.nE = 0
        self.e0 = 0

    def chunk(self, ex):
        """The static ChunkGraph the captured passes run on (PF offsets index the slot's own PF buffer)."""
        g = ChunkGraph()
        g.a, g.b, g.e0, g.e1 = self.a, self.b, 0, ex.e_cap
        g.nC, g.nE, g.n_nodes = ex.C, ex.e_cap, ex.n_cap
        g.rowptr, g.ls, g.nodes, g.node_spec = self.rowptr, self.ls, self.nodes, self.node_spec
        g.lists, g.list_counts = self.lists, self.list_counts
        # the edge and node kernels read the loaded chunk's counts from device memory, so a replay does the
        # chunk's own work, not the capacities' (the grids are sized for the capacities)
        g.E_dev, g.N_dev = self.rowptr[ex.C:], self.n_nodes_dev
        if getattr(ex.fl, "deterministic", False):
            g.sender_rowptr, g.sender_perm = self.sender_rowptr, self.sender_perm
        if ex.mode == "rij":
            g.rij, g.pair_i = self.rij, self.pair_i
        else:
            g.pos, g.box_host, g.recv_local = ex.pos, ex.box_host, self.recv_local
        return g


class ChunkGraphExec:
    """Captured passes A/B/C of full chunks.  mode "rij": edge vectors come from LAMMPS' rij (pair_i global
    receiver); mode "pos": edge vectors are minimum images of positions (standalone System).  exchange=True: pass A
    writes H1 and pass C reads G1r (the caller runs the ghost exchanges H1 -> H1x and G1 -> G1r in between);
    exchange=False: H1 is H1x and G1r is G1."""

    def __init__(self, fl, chunk, n_cap, e_cap, nt_cap, mode, cache_layer1, box_host=None, exchange=False):
        if mode not in ("rij", "pos"):
            raise ValueError(mode)
        dev = fl.dev
        self.fl, self.C, self.n_cap, self.e_cap, self.nt_cap, self.mode = fl, int(chunk), n_cap, e_cap, nt_cap, mode
        self.cache_layer1 = bool(cache_layer1)
        self.exchange = bool(exchange)
        self.sink = nt_cap
        D1 = 4 * C
        f32 = dict(dtype=torch.float32, device=dev)
        if mode == "rij":
            self.pad_rij = torch.tensor([1.5 * fl.spec.r_max, 0.0, 0.0], dtype=torch.float64, device=dev)
        else:
            self.pos = torch.zeros(nt_cap + 1, 3, dtype=torch.float64, device=dev)
            self.box_host = box_host
        self.H1x = torch.zeros(nt_cap + 1, D1, **f32)      # row nt_cap: sink of the pad nodes (stays 0)
        self.G1 = torch.zeros(nt_cap + 1, D1, **f32)
        self.H1 = torch.zeros(nt_cap + 1, D1, **f32) if self.exchange else self.H1x
        self.G1r = torch.zeros(nt_cap + 1, D1, **f32) if self.exchange else self.G1
        self.M = torch.zeros(nt_cap, 16 * C, **f32) if self.cache_layer1 else None
        self.rho = torch.zeros(nt_cap, **f32) if self.cache_layer1 else None
        self.eat = torch.zeros(nt_cap, dtype=torch.float64, device=dev)
        self.slots = {}
        self.ws = None
        self.n_replays = 0
        self.n_captured = 0
        # one memory pool for the graphs of every slot: a replay's temporaries are dead when it ends and replays
        # never overlap (one stream), so graphs of different slots can share the pool's blocks
        self.pool = None

    def cache(self):
        return dict(M=self.M, rho=self.rho) if self.cache_layer1 else None

    def fits(self, n_nodes, nE, nt):
        return n_nodes <= self.n_cap - 1 and nE <= self.e_cap and nt <= self.nt_cap

    def set_positions(self, pos):
        """Standalone mode: the positions of the current call (rows beyond them and the sink row are 0)."""
        n = pos.shape[0]
        if n > self.nt_cap:
            raise ValueError("more atoms than the captured capacity")
        self.pos[:n].copy_(pos)
        self.pos[n:].zero_()

    # ------------------------------------------------------------------ per-call topology
    def _load(self, s, g):
        n, nE = g.n_nodes, g.nE
        if g.nC != self.C or not self.fits(n, nE, 0):
            raise ValueError(f"chunk ({g.nC} receivers, {n} nodes, {nE} edges) does not fit the captured "
                             f"capacities ({self.C}, {self.n_cap - 1}, {self.e_cap})")
        if g.a != s.a:
            raise ValueError(f"chunk starting at receiver {g.a} loaded into the slot of receiver {s.a}")
        # the per-species receiver lists, built once per chunk object (as the eager path keeps them)
        if getattr(g, "lists", None) is None:
            fl = self.fl
            g.lists = torch.empty(fl.S * g.nC, dtype=torch.int32, device=fl.dev)
            g.list_counts = torch.empty(fl.S, dtype=torch.int32, device=fl.dev)
            K.mm_species_lists(g.node_spec, g.nC, fl.S, g.lists, g.nC, g.list_counts, stream())
        # the node set (nodes, species, lists) changes only with the chunk object or an in-place write to one of its
        # tensors: MD keeps its chunk objects until a neighbour-list rebuild, so most calls load edges only.  The
        # slot holds references to the tensors it copied (so that they stay the same objects) and their versions.
        src = (g.nodes, g.node_spec, g.lists, g.list_counts)
        key = tuple(t._version for t in src)
        same = s.node_src is not None and all(a is b for a, b in zip(s.node_src, src)) and s.node_key == key
        if not same:
            s.nodes[:n].copy_(g.nodes)
            s.nodes[n:].fill_(self.sink)
            s.node_spec[:n].copy_(g.node_spec)
            s.node_spec[n:].fill_(0)
            s.lists.copy_(g.lists)
            s.list_counts.copy_(g.list_counts)
            s.n_nodes_dev.fill_(n)
            s.node_src, s.node_key = src, key
        s.rowptr.copy_(g.rowptr)
        s.ls[:nE].copy_(g.ls)
        # edges beyond nE are read by no kernel (the edge kernels stop at the device count rowptr[nC], the
        # convolutions at each receiver's CSR range); they are given harmless values at the slot's first load and
        # otherwise keep those of an earlier load, which are valid indices as well
        first = not s.loaded
        if self.mode == "rij":
            s.rij[:nE].copy_(g.rij)
            s.pair_i[:nE].copy_(g.pair_i)                   # global receivers, as the eager chunk has them
            if first:
                s.ls[nE:].fill_(0)
                s.rij[nE:].copy_(self.pad_rij.expand(self.e_cap - nE, 3))
                s.pair_i[nE:].fill_(s.a)
        else:
            s.recv_local[:nE].copy_(g.recv_local)
            if first:
                s.ls[nE:].fill_(self.n_cap - 1)             # a pad node: its position is the sink row
                s.recv_local[nE:].fill_(0)
        s.loaded = True
        if getattr(self.fl, "deterministic", False):   # pad edges are in no sender's range; pad nodes get empty ranges
            from .fast_layers import sender_csr
            g.sender_rowptr = None
            rp, perm = sender_csr(g)
            s.sender_rowptr[:n + 1].copy_(rp)
            s.sender_rowptr[n + 1:].fill_(nE)
            s.sender_perm[:nE].copy_(perm)
        s.nE, s.e0 = nE, g.e0

    def check(self, s):
        """Host-side check of a loaded slot: every index a captured kernel dereferences lies in its buffer
        (receivers of the chunk, chunk nodes, atom rows or the sink row, a monotone CSR inside the edge capacity).
        Raises ValueError; run before a slot's first eager run and capture (one device-to-host copy)."""
        nC, n_cap, e_cap = self.C, self.n_cap, self.e_cap
        rp = s.rowptr.cpu()
        if int(rp[0]) != 0 or int(rp[-1]) > e_cap or bool((rp[1:] < rp[:-1]).any()):
            raise ValueError("slot CSR is not monotone inside the edge capacity")
        recv = (s.pair_i.cpu().long() - s.a) if self.mode == "rij" else s.recv_local.cpu().long()
        if bool((recv < 0).any()) or bool((recv >= nC).any()):
            raise ValueError(f"slot {s.j}: edge receivers outside the chunk [0, {nC})")
        ls = s.ls.cpu().long()
        if bool((ls < 0).any()) or bool((ls >= n_cap).any()):
            raise ValueError(f"slot {s.j}: local senders outside [0, {n_cap})")
        nodes = s.nodes.cpu().long()
        if bool((nodes < 0).any()) or bool((nodes > self.sink).any()):
            raise ValueError(f"slot {s.j}: node rows outside [0, {self.sink}]")
        if s.b > self.nt_cap:
            raise ValueError(f"slot {s.j}: receivers [{s.a}, {s.b}) beyond the atom capacity {self.nt_cap}")

    def begin(self, graphs):
        """Loads the topology of every full chunk of this call into its slot; slots seen for the first time are
        captured (with this call's topology loaded)."""
        for g in graphs:
            if g.nC != self.C:
                continue
            j = g.a // self.C
            s = self.slots.get(j)
            new = s is None
            if new:
                s = self.slots[j] = _Slot(self, j)
            self._load(s, g)
            if new:
                self.check(s)
                self._capture(s)

    def finish(self, graphs, PF):
        """PF[e0:e1] of every full chunk from its slot (pass B stores, pass C adds)."""
        for g in graphs:
            if g.nC == self.C:
                s = self.slots[g.a // self.C]
                PF[g.e0:g.e1].copy_(s.PF[:g.nE])

    # ------------------------------------------------------------------ captured bodies
    def _body_A(self, s):
        self.fl.pass_a(s.chunk(self), self.H1, self.cache())

    def _body_B(self, s):
        self.fl.pass_b(s.chunk(self), self.H1x, self.G1, s.PF, self.eat)

    def _body_C(self, s):
        g = s.chunk(self)
        if self.cache_layer1:
            self.fl.pass_c(g, self.G1r, s.PF, self.eat, self.H1x, self.cache())
        else:
            self.fl.pass_c(g, self.G1r, s.PF, self.eat)

    def _capture(self, s):
        """Captures the three bodies of slot s (one eager run of each first, on a side stream).  The eager runs
        write the shared buffers; begin() is called before any pass of the call, and the caller clears them."""
        fl = self.fl
        saved_ws, saved_timer = fl.ws, fl.ktimer
        fl.ws, fl.ktimer = self.ws, None
        try:
            fl.workspace(self.C, self.n_cap, self.e_cap)
            self.ws = fl.ws
            bodies = (("A", self._body_A), ("B", self._body_B), ("C", self._body_C))
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _, fn in bodies:
                    fn(s)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            graphs = {}
            for name, fn in bodies:
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, pool=self.pool):
                    fn(s)
                graphs[name] = gr
            torch.cuda.synchronize()
            s.graphs = graphs
            self.n_captured += 1
        finally:
            fl.ws, fl.ktimer = saved_ws, saved_timer

    # ------------------------------------------------------------------ replays
    def _replay(self, g, name):
        s = self.slots[g.a // self.C]
        if s.e0 != g.e0 or s.nE != g.nE:
            raise ValueError("chunk replayed without begin() for this call")
        s.graphs[name].replay()
        self.n_replays += 1

    def pass_a(self, g):
        """H1[a:b] and the layer-1 cache rows of the chunk."""
        self._replay(g, "A")

    def pass_b(self, g):
        """Reads H1x, adds into G1 and eat[a:b], stores the chunk's pair forces in its slot."""
        self._replay(g, "B")

    def pass_c(self, g):
        """Reads G1r (and H1x with the cache), adds into the slot's pair forces and eat[a:b]."""
        self._replay(g, "C")

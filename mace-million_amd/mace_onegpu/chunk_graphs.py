"""HIP-graph execution of full receiver chunks (MACE3P_GRAPHS=1), the MI355X counterpart of the reference's
_GraphExec / _prepare_graphs (mliap_threepass.py:58-152, 390-431).

The kernel sequence of each pass (A, B, C) of a FULL chunk (nC == chunk) is captured once into a HIP graph over
static buffers of fixed capacity -- n_cap chunk nodes, e_cap chunk edges, nt_cap atoms (local + ghost) -- and
replayed for every full chunk after its inputs are copied into the static buffers; outputs are read back from
static buffers.  The arithmetic is the eager path's (FastLayers.pass_a/b/c run on a static ChunkGraph), so the
results agree with the eager path up to the order of the fp32 atomic additions of the sender-feature gradient.

Padding: edges beyond the chunk's nE are outside every receiver's CSR range, so no convolution reads them; their
geometry is computed from harmless inputs (LAMMPS path: rij = (1.5 r_max, 0, 0), receiver 0; standalone path:
sender = a pad node).  Nodes beyond the chunk's n_nodes point at a sink row (index nt_cap) of the static H1x / G1
/ position buffers: H1x[sink] = 0, and the G1 scatter of pad rows lands in G1[sink], never in a real atom's row.
The tail chunk (nC < chunk) runs eagerly.  Buffers are cleared inside the graphs with fill kernels only.
"""
import torch

from ._lib import K, stream
from .receiver_chunk_mace import ChunkGraph

C = 128


def _align(x, a):
    return ((int(x) + a - 1) // a) * a


def capacities(n_max, e_max, nt, e_align=65536, margin=1.25):
    """(n_cap, e_cap, nt_cap) with the reference's headroom (mliap_threepass.py:418-421)."""
    return _align(int(n_max * margin) + 2, 1024), _align(int(e_max * margin), e_align), int(nt * margin) + 1024


class ChunkGraphExec:
    """Captured passes A/B/C of full chunks.  mode "rij": edge vectors come from LAMMPS' rij (pair_i global
    receiver); mode "pos": edge vectors are minimum images of positions (standalone System)."""

    def __init__(self, fl, chunk, n_cap, e_cap, nt_cap, mode, cache_layer1, box_host=None):
        if mode not in ("rij", "pos"):
            raise ValueError(mode)
        dev = fl.dev
        self.fl, self.C, self.n_cap, self.e_cap, self.nt_cap, self.mode = fl, int(chunk), n_cap, e_cap, nt_cap, mode
        self.cache_layer1 = bool(cache_layer1)
        self.sink = nt_cap
        D1 = 4 * C
        i32 = dict(dtype=torch.int32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        f64 = dict(dtype=torch.float64, device=dev)
        nC = self.C
        self.rowptr = torch.zeros(nC + 1, **i32)
        self.ls = torch.zeros(e_cap, **i32)
        self.nodes = torch.full((n_cap,), self.sink, **i32)
        self.node_spec = torch.zeros(n_cap, **i32)
        if mode == "rij":
            self.rij = torch.zeros(e_cap, 3, **f64)
            self.pair_i = torch.zeros(e_cap, **i32)
            self.pad_rij = torch.tensor([1.5 * fl.spec.r_max, 0.0, 0.0], **f64)
        else:
            self.recv_local = torch.zeros(e_cap, **i32)
            self.pos = torch.zeros(nt_cap + 1, 3, **f64)
            self.box_host = box_host
        self.h1 = torch.zeros(nC, D1, **f32)
        self.g1 = torch.zeros(nC, D1, **f32)
        self.M = torch.zeros(nC, 16 * C, **f32) if self.cache_layer1 else None
        self.rho = torch.zeros(nC, **f32) if self.cache_layer1 else None
        self.PF = torch.zeros(e_cap, 3, **f32)
        self.eat = torch.zeros(nC, **f64)
        self.H1x = torch.zeros(nt_cap + 1, D1, **f32)      # row nt_cap: sink of the pad nodes (stays 0)
        self.G1 = torch.zeros(nt_cap + 1, D1, **f32)
        self.lists = torch.zeros(fl.S * nC, **i32)
        self.list_counts = torch.zeros(fl.S, **i32)
        self.ws = None
        self.graphs = None
        self.n_replays = 0

    # ------------------------------------------------------------------ static chunk seen by the captured passes
    def _static_chunk(self):
        g = ChunkGraph()
        g.a, g.b, g.e0, g.e1 = 0, self.C, 0, self.e_cap
        g.nC, g.nE, g.n_nodes = self.C, self.e_cap, self.n_cap
        g.rowptr, g.ls, g.nodes, g.node_spec = self.rowptr, self.ls, self.nodes, self.node_spec
        g.lists, g.list_counts, g.recompute_lists = self.lists, self.list_counts, True
        if self.mode == "rij":
            g.rij, g.pair_i = self.rij, self.pair_i
        else:
            g.pos, g.box_host, g.recv_local = self.pos, self.box_host, self.recv_local
        return g

    def fits(self, n_nodes, nE, nt):
        return n_nodes <= self.n_cap - 1 and nE <= self.e_cap and nt <= self.nt_cap

    def load(self, g):
        """Copies the chunk's inputs into the static buffers (padding as described in the module docstring)."""
        n, nE = g.n_nodes, g.nE
        if g.nC != self.C or not self.fits(n, nE, 0):
            raise ValueError(f"chunk ({g.nC} receivers, {n} nodes, {nE} edges) does not fit the captured "
                             f"capacities ({self.C}, {self.n_cap - 1}, {self.e_cap})")
        self.nodes[:n].copy_(g.nodes)
        self.nodes[n:].fill_(self.sink)
        self.node_spec[:n].copy_(g.node_spec)
        self.node_spec[n:].fill_(0)
        self.rowptr.copy_(g.rowptr)
        self.ls[:nE].copy_(g.ls)
        if self.mode == "rij":
            self.ls[nE:].fill_(0)
            self.rij[:nE].copy_(g.rij)
            self.rij[nE:].copy_(self.pad_rij.expand(self.e_cap - nE, 3))
            torch.sub(g.pair_i, g.a, out=self.pair_i[:nE])
            self.pair_i[nE:].fill_(0)
        else:
            self.ls[nE:].fill_(self.n_cap - 1)              # a pad node: its position is the sink row
            self.recv_local[:nE].copy_(g.recv_local)
            self.recv_local[nE:].fill_(0)

    def set_positions(self, pos):
        """Standalone mode: the positions of the current call (rows beyond them and the sink row are 0)."""
        n = pos.shape[0]
        if n > self.nt_cap:
            raise ValueError("more atoms than the captured capacity")
        self.pos[:n].copy_(pos)
        self.pos[n:].zero_()

    # ------------------------------------------------------------------ captured bodies
    def _cache(self):
        return dict(M=self.M, rho=self.rho) if self.cache_layer1 else None

    def _body_A(self):
        self.fl.pass_a(self._static_chunk(), self.h1, self._cache())

    def _body_B(self):
        K.mm_fill_f64(self.eat, self.C, 0.0, stream())
        self.fl.pass_b(self._static_chunk(), self.H1x, self.G1, self.PF, self.eat)

    def _body_C(self):
        K.mm_fill_f64(self.eat, self.C, 0.0, stream())
        K.mm_fill_f32(self.PF, self.e_cap * 3, 0.0, stream())
        if self.cache_layer1:
            self.fl.pass_c(self._static_chunk(), self.g1, self.PF, self.eat, self.h1, self._cache())
        else:
            self.fl.pass_c(self._static_chunk(), self.g1, self.PF, self.eat)

    def capture(self, g_first):
        """Captures the three bodies with the first full chunk loaded (one eager run of each body first)."""
        fl = self.fl
        saved_ws, saved_timer = fl.ws, fl.ktimer
        fl.ws, fl.ktimer = None, None
        try:
            fl.workspace(self.C, self.n_cap, self.e_cap)
            self.ws = fl.ws
            self.load(g_first)
            bodies = (("A", self._body_A), ("B", self._body_B), ("C", self._body_C))
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _, fn in bodies:
                    fn()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            pool = torch.cuda.graph_pool_handle()
            graphs = {}
            for name, fn in bodies:
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, pool=pool):
                    fn()
                graphs[name] = gr
            torch.cuda.synchronize()
            self.graphs = graphs
            self.G1.zero_()
        finally:
            fl.ws, fl.ktimer = saved_ws, saved_timer

    # ------------------------------------------------------------------ replays
    def pass_a(self, g, H1, cache):
        self.load(g)
        self.graphs["A"].replay()
        self.n_replays += 1
        H1[g.a:g.b].copy_(self.h1)
        if cache is not None and self.cache_layer1:
            cache["M"][g.a:g.b].copy_(self.M)
            cache["rho"][g.a:g.b].copy_(self.rho)

    def pass_b(self, g, PF, eat):
        """Layer-2 pass; reads self.H1x and scatters into self.G1 (the caller's H1x / G1 are their views)."""
        self.load(g)
        self.graphs["B"].replay()
        self.n_replays += 1
        PF[g.e0:g.e1].copy_(self.PF[:g.nE])
        eat[g.a:g.b] += self.eat

    def pass_c(self, g, G1r, PF, eat, H1=None, cache=None):
        self.load(g)
        self.g1.copy_(G1r[g.a:g.b])
        if self.cache_layer1:
            if cache is None or H1 is None:
                raise ValueError("this executor was captured with the layer-1 cache: pass H1 and the cache")
            self.h1.copy_(H1[g.a:g.b])
            self.M.copy_(cache["M"][g.a:g.b])
            self.rho.copy_(cache["rho"][g.a:g.b])
        self.graphs["C"].replay()
        self.n_replays += 1
        PF[g.e0:g.e1] += self.PF[:g.nE]
        eat[g.a:g.b] += self.eat

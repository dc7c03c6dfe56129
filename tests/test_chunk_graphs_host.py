"""Slot loading of the HIP-graph executor (chunk_graphs) on the CPU, without capturing: the topology a slot holds
is the one the captured kernels index, so every index must land inside its buffer.  Regression test for a slot
layout whose LAMMPS-path receivers were stored chunk-local while the static chunk also carries the chunk offset
(the geometry kernel subtracts it again: negative receiver rows); check() must reject such a slot before any
kernel runs."""
import types

import pytest
import torch

from mace_onegpu import chunk_graphs
from mace_onegpu.receiver_chunk_mace import ChunkGraph


def _stub_layers():
    return types.SimpleNamespace(dev="cpu", S=2, spec=types.SimpleNamespace(r_max=6.0))


def _chunks(mode, nC=8, n_chunks=3, seed=0):
    """Receiver-sorted pairs of n_chunks * nC atoms (each receiver 3..6 senders among all atoms), cut into chunks
    the way both callers cut them."""
    g0 = torch.Generator().manual_seed(seed)
    N = nC * n_chunks
    deg = torch.randint(3, 7, (N,), generator=g0)
    recv = torch.repeat_interleave(torch.arange(N), deg)
    send = torch.randint(0, N, (len(recv),), generator=g0)
    rp = torch.cat([torch.zeros(1, dtype=torch.long), torch.cumsum(deg, 0)])
    out = []
    for j in range(n_chunks):
        a, b = j * nC, (j + 1) * nC
        e0, e1 = int(rp[a]), int(rp[b])
        g = ChunkGraph()
        g.a, g.b, g.e0, g.e1, g.nC, g.nE = a, b, e0, e1, nC, e1 - e0
        outside = torch.unique(send[e0:e1][(send[e0:e1] < a) | (send[e0:e1] >= b)])
        g.nodes = torch.cat([torch.arange(a, b), outside]).int()
        g.n_nodes = len(g.nodes)
        loc = {int(v): i for i, v in enumerate(g.nodes)}
        g.ls = torch.tensor([loc[int(v)] for v in send[e0:e1]], dtype=torch.int32)
        g.node_spec = (g.nodes % 2).int()
        # per-species receiver lists as mm_species_lists builds them (stable partition, stride nC); a slot load
        # copies them (the production callers build them on the GPU, once per chunk object)
        spec_r = g.node_spec[:nC].long()
        g.lists = torch.zeros(2 * nC, dtype=torch.int32)
        g.list_counts = torch.zeros(2, dtype=torch.int32)
        for sp in range(2):
            idx = torch.nonzero(spec_r == sp).squeeze(1).int()
            g.lists[sp * nC: sp * nC + len(idx)] = idx
            g.list_counts[sp] = len(idx)
        g.rowptr = (rp[a:b + 1] - e0).int()
        if mode == "rij":
            g.pair_i = recv[e0:e1].int()
            g.rij = torch.randn(e1 - e0, 3, dtype=torch.float64, generator=g0)
        else:
            g.recv_local = (recv[e0:e1] - a).int()
        out.append(g)
    return out


@pytest.mark.parametrize("mode", ["rij", "pos"])
def test_loaded_slots_index_inside_their_buffers(mode):
    gs = _chunks(mode)
    n_cap, e_cap, nt_cap = chunk_graphs.capacities(max(g.n_nodes for g in gs), max(g.nE for g in gs), 24,
                                                   e_align=64)
    ex = chunk_graphs.ChunkGraphExec(_stub_layers(), 8, n_cap, e_cap, nt_cap, mode, True, exchange=(mode == "rij"))
    for g in gs:
        s = ex.slots[g.a // 8] = chunk_graphs._Slot(ex, g.a // 8)
        ex._load(s, g)
        ex.check(s)
        assert torch.equal(s.lists, g.lists) and torch.equal(s.list_counts, g.list_counts)
        if mode == "rij":     # what the kernel computes: pair_i - a, for real and pad edges
            recv = s.pair_i.long() - s.a
            assert torch.equal(recv[:g.nE], g.pair_i.long() - g.a) and bool((recv[g.nE:] == 0).all())
        assert torch.equal(s.nodes[:g.n_nodes], g.nodes) and bool((s.nodes[g.n_nodes:] == ex.sink).all())
    # the executor's shared buffers hold every chunk's rows and the sink row
    assert ex.H1x.shape[0] == nt_cap + 1 and ex.G1.shape[0] == nt_cap + 1 and ex.eat.shape[0] >= 24


def test_check_rejects_chunk_local_receivers():
    gs = _chunks("rij")
    n_cap, e_cap, nt_cap = chunk_graphs.capacities(max(g.n_nodes for g in gs), max(g.nE for g in gs), 24,
                                                   e_align=64)
    ex = chunk_graphs.ChunkGraphExec(_stub_layers(), 8, n_cap, e_cap, nt_cap, "rij", True, exchange=True)
    g = gs[2]
    s = chunk_graphs._Slot(ex, 2)
    ex._load(s, g)
    s.pair_i[:g.nE] -= g.a                      # the faulty layout: receivers already made chunk-local
    with pytest.raises(ValueError, match="receivers outside"):
        ex.check(s)


def test_load_rejects_a_chunk_of_another_slot():
    gs = _chunks("pos")
    n_cap, e_cap, nt_cap = chunk_graphs.capacities(max(g.n_nodes for g in gs), max(g.nE for g in gs), 24,
                                                   e_align=64)
    ex = chunk_graphs.ChunkGraphExec(_stub_layers(), 8, n_cap, e_cap, nt_cap, "pos", False)
    s = chunk_graphs._Slot(ex, 0)
    with pytest.raises(ValueError, match="slot of receiver"):
        ex._load(s, gs[1])


def test_reload_copies_the_node_set_only_when_it_changed():
    """A slot reloads edges every call but copies nodes / species / lists only for another chunk object or after an
    in-place write to one of its tensors (MD keeps its chunk objects between neighbour-list rebuilds); a reload with
    fewer edges keeps every index inside its buffer."""
    gs = _chunks("pos")
    n_cap, e_cap, nt_cap = chunk_graphs.capacities(max(g.n_nodes for g in gs), max(g.nE for g in gs), 24,
                                                   e_align=64)
    ex = chunk_graphs.ChunkGraphExec(_stub_layers(), 8, n_cap, e_cap, nt_cap, "pos", False)
    g = gs[1]
    s = ex.slots[1] = chunk_graphs._Slot(ex, 1)
    ex._load(s, g)
    s.nodes[0] = -5                               # marks the slot's copy
    ex._load(s, g)                                # same objects, same versions: no node copy
    assert int(s.nodes[0]) == -5
    g.nodes[1] = g.nodes[1]                       # an in-place write bumps the tensor's version
    ex._load(s, g)
    assert torch.equal(s.nodes[:g.n_nodes], g.nodes)
    # a new chunk object for the same receivers, with fewer edges: nodes reloaded, edges checked
    h = _chunks("pos", seed=3)[1]
    h.nE = h.nE - 5
    h.ls, h.recv_local = h.ls[:h.nE], h.recv_local[:h.nE]
    h.rowptr = torch.clamp(h.rowptr, max=h.nE)
    ex._load(s, h)
    assert torch.equal(s.nodes[:h.n_nodes], h.nodes) and bool((s.nodes[h.n_nodes:] == ex.sink).all())
    assert torch.equal(s.ls[:h.nE], h.ls)
    ex.check(s)


def test_capacities_headroom():
    """25 % headroom on chunk nodes and edges (aligned), and on the atom rows unless nt_margin says otherwise (a
    standalone system keeps its atom count)."""
    from mace_onegpu import chunk_graphs
    n_cap, e_cap, nt_cap = chunk_graphs.capacities(1000, 100000, 5000, 65536, 1.25)
    assert n_cap == 2048 and e_cap == 131072 and nt_cap == 6250 + 1024
    assert chunk_graphs.capacities(1000, 100000, 5000, 65536, 1.25, nt_margin=1.0) == (2048, 131072, 6024)

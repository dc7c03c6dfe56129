"""Host-side index checks of the eager path (CPU only): check_chunk on one chunk's index arrays, and the pair
grouping of the ML-IAP boundary (receiver CSR, inverse permutation, range check of pair_i / pair_j)."""
import numpy as np
import pytest
import torch

from mace_onegpu.mliap_threepass import _PairBatch
from mace_onegpu.receiver_chunk_mace import check_chunk, chunk_topology, make_chunk

CPU = torch.device("cpu")


def _chunk(rij_mode=True):
    """Chunk [4, 8) of a 12-atom ring-like pair list (every atom sends to its 3 successors)."""
    N = 12
    recv = np.repeat(np.arange(N), 3)
    send = (recv + np.tile([1, 2, 3], N)) % N
    pj = torch.as_tensor(send, dtype=torch.int32)
    rp = torch.as_tensor(np.arange(N + 1) * 3, dtype=torch.int64)
    loc = torch.full((N,), -1, dtype=torch.int32)
    flag = torch.zeros(N, dtype=torch.bool)
    a, b = 4, 8
    e0, e1 = int(rp[a]), int(rp[b])
    nodes, ls = chunk_topology(a, b, e0, e1, pj, loc, flag)
    g = make_chunk(a, b, e0, e1, nodes, ls, rp, torch.zeros(N, dtype=torch.int32))
    if rij_mode:
        g.rij = torch.ones(e1 - e0, 3, dtype=torch.float64)
        g.pair_i = torch.as_tensor(recv[e0:e1], dtype=torch.int32)
    else:
        g.recv_local = torch.as_tensor(recv[e0:e1] - a, dtype=torch.int32)
    return g, N


@pytest.mark.parametrize("rij_mode", [True, False])
def test_check_chunk_accepts_a_valid_chunk(rij_mode):
    g, N = _chunk(rij_mode)
    assert g.nodes[:4].tolist() == [4, 5, 6, 7] and g.nodes[4:].tolist() == [8, 9, 10]
    check_chunk(g, N, 1)


@pytest.mark.parametrize("bad,match", [
    ("ls_high", "local senders"), ("ls_neg", "local senders"), ("node_high", "node rows"),
    ("node_order", "receivers a..b-1"), ("rowptr", "monotone"), ("species", "species"),
    ("recv", "edge receivers"), ("recv_local", "edge receivers")])
def test_check_chunk_names_the_bad_array(bad, match):
    g, N = _chunk(rij_mode=bad != "recv_local")
    if bad == "ls_high":
        g.ls = g.ls.clone()
        g.ls[5] = g.n_nodes
    elif bad == "ls_neg":
        g.ls = g.ls.clone()
        g.ls[0] = -1
    elif bad == "node_high":
        g.nodes = g.nodes.clone()
        g.nodes[-1] = N
    elif bad == "node_order":
        g.nodes = g.nodes.clone()
        g.nodes[[0, 1]] = g.nodes[[1, 0]]
    elif bad == "rowptr":
        g.rowptr = g.rowptr.clone()
        g.rowptr[2] = g.rowptr[1] - 1
    elif bad == "species":
        g.node_spec = g.node_spec.clone()
        g.node_spec[3] = -1                       # a species missing from the model's present columns
    elif bad == "recv":
        g.pair_i = g.pair_i.clone()
        g.pair_i[0] = g.a - 1                     # global receiver outside the chunk (chunk-local -1)
    else:
        g.recv_local = g.recv_local.clone()
        g.recv_local[-1] = g.nC
    with pytest.raises(ValueError, match=match):
        check_chunk(g, N, 1)


class _Data:
    def __init__(self, pi, pj):
        self.pair_i, self.pair_j = torch.as_tensor(pi, dtype=torch.int32), torch.as_tensor(pj, dtype=torch.int32)
        self.rij = torch.randn(len(pi), 3, dtype=torch.float64, generator=torch.Generator().manual_seed(1))


def test_pair_batch_groups_by_receiver_and_restores_the_order():
    pi = [3, 0, 2, 0, 3, 1, 3]
    pj = [5, 1, 6, 2, 0, 4, 1]
    d = _Data(pi, pj)
    b = _PairBatch(d, 4, 7, CPU, check=True)
    assert b.pair_i.tolist() == [0, 0, 1, 2, 3, 3, 3]
    assert b.pair_j.tolist() == [1, 2, 4, 6, 5, 0, 1]               # stable within a receiver
    assert b.rowptr.tolist() == [0, 2, 3, 4, 7]
    assert torch.equal(b.rij, d.rij[b.perm])
    back = b.restore(b.rij)
    assert torch.equal(back, d.rij)
    s = _PairBatch(_Data(sorted(pi), pj), 4, 7, CPU, check=True)
    assert s.perm is None and s.restore(s.rij) is s.rij


@pytest.mark.parametrize("pi,pj,nl,nt", [([0, 1, 4], [1, 0, 0], 4, 6), ([0, 1, 2], [1, 6, 0], 4, 6),
                                          ([0, 1, 2], [1, -1, 0], 4, 6)])
def test_pair_batch_range_check(pi, pj, nl, nt):
    with pytest.raises(ValueError, match="pair_i"):
        _PairBatch(_Data(pi, pj), nl, nt, CPU, check=True)


def test_pair_batch_rejects_a_ghost_receiver_without_the_check():
    with pytest.raises(ValueError, match="not a local atom"):
        _PairBatch(_Data([0, 1, 4], [1, 0, 0]), 4, 6, CPU, check=False)

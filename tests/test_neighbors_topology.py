"""Oracle neighbour list and chunk topology against the golden vectors written from the reference's own
System / _topology_all (tests/golden/make_golden.py) and against brute-force enumeration (CPU)."""
import os

import numpy as np
import pytest

from oracle import neighbors, topology

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "neighbors.npz"))
CASES = sorted({k.split("__")[0] for k in G.files})


def golden(name):
    return {k.split("__")[1]: G[k] for k in G.files if k.startswith(name + "__")}


@pytest.mark.parametrize("name", CASES)
def test_oracle_neighbors_bit_exact_with_reference(name):
    g = golden(name)
    s = neighbors.SystemRef(g["pos"], g["box"], g["spidx"], 6.0)
    NN, rp, send = s.build_neighbors()
    assert np.array_equal(s.perm, g["perm"])
    assert np.array_equal(s.pos, g["pos_sorted"])
    assert np.array_equal(NN, g["NN"])
    assert np.array_equal(send, g["send"])


@pytest.mark.parametrize("name", ["water192_ref", "random700_wrap"])
def test_oracle_neighbors_equal_brute_force_set(name):
    g = golden(name)
    s = neighbors.SystemRef(g["pos"], g["box"], g["spidx"], 6.0)
    NN, rp, send = s.build_neighbors()
    recv = np.repeat(np.arange(s.N), NN)
    got = set(zip(recv.tolist(), send.tolist()))
    assert got == neighbors.brute_force_pairs(s.pos, s.box, 6.0)


@pytest.mark.parametrize("name", CASES)
def test_c_oracle_neighbors_bit_exact_with_reference(name):
    """The plain-C restatement (oracle/nlist_c) reproduces the reference's golden neighbour lists."""
    from oracle import nlist_c
    g = golden(name)
    perm, pos_sorted, NN, rowptr, send = nlist_c.neighbor_list(g["pos"], g["box"], 6.0)
    assert np.array_equal(perm, g["perm"])
    assert np.array_equal(pos_sorted, g["pos_sorted"])
    assert np.array_equal(NN, g["NN"])
    assert np.array_equal(send, g["send"])


def test_c_oracle_equals_numpy_oracle_on_a_larger_box():
    """C and numpy restatements agree on a 3,000-atom random box with ties at the cutoff and atoms on cell faces."""
    from oracle import nlist_c
    rng = np.random.default_rng(11)
    box = np.array([21.0, 19.5, 24.25])
    pos = rng.uniform(-5.0, 30.0, size=(3000, 3))
    pos[:40] = np.round(pos[:40])                       # lattice points: exact 6.0 A separations exist
    pos[40:60, 0] = 6.5                                 # on a cell face (box / ncell = 7.0 ... 6.5)
    s = neighbors.SystemRef(pos, box, np.zeros(3000, int), 6.0)
    NN0, rp0, send0 = s.build_neighbors()
    perm, pos_sorted, NN, rowptr, send = nlist_c.neighbor_list(pos, box, 6.0)
    assert np.array_equal(perm, s.perm) and np.array_equal(pos_sorted, s.pos)
    assert np.array_equal(NN, NN0) and np.array_equal(rowptr, rp0) and np.array_equal(send, send0)


T = np.load(os.path.join(HERE, "golden", "topology.npz"))


@pytest.mark.parametrize("ci", [0, 1, 2])
def test_topology_matches_reference(ci):
    pi, pj = T[f"c{ci}__pi"], T[f"c{ci}__pj"]
    nl, nt, C = (int(x) for x in T[f"c{ci}__meta"])
    rp = np.searchsorted(pi, np.arange(nl + 1))
    nodes_all, ls_all = [], []
    for a in range(0, nl, C):
        b = min(a + C, nl)
        nodes, ls = topology.topology(a, b, pi[rp[a]:rp[b]], pj[rp[a]:rp[b]])
        assert np.array_equal(nodes[ls], pj[rp[a]:rp[b]])                 # invariants of test_topology.py:72-73
        assert np.array_equal(nodes[pi[rp[a]:rp[b]] - a], pi[rp[a]:rp[b]])
        nodes_all.append(nodes)
        ls_all.append(ls)
    assert np.array_equal(np.concatenate(nodes_all), T[f"c{ci}__nodes"])
    assert np.array_equal(np.concatenate(ls_all), T[f"c{ci}__ls"])


@pytest.mark.parametrize("ci", [0, 1, 2])
def test_product_chunk_topology_matches_reference(ci):
    """The product's chunk builder (receiver_chunk_mace.chunk_topology, as the standalone, ML-IAP and MD paths
    call it) reproduces the reference's golden nodes and local sender indices (plain torch, run here on the
    CPU), and restores its scratch arrays."""
    import torch
    from mace_onegpu.receiver_chunk_mace import chunk_topology
    pi, pj = T[f"c{ci}__pi"], T[f"c{ci}__pj"]
    nl, nt, C = (int(x) for x in T[f"c{ci}__meta"])
    rp = np.searchsorted(pi, np.arange(nl + 1))
    pj_t = torch.as_tensor(pj.astype(np.int32))
    loc = torch.full((nt,), -1, dtype=torch.int32)
    flag = torch.zeros(nt, dtype=torch.bool)
    topo = [chunk_topology(a, min(a + C, nl), int(rp[a]), int(rp[min(a + C, nl)]), pj_t, loc, flag)
            for a in range(0, nl, C)]
    assert np.array_equal(torch.cat([n for n, _ in topo]).numpy(), T[f"c{ci}__nodes"])
    assert np.array_equal(torch.cat([l for _, l in topo]).numpy(), T[f"c{ci}__ls"])
    assert bool((loc == -1).all()) and not bool(flag.any())


def _reverse_by_sort(rp, send):
    """The reverse-pair map by sorting the pairs by (receiver, sender) (numpy)."""
    N = len(rp) - 1
    recv = np.repeat(np.arange(N, dtype=np.int64), np.diff(rp))
    key = recv * N + send
    order = np.argsort(key, kind="stable")
    pos = np.searchsorted(key[order], send.astype(np.int64) * N + recv)
    return order[pos]


def _random_symmetric(N, p, seed):
    """A symmetric pair list with every row in a random order (rows of 0 to about p N pairs)."""
    rng = np.random.default_rng(seed)
    adj = np.triu(rng.random((N, N)) < p, 1)
    adj |= adj.T
    rows = [rng.permutation(np.flatnonzero(adj[i])) for i in range(N)]
    rp = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    return rp, np.concatenate(rows).astype(np.int32)


def _random_pairs(nl, nt, kmax, seed, self_pairs):
    """Receivers 0..nl-1 in order with random degrees 0..kmax (one receiver without pairs when nl > 3), senders
    anywhere in 0..nt-1 (nt > nl: ghosts); without self_pairs a sender equal to its receiver is moved to the next
    atom."""
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, kmax + 1, size=nl)
    if nl > 3:
        deg[rng.integers(0, nl)] = 0
    pi = np.repeat(np.arange(nl), deg).astype(np.int32)
    pj = rng.integers(0, nt, size=pi.size).astype(np.int32)
    if not self_pairs:
        same = pj == pi
        pj[same] = (pj[same] + 1) % nt
    return pi, pj


# the pair-list shapes of the reference's tests/test_topology.py:40-51 (nl, nt, chunk, kmax, seed, self pairs)
TOPO_CASES = [(1000, 1300, 128, 12, 0, False), (1000, 1300, 1000, 12, 1, False), (1000, 1000, 4096, 12, 2, False),
              (1000, 1000, 100, 12, 3, False), (777, 901, 64, 30, 4, False), (5, 9, 2, 3, 5, False),
              (1, 4, 16, 3, 6, False), (3000, 3400, 256, 8, 7, True), (20000, 23000, 2048, 20, 8, False)]


@pytest.mark.parametrize("nl,nt,C,kmax,seed,self_pairs", TOPO_CASES)
def test_product_chunk_topology_on_random_pair_lists(nl, nt, C, kmax, seed, self_pairs):
    """The product's chunk builder equals the oracle's topology (pinned on the golden vectors above) on the
    reference's pair-list shapes: ghosts, a partial last chunk, one chunk with or without ghosts, chunks larger
    than the receiver count, a single local atom, pairs i == i, receivers without pairs."""
    import torch
    from mace_onegpu.receiver_chunk_mace import chunk_topology
    pi, pj = _random_pairs(nl, nt, kmax, seed, self_pairs)
    rp = np.searchsorted(pi, np.arange(nl + 1))
    pj_t = torch.as_tensor(pj)
    loc = torch.full((nt,), -1, dtype=torch.int32)
    flag = torch.zeros(nt, dtype=torch.bool)
    for a in range(0, nl, C):
        b = min(a + C, nl)
        e0, e1 = int(rp[a]), int(rp[b])
        nodes, ls = chunk_topology(a, b, e0, e1, pj_t, loc, flag)
        nodes_o, ls_o = topology.topology(a, b, pi[e0:e1], pj[e0:e1])
        assert nodes.dtype == torch.int32 and ls.dtype == torch.int32
        assert np.array_equal(nodes.numpy(), nodes_o) and np.array_equal(ls.numpy(), ls_o), (a, b)
        n = nodes.numpy().astype(np.int64)
        assert np.array_equal(n[ls.numpy()], pj[e0:e1]) and np.array_equal(n[pi[e0:e1] - a], pi[e0:e1])
        assert np.array_equal(n[:b - a], np.arange(a, b))                      # receivers first
        out = n[b - a:]
        assert np.all(np.diff(out) > 0) and not np.any((out >= a) & (out < b))  # then outside senders, ascending
    assert bool((loc == -1).all()) and not bool(flag.any())


@pytest.mark.gpu
def test_reverse_pairs_map():
    """reverse_pairs (mm_nl_reverse, the MD force sum's reverse-pair map) maps (i, j) to (j, i), equal to the map
    found by sorting: on the cell list of the golden water box (rows of about 90 pairs in candidate order), on a
    complete graph (rows of 599 pairs: three 256-candidate rounds, ten 64-pair blocks) and on a random graph with
    rows of 0 to 400 pairs; a list without a reverse pair raises."""
    import torch
    from mace_onegpu.md import reverse_pairs

    assert torch.cuda.is_available(), "GPU test without a GPU"
    g = golden("water648_cells")
    s = neighbors.SystemRef(g["pos"], g["box"], g["spidx"], 6.0)
    NN, rp, send = s.build_neighbors()
    n = 600
    full = np.array([np.random.default_rng(i).permutation(np.delete(np.arange(n), i)) for i in range(n)]).ravel()
    cases = [(np.asarray(rp, np.int64), np.asarray(send, np.int32)),
             (np.arange(n + 1, dtype=np.int64) * (n - 1), full.astype(np.int32)),
             _random_symmetric(1000, 0.4, 3), _random_symmetric(700, 0.02, 4)]

    class V:
        pass
    for rp_c, send_c in cases:
        v = V()
        v.N = len(rp_c) - 1
        v.rowptr = torch.as_tensor(rp_c, device="cuda")
        v.send = torch.as_tensor(send_c, device="cuda")
        rev = reverse_pairs(v).cpu().numpy().astype(np.int64)
        assert np.array_equal(rev, _reverse_by_sort(rp_c, send_c)), v.N
        assert np.array_equal(rev[rev], np.arange(len(send_c)))
    v = V()
    v.N, v.rowptr = 2, torch.tensor([0, 1, 1], device="cuda")
    v.send = torch.tensor([1], dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="not symmetric"):
        reverse_pairs(v)


def test_reverse_map_by_sort_is_an_involution():
    """The sorting restatement that the GPU map is checked against: (i, j) -> (j, i) on the golden water box."""
    g = golden("water648_cells")
    s = neighbors.SystemRef(g["pos"], g["box"], g["spidx"], 6.0)
    NN, rp, send = s.build_neighbors()
    rev = _reverse_by_sort(np.asarray(rp, np.int64), np.asarray(send, np.int64))
    recv = np.repeat(np.arange(s.N), NN)
    assert np.array_equal(rev[rev], np.arange(len(send)))
    assert np.array_equal(recv[rev], send) and np.array_equal(np.asarray(send)[rev], recv)

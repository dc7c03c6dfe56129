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

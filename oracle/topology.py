"""numpy restatement of the per-chunk local topology (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Restates ThreePassMLIAP._topology (mliap_threepass.py:288-310), which LocalGraph (receiver_chunk_mace.py:175-193)
computes the same way: for the receiver chunk [a, b) with CSR edge range [e0, e1) the local node list is the
receivers a..b-1 followed by the senders outside [a, b) in ascending order, and every edge's sender gets its
position in that list.  The receiver's local index is its global index minus a.
Pinned by: the invariants of the reference test tests/test_topology.py:67-74 (nodes[ls] == pj,
nodes[pi - a] == pi, receivers first, outside senders ascending and unique) and by golden vectors written by
importing the reference's _topology_all.
"""
import numpy as np


def topology(a, b, pi, pj):
    """pi, pj: receivers / senders of the chunk's edges (int). Returns (nodes int32, ls int32)."""
    pj = np.asarray(pj, dtype=np.int64)
    outside = np.unique(pj[(pj < a) | (pj >= b)])
    nodes = np.concatenate([np.arange(a, b, dtype=np.int64), outside]).astype(np.int32)
    loc = {int(g): k for k, g in enumerate(nodes)}
    ls = np.array([loc[int(s)] for s in pj], dtype=np.int32)
    return nodes, ls

"""Writes the golden neighbour-list and topology vectors of tests/golden/*.npz from the REFERENCE's own code.

Run in the build container only (needs /root/reference, read-only; torch + numpy):
    python tests/golden/make_golden.py
Imports only the torch/numpy functions that nothing else pins: receiver_chunk_mace.System
(wrap, Morton order, build_neighbors: edge order, perm tie-breaks, fp64 boundary cases) and
mliap_threepass.ThreePassMLIAP._topology_all (local index assignment).  Nothing from the reference is copied:
the .npz files hold inputs and outputs only.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
sys.path.insert(0, REF)

from mace_onegpu import receiver_chunk_mace as ref_rc  # noqa: E402  (the reference package, first on sys.path)
from mace_onegpu.mliap_threepass import ThreePassMLIAP as RefTP  # noqa: E402

R_MAX = 6.0


def _build_generator():
    """The build's systems.py, loaded by path (its package name is the same as the reference's)."""
    import importlib.util
    path = os.path.join(HERE, "..", "..", "mace-million_amd", "mace_onegpu", "systems.py")
    spec = importlib.util.spec_from_file_location("_build_systems", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def read_lammps_data(path):
    """Positions, box and types of examples/data/water64_1x1x1_N192.data (atomic style)."""
    lines = open(path).read().splitlines()
    box = []
    for ln in lines:
        if ln.strip().endswith("xlo xhi") or ln.strip().endswith("ylo yhi") or ln.strip().endswith("zlo zhi"):
            lo, hi = ln.split()[:2]
            box.append(float(hi) - float(lo))
    k = next(i for i, ln in enumerate(lines) if ln.startswith("Atoms"))
    rows = [ln.split() for ln in lines[k + 1:] if ln.strip()]
    rows = [r for r in rows if len(r) >= 5 and r[0].isdigit()]
    rows.sort(key=lambda r: int(r[0]))
    typ = np.array([int(r[1]) for r in rows])
    pos = np.array([[float(r[2]), float(r[3]), float(r[4])] for r in rows])
    Z = np.where(typ == 1, 8, 1)
    return pos, np.array(box), Z


def cases():
    out = {}
    pos, box, Z = read_lammps_data(os.path.join(REF, "examples", "data", "water64_1x1x1_N192.data"))
    out["water192_ref"] = (pos, box, Z - 1)
    rng = np.random.default_rng(7)
    # 216-molecule water (box 18.6 A -> 3 cells: the cell-list path) from the build's generator
    water_box = _build_generator().water_box     # the build's own input generator (inputs only)
    p, b, Zw = water_box(216, seed=3)
    out["water648_cells"] = (p, b, Zw - 1)
    # exact-distance ties: simple cubic lattices where (k, 0, 0) * a == r_max exactly, with sub-ulp jitter
    a = 2.0
    g = np.stack(np.meshgrid(*[np.arange(12)] * 3, indexing="ij"), -1).reshape(-1, 3) * a
    g = g + rng.choice([0.0, 1e-15, -1e-15, 4e-15], size=g.shape)
    out["sc1728_ties"] = (g, np.array([24.0, 24.0, 24.0]), np.zeros(len(g), dtype=np.int64))
    # negative and out-of-box coordinates (wrap), non-cubic box
    q = rng.uniform(-30, 60, size=(700, 3))
    out["random700_wrap"] = (q, np.array([19.0, 25.5, 31.25]), rng.integers(0, 4, 700))
    return out


def main():
    res = {}
    for name, (pos, box, sp) in cases().items():
        sysm = ref_rc.System(torch.tensor(pos, dtype=torch.float64), box, torch.tensor(sp, dtype=torch.int16),
                             R_MAX, "cpu")
        sysm.build_neighbors()
        NN = sysm.NN.numpy().astype(np.int32)
        NL = sysm.NL.numpy()
        send = np.concatenate([NL[i, :NN[i]] for i in range(len(NN))]).astype(np.int32)
        res[name] = dict(pos=pos, box=np.asarray(box, dtype=np.float64), spidx=np.asarray(sp, dtype=np.int64),
                         perm=sysm.perm.numpy().astype(np.int64), pos_sorted=sysm.pos.numpy(), NN=NN, send=send)
        print(f"{name}: N={len(NN)} edges={len(send)} ncell={sysm.ncell.tolist()}")
    np.savez_compressed(os.path.join(HERE, "neighbors.npz"),
                        **{f"{c}__{k}": v for c, d in res.items() for k, v in d.items()})
    # topology of the batched build, with ghosts and a partial tail chunk
    rng = np.random.default_rng(11)
    topo = {}
    for ci, (nl, nt, C, kmax) in enumerate([(1000, 1300, 128, 12), (777, 901, 64, 30), (3000, 3400, 1024, 8)]):
        deg = rng.integers(0, kmax + 1, size=nl)
        deg[rng.integers(0, nl)] = 0
        pi = np.repeat(np.arange(nl, dtype=np.int32), deg)
        pj = rng.integers(0, nt, size=pi.size).astype(np.int32)
        bad = pj == pi
        pj[bad] = (pj[bad] + 1) % nt
        o = RefTP.__new__(RefTP)
        o._dev = torch.device("cpu")
        o.chunk = C
        o._loc = torch.full((nt,), -1, dtype=torch.int32)
        o._flag = None
        rp = torch.searchsorted(torch.as_tensor(pi), torch.arange(nl + 1, dtype=torch.int32)).numpy()
        bounds = [(a, min(a + C, nl)) for a in range(0, nl, C)]
        got = o._topology_all(bounds, rp, torch.as_tensor(pi), torch.as_tensor(pj), nl, nt)
        nodes = np.concatenate([got[bd][0].numpy() for bd in bounds])
        nn = np.array([got[bd][0].numel() for bd in bounds])
        ls = np.concatenate([got[bd][1].numpy() for bd in bounds])
        topo.update({f"c{ci}__pi": pi, f"c{ci}__pj": pj, f"c{ci}__meta": np.array([nl, nt, C]),
                     f"c{ci}__nodes": nodes, f"c{ci}__n_nodes": nn, f"c{ci}__ls": ls})
        print(f"topology case {ci}: nl={nl} nt={nt} C={C} edges={len(pi)} chunks={len(bounds)}")
    np.savez_compressed(os.path.join(HERE, "topology.npz"), **topo)


if __name__ == "__main__":
    main()

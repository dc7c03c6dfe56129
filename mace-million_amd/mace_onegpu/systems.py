"""Synthetic inputs of the benchmark configurations (seeded, deterministic).

* water_box: n_mol rigid H2O molecules at 1.0 g/cm^3 in a cubic periodic box; O placed uniformly by random
  sequential addition with minimum-image O-O >= 2.5 A, O-H 0.9572 A, HOH 104.52 deg, uniformly random
  orientation (unit quaternion from 4 normals); atom order O, H, H per molecule.  This is the generator the
  reference's water boxes stand for (it replicates a 192-atom cell, receiver_chunk_mace.py:390-420, and the
  benchmark decks use replicated water64 cells); the build generates boxes of any size directly.
* fcc_alloy: FCC lattice, species drawn uniformly from a list, Gaussian jitter.
* maxwell_boltzmann: velocities at temperature T (metal units), centre-of-mass momentum removed.
All generators use numpy.random.default_rng(seed).
"""
import math

import numpy as np

WATER_VOLUME_A3 = 18.01528 / 6.02214076e23 / 1.0 * 1e24    # A^3 per molecule at 1.0 g/cm^3 (= 29.9151)
OH, HOH_DEG = 0.9572, 104.52
MASS = {1: 1.008, 8: 15.999, 24: 51.9961, 26: 55.845, 27: 58.933194, 28: 58.6934}
KB_EV = 8.617333262e-5
MVV2E = 1.0 / 9648.533212331     # amu * (A/ps)^2 -> eV  (1 eV/(A amu) = 9648.533 A/ps^2)


def water_box_length(n_mol):
    return (n_mol * WATER_VOLUME_A3) ** (1.0 / 3.0)


def _random_rotations(rng, n):
    q = rng.normal(size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    a, b, c, d = q.T
    R = np.empty((n, 3, 3))
    R[:, 0, 0] = a * a + b * b - c * c - d * d
    R[:, 0, 1] = 2 * (b * c - a * d)
    R[:, 0, 2] = 2 * (b * d + a * c)
    R[:, 1, 0] = 2 * (b * c + a * d)
    R[:, 1, 1] = a * a - b * b + c * c - d * d
    R[:, 1, 2] = 2 * (c * d - a * b)
    R[:, 2, 0] = 2 * (b * d - a * c)
    R[:, 2, 1] = 2 * (c * d + a * b)
    R[:, 2, 2] = a * a - b * b - c * c + d * d
    return R


def _rsa(rng, n, L, dmin):
    """Random sequential addition of n points in a periodic cube with minimum-image distance >= dmin.

    Exactly sequential RSA on the proposal stream rng.uniform(0, L, (batch, 3)): a proposal is kept iff it is at
    least dmin from every point kept before it.  Proposals are tested in batches (batch = n/8, at least 256):
    against earlier batches through a periodic k-d tree, and inside the batch in proposal order."""
    from scipy.spatial import cKDTree

    pts = np.empty((n, 3))
    k = 0
    batch = max(256, n // 8)
    while k < n:
        cand = rng.uniform(0.0, L, size=(batch, 3))
        valid = np.ones(batch, dtype=bool)
        if k:
            d, _ = cKDTree(pts[:k], boxsize=L).query(cand, k=1, distance_upper_bound=dmin)
            valid = d >= dmin
        idx = np.nonzero(valid)[0]
        pairs = cKDTree(cand[idx], boxsize=L).query_pairs(dmin, output_type="ndarray")
        nbr = {}
        for i, j in pairs:
            lo, hi = (i, j) if i < j else (j, i)
            nbr.setdefault(hi, []).append(lo)
        kept = np.zeros(len(idx), dtype=bool)
        for t in range(len(idx)):
            kept[t] = not any(kept[s] for s in nbr.get(t, ()))
        take = idx[kept][: n - k]
        pts[k:k + len(take)] = cand[take]
        k += len(take)
    return pts


def water_box(n_mol, seed=0):
    """Returns (pos [3 n_mol, 3] fp64 wrapped, box [3], Z [3 n_mol] int)."""
    rng = np.random.default_rng(seed)
    L = water_box_length(n_mol)
    if L < 2.5 * 3:
        raise ValueError("box too small")
    O = _rsa(rng, n_mol, L, 2.5)
    R = _random_rotations(rng, n_mol)
    th = math.radians(HOH_DEG) / 2
    h1 = np.array([OH * math.sin(th), 0.0, OH * math.cos(th)])
    h2 = np.array([-OH * math.sin(th), 0.0, OH * math.cos(th)])
    H1 = O + np.einsum("nij,j->ni", R, h1)
    H2 = O + np.einsum("nij,j->ni", R, h2)
    pos = np.stack([O, H1, H2], 1).reshape(-1, 3)
    pos = np.mod(pos, L)
    Z = np.tile(np.array([8, 1, 1]), n_mol)
    return pos, np.array([L, L, L]), Z


def fcc_alloy(n_cells=50, a=3.6, species=(26, 28, 24, 27), sigma=0.05, seed_species=0, seed_jitter=1):
    base = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    g = np.stack(np.meshgrid(*[np.arange(n_cells)] * 3, indexing="ij"), -1).reshape(-1, 3)
    pos = ((g[:, None, :] + base[None, :, :]) * a).reshape(-1, 3).astype(np.float64)
    Z = np.asarray(species)[np.random.default_rng(seed_species).integers(0, len(species), len(pos))]
    pos = pos + np.random.default_rng(seed_jitter).normal(scale=sigma, size=pos.shape)
    L = n_cells * a
    return np.mod(pos, L), np.array([L, L, L]), Z


def maxwell_boltzmann(Z, T=300.0, seed=4):
    """Velocities in A/ps for masses in amu at temperature T (K); total momentum removed."""
    m = np.array([MASS[int(z)] for z in Z])
    rng = np.random.default_rng(seed)
    sd = np.sqrt(KB_EV * T / (m * MVV2E))
    v = rng.normal(size=(len(Z), 3)) * sd[:, None]
    v -= (m[:, None] * v).sum(0) / m.sum()
    return v, m

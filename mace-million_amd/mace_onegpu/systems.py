"""Synthetic inputs of the benchmark configurations (seeded, deterministic).

* water_box: n_mol rigid H2O molecules at 1.0 g/cm^3 in a cubic periodic box; O placed uniformly by random
  sequential addition with minimum-image O-O >= 2.5 A, O-H 0.9572 A, HOH 104.52 deg, uniformly random
  orientation (unit quaternion from 4 normals); atom order O, H, H per molecule.  This is the generator the
  reference's water boxes stand for (it replicates a 192-atom cell, receiver_chunk_mace.py:390-420, and the
  benchmark decks use replicated water64 cells); the build generates boxes of any size directly.
* fcc_alloy: FCC lattice, species drawn uniformly from a list, Gaussian jitter.
* maxwell_boltzmann: velocities at temperature T (metal units), centre-of-mass momentum removed.
All generators use numpy.random.default_rng(seed).
* read_structure: orthorhombic periodic structures from extended XYZ, LAMMPS data (atomic style) or npz files;
  replicate: periodic replicas of a box (what the reference's --base / --rep options build,
  receiver_chunk_mace.py:390-420); add_structure_args / structure_from_args: the command-line options of the
  evaluator and MD entry points.
"""
import math
import os
import re

import numpy as np

WATER_VOLUME_A3 = 18.01528 / 6.02214076e23 / 1.0 * 1e24    # A^3 per molecule at 1.0 g/cm^3 (= 29.9151)
OH, HOH_DEG = 0.9572, 104.52
# chemical symbols and standard atomic weights (amu) of Z = 1 .. 89, the elements of the model
SYMBOLS = ("H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn Ga Ge As Se Br Kr Rb "
           "Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce Pr Nd Pm Sm Eu Gd Tb Dy Ho Er Tm Yb Lu "
           "Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Po At Rn Fr Ra Ac").split()
_WEIGHTS = (1.008, 4.0026, 6.94, 9.0122, 10.81, 12.011, 14.007, 15.999, 18.998, 20.180, 22.990, 24.305, 26.982,
            28.085, 30.974, 32.06, 35.45, 39.948, 39.098, 40.078, 44.956, 47.867, 50.942, 51.996, 54.938, 55.845,
            58.933, 58.693, 63.546, 65.38, 69.723, 72.630, 74.922, 78.971, 79.904, 83.798, 85.468, 87.62, 88.906,
            91.224, 92.906, 95.95, 98.0, 101.07, 102.91, 106.42, 107.87, 112.41, 114.82, 118.71, 121.76, 127.60,
            126.90, 131.29, 132.91, 137.33, 138.91, 140.12, 140.91, 144.24, 145.0, 150.36, 151.96, 157.25, 158.93,
            162.50, 164.93, 167.26, 168.93, 173.05, 174.97, 178.49, 180.95, 183.84, 186.21, 190.23, 192.22, 195.08,
            196.97, 200.59, 204.38, 207.2, 208.98, 209.0, 210.0, 222.0, 223.0, 226.0, 227.0)
MASS = {z + 1: m for z, m in enumerate(_WEIGHTS)}
MASS.update({1: 1.008, 8: 15.999, 24: 51.9961, 26: 55.845, 27: 58.933194, 28: 58.6934})
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


def replicate(pos, box, Z, reps):
    """Periodic replica (nx, ny, nz) of a box: copy c = (ix, iy, iz) (ix slowest) holds atoms c * N .. c * N + N - 1
    at pos + (ix, iy, iz) * box, so atom j of the replica is atom j % N of the base box."""
    nx, ny, nz = (int(r) for r in reps)
    sh = np.array([(ix, iy, iz) for ix in range(nx) for iy in range(ny) for iz in range(nz)], dtype=np.float64)
    pos_r = (np.asarray(pos)[None, :, :] + (sh * np.asarray(box))[:, None, :]).reshape(-1, 3)
    return pos_r, np.asarray(box, dtype=np.float64) * np.array([nx, ny, nz]), np.tile(np.asarray(Z), len(sh))


def _z_of(token):
    if token.isdigit():
        return int(token)
    if token not in SYMBOLS:
        raise ValueError(f"unknown element {token!r} (the model has Z = 1 .. {len(SYMBOLS)})")
    return SYMBOLS.index(token) + 1


def _read_xyz(path):
    with open(path) as fh:
        lines = fh.read().splitlines()
    n = int(lines[0].split()[0])
    m = re.search(r'Lattice="([^"]+)"', lines[1])
    if not m:
        raise ValueError(f"{path}: extended XYZ needs Lattice=\"...\" on its second line (a periodic box)")
    cell = np.array([float(x) for x in m.group(1).split()]).reshape(3, 3)
    if np.abs(cell - np.diag(np.diag(cell))).max() > 0:
        raise ValueError(f"{path}: orthorhombic cells only")
    rows = [ln.split() for ln in lines[2:2 + n]]
    if len(rows) != n:
        raise ValueError(f"{path}: {n} atoms announced, {len(rows)} lines")
    Z = np.array([_z_of(r[0]) for r in rows])
    pos = np.array([[float(x) for x in r[1:4]] for r in rows], dtype=np.float64)
    return pos, np.diag(cell).copy(), Z


def _read_lammps_data(path, type_z):
    """LAMMPS data file, atom_style atomic ("id type x y z [ix iy iz]"); types map to Z through type_z (type 1 ->
    type_z[0], ...).  The reference reads its water decks with types 1 = O, 2 = H (receiver_chunk_mace.py:395-399)."""
    with open(path) as fh:
        lines = [ln.split("#")[0].strip() for ln in fh]
    n, lo, hi, atoms = None, [0.0] * 3, [0.0] * 3, None
    for k, ln in enumerate(lines):
        t = ln.split()
        if len(t) == 2 and t[1] == "atoms":
            n = int(t[0])
        elif len(t) == 4 and t[2][1:] == "lo" and t[3][1:] == "hi":
            d = "xyz".index(t[2][0])
            lo[d], hi[d] = float(t[0]), float(t[1])
        elif len(t) == 6 and t[3:] == ["xy", "xz", "yz"] and any(float(x) != 0.0 for x in t[:3]):
            raise ValueError(f"{path}: orthorhombic boxes only")
        elif t and t[0] == "Atoms":
            atoms = k + 1
            break
    if n is None or atoms is None:
        raise ValueError(f"{path}: no atom count or no Atoms section")
    rows = [ln.split() for ln in lines[atoms:] if ln][:n]
    rows.sort(key=lambda r: int(r[0]))
    types = np.array([int(r[1]) for r in rows])
    if types.min() < 1 or types.max() > len(type_z):
        raise ValueError(f"{path}: atom types {types.min()} .. {types.max()}, but {len(type_z)} elements given")
    pos = np.array([[float(x) for x in r[2:5]] for r in rows], dtype=np.float64) - np.asarray(lo)
    return pos, np.asarray(hi) - np.asarray(lo), np.asarray(type_z)[types - 1]


def read_structure(path, type_z=(8, 1)):
    """(pos fp64 [N, 3] wrapped into [0, L), box [3], Z [N]) of an orthorhombic periodic structure: extended XYZ
    (.xyz / .extxyz, Lattice on the comment line), LAMMPS data (.data / .lmp, atomic style; type_z maps types to
    Z) or npz (arrays pos, box, Z)."""
    ext = os.path.splitext(path)[1].lower()
    if ext in (".xyz", ".extxyz"):
        pos, box, Z = _read_xyz(path)
    elif ext in (".data", ".lmp"):
        pos, box, Z = _read_lammps_data(path, type_z)
    elif ext == ".npz":
        with np.load(path) as f:
            pos, box, Z = np.asarray(f["pos"], dtype=np.float64), np.asarray(f["box"], dtype=np.float64), f["Z"]
    else:
        raise ValueError(f"{path}: structure formats are .xyz/.extxyz, .data/.lmp and .npz")
    box = np.asarray(box, dtype=np.float64).reshape(3)
    return np.mod(pos, box), box, np.asarray(Z).astype(np.int64)


def add_structure_args(ap):
    """The structure options of the command-line entry points (one source; --rep replicates it)."""
    g = ap.add_mutually_exclusive_group(required=True)
    g.add_argument("--structure", help="structure file (.xyz/.extxyz, LAMMPS .data, .npz)")
    g.add_argument("--base", help="base cell file, replicated by --rep")
    g.add_argument("--water", type=int, metavar="N_MOL", help="generated water box of N_MOL molecules")
    g.add_argument("--fcc", type=int, metavar="N_CELLS", help="generated FCC Fe/Ni/Cr/Co box of N_CELLS^3 cells")
    ap.add_argument("--rep", nargs=3, type=int, default=[1, 1, 1], help="periodic replica of the base cell")
    ap.add_argument("--types", default="O,H", help="element of each LAMMPS data atom type (default O,H)")
    ap.add_argument("--seed", type=int, default=0, help="seed of a generated box")


def structure_from_args(a):
    """(pos, box, Z, base) of the options: base = (pos, box, Z) of the unreplicated cell."""
    if a.structure:
        if tuple(a.rep) != (1, 1, 1):
            raise ValueError("--rep replicates --base, --water or --fcc, not --structure")
        pos, box, Z = read_structure(a.structure, [_z_of(t) for t in a.types.split(",")])
    elif a.base:
        pos, box, Z = read_structure(a.base, [_z_of(t) for t in a.types.split(",")])
    elif a.water:
        pos, box, Z = water_box(a.water, seed=a.seed)
    else:
        pos, box, Z = fcc_alloy(n_cells=a.fcc)
    base = (pos, box, Z)
    if tuple(a.rep) != (1, 1, 1):
        pos, box, Z = replicate(pos, box, Z, a.rep)
    return pos, box, Z, base

"""Pins of the fp64 CPU oracle (the reference's criteria and the model's invariances), CPU only."""
import numpy as np
import pytest
import torch

from mace_onegpu import systems
from oracle import mace_ref, neighbors


def _rot(seed):
    q = np.random.default_rng(seed).normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([[a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
                     [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
                     [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d]])


def _cluster_edges(pos, r_max):
    """Open-boundary edges of a small cluster (no periodic images), receiver-sorted."""
    d = pos[:, None, :] - pos[None, :, :]
    dd = (d ** 2).sum(-1)
    recv, send = np.nonzero((dd < r_max ** 2) & ~np.eye(len(pos), dtype=bool))
    return recv, send


@pytest.fixture(scope="module")
def cluster():
    """36 atoms of water in a 30 A box (no periodic neighbours): rotations act on the whole geometry."""
    pos, box, Z = systems.water_box(64, seed=2)
    keep = np.nonzero(((pos - pos[0]) ** 2).sum(1) < 4.6 ** 2)[0][:36]
    p = pos[keep] - pos[keep].mean(0) + 15.0
    return p, np.array([30.0, 30.0, 30.0]), Z[keep] - 1


def test_three_pass_matches_full_graph(ref_model, water192):
    """fp64 three-pass vs full graph (the reference's test_fp64_matches_full_graph, test_threepass.py:66-71)."""
    w = water192
    E, e, F = mace_ref.energy_forces_full(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"])
    E3, eat, F3, _, _ = mace_ref.three_pass(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"], chunk=48)
    assert abs(E3 - E) < 1e-7 * len(e)
    assert float((F3 - F).abs().max()) < 1e-9


def test_chunk_invariance(ref_model, water192):
    w = water192
    a = mace_ref.three_pass(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"], chunk=48)
    b = mace_ref.three_pass(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"], chunk=192)
    assert abs(a[0] - b[0]) < 1e-8 * len(w["pos"])
    assert float((a[2] - b[2]).abs().max()) < 1e-9


def test_rotation_translation_permutation_invariance(ref_model, cluster):
    """E invariant, F covariant under rotation, translation and atom permutation; fails for a wrong coupling
    sign, a transposed coupling, a wrong SH component or a mismatched parity."""
    p, box, sp = cluster
    recv, send = _cluster_edges(p, 6.0)
    E0, _, F0 = mace_ref.energy_forces_full(ref_model, p, box, sp, recv, send)
    assert abs(E0) > 1e-4 and float(F0.abs().max()) > 1e-4       # a non-trivial function
    R = _rot(3)
    c = p.mean(0)
    pr = (p - c) @ R.T + c + np.array([0.3, -0.7, 1.1])
    E1, _, F1 = mace_ref.energy_forces_full(ref_model, pr, box, sp, recv, send)
    assert abs(E1 - E0) < 1e-10 * max(1.0, abs(E0))
    np.testing.assert_allclose(F1.numpy(), F0.numpy() @ R.T, atol=1e-11)
    perm = np.random.default_rng(0).permutation(len(p))
    inv = np.argsort(perm)
    r2, s2 = _cluster_edges(p[perm], 6.0)
    E2, _, F2 = mace_ref.energy_forces_full(ref_model, p[perm], box, sp[perm], r2, s2)
    assert abs(E2 - E0) < 1e-10 * max(1.0, abs(E0))
    np.testing.assert_allclose(F2.numpy()[inv], F0.numpy(), atol=1e-11)
    # inversion (parity): every vector flips; the natural-parity model is inversion invariant
    E3, _, F3 = mace_ref.energy_forces_full(ref_model, 2 * c - p, box, sp, recv, send)
    assert abs(E3 - E0) < 1e-10 * max(1.0, abs(E0))


def test_forces_are_minus_energy_gradient(ref_model, cluster):
    """Central finite differences of E along a random displacement field against -F . u (fp64)."""
    p, box, sp = cluster
    recv, send = _cluster_edges(p, 6.0)
    E0, _, F0 = mace_ref.energy_forces_full(ref_model, p, box, sp, recv, send)
    u = np.random.default_rng(5).normal(size=p.shape)
    u /= np.linalg.norm(u)

    def energy(x):
        with torch.no_grad():
            e = mace_ref.energy_full(ref_model, torch.as_tensor(x), box, torch.as_tensor(sp),
                                     torch.as_tensor(recv), torch.as_tensor(send))
        return float(e.sum())
    h = 1e-4
    d1 = (energy(p + h * u) - energy(p - h * u)) / (2 * h)
    d2 = (energy(p + 2 * h * u) - energy(p - 2 * h * u)) / (4 * h)
    fd = (4 * d1 - d2) / 3                       # Richardson: O(h^4)
    an = -float((F0.numpy() * u).sum())
    assert abs(fd - an) < 1e-9 + 1e-6 * abs(an), (fd, an)


def test_replica_reproduces_base_cell(ref_model, water192):
    """A 2x1x1 periodic replica gives every atom the force of its base-cell image and the same E/N
    (the reference's test_replica_reproduces_base_cell, test_threepass.py:80-88)."""
    pos, box, Z = water192["raw"]
    rep = np.concatenate([pos, pos + np.array([box[0], 0, 0])])
    box2 = box * np.array([2, 1, 1])
    Zr = np.concatenate([Z, Z])
    s = neighbors.SystemRef(rep, box2, Zr - 1, 6.0)
    NN, rp, send = s.build_neighbors()
    recv = np.repeat(np.arange(s.N), NN)
    E2, _, F2, _, _ = mace_ref.three_pass(ref_model, s.pos, box2, s.spidx, recv, send, chunk=200)
    w = water192
    sb = w["sys"]
    E1, _, F1, _, _ = mace_ref.three_pass(ref_model, w["pos"], box, w["spec"], w["recv"], w["send"], chunk=192)
    base_of_sorted = s.perm % len(pos)               # replica atom -> original base atom
    base_sorted_index = np.argsort(sb.perm)          # original base atom -> base sorted index
    Fb = F1.numpy()[base_sorted_index[base_of_sorted]]
    assert abs(E2 / s.N - E1 / len(pos)) < 1e-12
    assert np.abs(F2.numpy() - Fb).max() < 1e-11


def test_tables_converge_to_the_mlp(ref_model, water192):
    """Hermite tables (fp64 samples, 512 knots) vs the exact radial MLP: the interpolation error is small and
    falls ~ knots^-3 (numerics_water.json: 1.6e-5 eV/A at 512 knots for the trained MPA-0)."""
    w = water192
    E, e, F = mace_ref.energy_forces_full(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"])
    errs = []
    for M in (128, 256):
        tab = mace_ref.Tables64(ref_model, sorted(set(w["spec"].tolist())), n_grid=M)
        Et, et, Ft = mace_ref.energy_forces_full(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"],
                                                 tables=tab)
        errs.append(float((Ft - F).abs().max()))
    assert errs[1] < 1e-4 * float(F.abs().max())
    assert errs[1] < errs[0] / 4                    # cubic convergence (factor ~8 per halving of h)


def test_atom_energy_local_matches_whole_system(ref_model, water192):
    """The per-atom energy evaluated from the atom's own 2 r_max neighbourhood (the production-scale spot check's
    oracle) equals the whole-system three-pass per-atom energy (fp64 rounding), for O and H atoms of the periodic
    192-atom box; with the 512-knot tables as well."""
    w = water192
    E3, eat, F3, _, _ = mace_ref.three_pass(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"], chunk=192)
    for i in (0, 1, 2, 97, 191):
        e = mace_ref.atom_energy_local(ref_model, w["pos"], w["box"], w["spec"], i)
        assert abs(e - float(eat[i])) < 1e-12 * max(1.0, abs(e)), (i, e, float(eat[i]))
    tab = mace_ref.Tables64(ref_model, sorted(set(np.asarray(w["spec"]).tolist())), n_grid=512)
    E3t, eat_t, _, _, _ = mace_ref.three_pass(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"],
                                              chunk=96, tables=tab)
    for i in (4, 150):
        e = mace_ref.atom_energy_local(ref_model, w["pos"], w["box"], w["spec"], i, tables=tab)
        assert abs(e - float(eat_t[i])) < 1e-12 * max(1.0, abs(e))


def _pair_networks(model, seed, pairs):
    """Random radial networks (fp32-representable fp64 values, the model's layer sizes) for the given ordered
    (sender column, receiver column) pairs: {pair: {block k: [r0..r3]}}; pairs listed together share one network."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for group in pairs:
        nets = {k: [torch.randn(*model.p[f"i{k}_r{j}"].shape, generator=g, dtype=torch.float64).float().double()
                    for j in range(4)] for k in range(2)}
        for pr in group:
            out[pr] = nets
    return out


@pytest.fixture(scope="module")
def pair_model():
    """The seed-0 model with a radial network per ordered pair of H (column 0) and O (column 7): (H, H) and
    (O, O) share one, (H, O) and (O, H) (sender, receiver) have their own."""
    from mace_onegpu import model as mm
    m = mm.MaceModel(seed=0)
    m.pair_radial = _pair_networks(m, 5, [[(0, 0), (7, 7)], [(0, 7)], [(7, 0)]])
    return m


def test_pair_networks_equal_to_the_default_reproduce_it(model, ref_model, water192):
    """Per-pair networks that are all the model's own network: the per-edge selection gives the default result."""
    from mace_onegpu import model as mm, o3
    w = water192
    m = mm.MaceModel(seed=0)
    own = {k: [model.p[f"i{k}_r{j}"].detach().double() for j in range(4)] for k in range(2)}
    m.pair_radial = {(a, b): own for a in (0, 7) for b in (0, 7)}
    rm = mace_ref.RefModel(m, o3.coupling)
    E0, e0, F0 = mace_ref.energy_forces_full(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"])
    E1, e1, F1 = mace_ref.energy_forces_full(rm, w["pos"], w["box"], w["spec"], w["recv"], w["send"])
    assert abs(E1 - E0) < 1e-12 * abs(E0) + 1e-12 and float((F1 - F0).abs().max()) < 1e-12


def test_pair_tables_follow_the_per_edge_networks(pair_model, water192):
    """Three-pass with the per-pair 512-knot tables (ordered pair p = s_send S + s_recv) against the full graph with
    each edge's own (sender, receiver) network: equal to the tables' interpolation error.  Swapping the (H, O) and
    (O, H) networks changes the result by far more, so a transposed pair index would fail."""
    from mace_onegpu import o3
    w = water192
    rm = mace_ref.RefModel(pair_model, o3.coupling)
    E, e, F = mace_ref.energy_forces_full(rm, w["pos"], w["box"], w["spec"], w["recv"], w["send"])
    tab = mace_ref.Tables64(rm, [0, 7], n_grid=512)
    Et, et, Ft, _, _ = mace_ref.three_pass(rm, w["pos"], w["box"], w["spec"], w["recv"], w["send"], chunk=96,
                                           tables=tab)
    N = len(w["pos"])
    dF = float((Ft - F).abs().max())
    assert abs(Et - E) / N < 1e-6 and dF < 1e-4 * float(F.abs().max())
    swapped = dict(rm.pair_radial)
    swapped[(0, 7)], swapped[(7, 0)] = rm.pair_radial[(7, 0)], rm.pair_radial[(0, 7)]
    rs = mace_ref.RefModel(pair_model, o3.coupling)
    rs.pair_radial = swapped
    Es, es, Fs = mace_ref.energy_forces_full(rs, w["pos"], w["box"], w["spec"], w["recv"], w["send"])
    assert float((Fs - F).abs().max()) > 100 * dF and abs(Es - E) / N > 100 * abs(Et - E) / N

"""GPU parity of the HIP path against the CPU oracle (marked gpu; run on the MI355X box).

Tolerances: the parity bar (energy 1e-5 eV/atom, forces 1e-3 eV/A max-abs) and, because the random-init model's
outputs are small (|F| ~ 0.03 eV/A), also relative bars: forces within 1e-4 of max|F| against the exact fp64
oracle (fp32 arithmetic + 512-knot tables, the reference's production numerics) and within 2e-5 against the fp64
oracle that uses the same tables (fp32 rounding only).  Integer outputs (neighbour lists) are bit-exact.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU test without a GPU"
    return "cuda"


def _oracle_three_pass(ref_model, s, chunk, tables=None):
    from oracle import mace_ref
    recv = np.repeat(np.arange(s.N), s.NN.cpu().numpy())
    return mace_ref.three_pass(ref_model, s.pos.cpu().numpy(), s.box, s.spidx.cpu().numpy(), recv,
                               s.send.cpu().numpy(), chunk=chunk, tables=tables)


def _check(E, eat, F, ref, N, rel=1e-4):
    E0, e0, F0 = ref[0], ref[1], ref[2]
    dE = abs(E - E0) / N
    de = float((eat.cpu() - e0).abs().max())
    dF = float((F.cpu() - F0).abs().max())
    Fm = float(F0.abs().max())
    _say(f"  |dE|/N={dE:.2e} max|de_i|={de:.2e} max|dF|={dF:.2e} (max|F|={Fm:.3e}, rel {dF / Fm:.2e})")
    assert dE < 1e-5 and de < 1e-5
    assert dF < 1e-3 and dF < rel * Fm


# ----------------------------------------------------------------------------- neighbour list
G = np.load(os.path.join(HERE, "golden", "neighbors.npz"))


@pytest.mark.parametrize("name", sorted({k.split("__")[0] for k in G.files}))
def test_neighbor_list_bit_exact(dev, name):
    from mace_onegpu.receiver_chunk_mace import System
    g = {k.split("__")[1]: G[k] for k in G.files if k.startswith(name + "__")}
    _say(f"case {name}")
    s = System(g["pos"], g["box"], g["spidx"], 6.0, dev)
    s.build_neighbors()
    assert np.array_equal(s.perm.cpu().numpy(), g["perm"])
    assert np.array_equal(s.pos.cpu().numpy(), g["pos_sorted"])
    assert np.array_equal(s.NN.cpu().numpy(), g["NN"])
    assert np.array_equal(s.send.cpu().numpy(), g["send"])


def test_neighbor_list_large_box_matches_oracle(dev):
    """Cell-list path at config-3 density on a 4,608-atom box (3 x 3 x 3 cells or more)."""
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import System
    from oracle import neighbors
    pos, box, Z = systems.water_box(1536, seed=9)
    s = System(pos, box, Z - 1, 6.0, dev)
    s.build_neighbors()
    r = neighbors.SystemRef(pos, box, Z - 1, 6.0)
    NN, rp, send = r.build_neighbors()
    assert np.array_equal(s.perm.cpu().numpy(), r.perm)
    assert np.array_equal(s.NN.cpu().numpy(), NN)
    assert np.array_equal(s.send.cpu().numpy(), send)


@pytest.mark.parametrize("case", ["water98304", "fcc500000"])
def test_neighbor_list_full_size_matches_c_oracle(dev, case):
    """Bit-exact at benchmark sizes: config 3's 98,304-atom water box and config 4's 500,000-atom FCC alloy
    (GPU cell list vs the plain-C restatement of the reference's build)."""
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import System
    from oracle import nlist_c
    _say(f"case {case}")
    if case == "water98304":
        pos, box, Z = systems.water_box(32768, seed=0)
    else:
        pos, box, Z = systems.fcc_alloy(n_cells=50)
    s = System(pos, box, np.zeros(len(pos), np.int32), 6.0, dev)
    s.build_neighbors()
    perm, pos_sorted, NN, rowptr, send = nlist_c.neighbor_list(pos, box, 6.0)
    _say(f"  {len(pos)} atoms, {len(send)} pairs")
    assert np.array_equal(s.perm.cpu().numpy(), perm)
    assert np.array_equal(s.pos.cpu().numpy(), pos_sorted)
    assert np.array_equal(s.NN.cpu().numpy(), NN)
    assert np.array_equal(s.rowptr.cpu().numpy(), rowptr)
    assert np.array_equal(s.send.cpu().numpy(), send)


# ----------------------------------------------------------------------------- kernels
def test_mfma_linear_against_torch(dev):
    """mm_linear: several K-chunks, row gathers/scatters, species lists, 1/(rho+1) scaling, accumulate."""
    from mace_onegpu import _lib
    from mace_onegpu.fast_layers import LinPlan, mfma_block
    torch.manual_seed(0)
    n, S = 333, 3
    Ws = [torch.randn(128, 128, dtype=torch.float64) for _ in range(2 * S)]
    W = torch.cat([mfma_block(w.float()) for w in Ws]).to(dev)
    x = torch.randn(n, 768, dtype=torch.float64)
    rho = torch.rand(n, dtype=torch.float64) * 3
    spec = torch.randint(0, S, (n,))
    plan = LinPlan([(0, [(0, 0), (384, 1)]), (128, [(128, 0), (512, 1)]), (256, [(640, 1)])])
    out0 = torch.randn(n, 384, dtype=torch.float64)
    out = out0.float().to(dev)
    lists = torch.zeros(S, n, dtype=torch.int32, device=dev)
    counts = torch.zeros(S, dtype=torch.int32, device=dev)
    _lib.K.mm_species_lists(spec.int().to(dev), n, S, lists, n, counts, _lib.stream())
    _lib.K.mm_linear(x.float().to(dev), 768, None, out, 384, None, W, rho.float().to(dev), 1, lists, counts, n, S, 2, n,
                     1, plan.n, plan.nsrc, plan.inoff, plan.widx, plan.outoff, 0, _lib.stream())
    ref = out0.clone()
    inv = 1.0 / (rho + 1)
    for i in range(n):
        s = int(spec[i])
        w0, w1 = Ws[2 * s], Ws[2 * s + 1]
        ref[i, 0:128] += inv[i] * (x[i, 0:128] @ w0 + x[i, 384:512] @ w1)
        ref[i, 128:256] += inv[i] * (x[i, 128:256] @ w0 + x[i, 512:640] @ w1)
        ref[i, 256:384] += inv[i] * (x[i, 640:768] @ w1)
    err = float((out.double().cpu() - ref).abs().max() / ref.abs().max())
    # the same sums in fp32 on the CPU: the split bf16 products must be as accurate as fp32 arithmetic
    ref32 = out0.float().clone()
    x32, inv32 = x.float(), inv.float()
    W32 = [w.float() for w in Ws]
    for i in range(n):
        s = int(spec[i])
        w0, w1 = W32[2 * s], W32[2 * s + 1]
        ref32[i, 0:128] += inv32[i] * (x32[i, 0:128] @ w0 + x32[i, 384:512] @ w1)
        ref32[i, 128:256] += inv32[i] * (x32[i, 128:256] @ w0 + x32[i, 512:640] @ w1)
        ref32[i, 256:384] += inv32[i] * (x32[i, 640:768] @ w1)
    err32 = float((ref32.double() - ref).abs().max() / ref.abs().max())
    _say(f"  mm_linear rel err {err:.2e} (fp32 CPU {err32:.2e})")
    assert err < 2e-6 and err <= max(4 * err32, 3e-7)
    # species lists are a stable partition
    for s in range(S):
        c = int(counts[s])
        assert torch.equal(lists[s, :c].cpu().long(), torch.nonzero(spec == s).squeeze(1))
    # the row count from device memory (graph replays): a launch sized for n rows computes rows 0 .. n_dev - 1
    # only, bit for bit as a launch of n_dev rows, and leaves the rest untouched
    n_dev = 150
    xs = x[:, :128].float().to(dev).contiguous()
    p1 = LinPlan([(0, [(0, 0)])])
    a = torch.full((n, 128), float("nan"), device=dev)
    b = torch.full((n, 128), float("nan"), device=dev)
    _lib.K.mm_linear(xs, 128, None, a, 128, None, W, None, 0, None, None, 0, 1, 0, n_dev, 0, p1.n, p1.nsrc,
                     p1.inoff, p1.widx, p1.outoff, 0, _lib.stream())
    _lib.K.mm_linear(xs, 128, None, b, 128, None, W, None, 0, None,
                     torch.tensor([n_dev], dtype=torch.int32, device=dev), 0, 1, 0, n, 0, p1.n, p1.nsrc, p1.inoff,
                     p1.widx, p1.outoff, 0, _lib.stream())
    torch.cuda.synchronize()
    assert torch.equal(a[:n_dev], b[:n_dev]) and bool(torch.isfinite(b[:n_dev]).all())
    assert bool(b[n_dev:].isnan().all())
    # 16-channel-block-major input rows (in_cb, the layout of mm_conv2_bwd's dL/dX): the same sums, bit for bit, as
    # the component-major rows they permute; row gathers and 4 components of which 3 share a weight block
    x4 = x[:, :512].float().to(dev).contiguous()                               # [n, 4 components x 128]
    x4cb = x4.view(n, 4, 8, 16).permute(0, 2, 1, 3).contiguous().view(n, 512)  # [n, 8 blocks x 4 x 16]
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(3))[:200].int().to(dev)
    p4 = LinPlan([(0, [(0, 0)]), (128, [(128, 1)]), (256, [(256, 1)]), (384, [(384, 1)])])
    c0 = torch.empty(200, 512, device=dev)
    c1 = torch.empty(200, 512, device=dev)
    _lib.K.mm_linear(x4, 512, rows, c0, 512, None, W, None, 0, None, None, 0, 1, 0, 200, 0, p4.n, p4.nsrc,
                     p4.inoff, p4.widx, p4.outoff, 0, _lib.stream())
    _lib.K.mm_linear(x4cb, 512, rows, c1, 512, None, W, None, 0, None, None, 0, 1, 0, 200, 0, p4.n, p4.nsrc,
                     p4.inoff, p4.widx, p4.outoff, 4, _lib.stream())
    torch.cuda.synchronize()
    assert torch.equal(c0, c1)
    ref4 = torch.cat([x[rows.long().cpu(), 0:128] @ Ws[0]] + [x[rows.long().cpu(), 128 * k:128 * k + 128] @ Ws[1]
                                                              for k in (1, 2, 3)], dim=1)
    assert float((c1.double().cpu() - ref4).abs().max() / ref4.abs().max()) < 2e-6
    with pytest.raises(RuntimeError, match="channel-block-major"):
        _lib.K.mm_linear(x4cb, 512, None, c1, 512, None, W, None, 0, None, None, 0, 1, 0, 200, 0, p4.n, p4.nsrc,
                         p4.inoff, p4.widx, p4.outoff, 3, _lib.stream())


def test_spline_tables_against_oracle_hermite(dev, model, ref_model):
    """The interval coefficients reproduce the fp64 Hermite tables (same interpolant) to fp32 rounding."""
    from mace_onegpu.fast_layers import FastLayers
    from oracle import mace_ref
    fl = FastLayers(model, [0, 7], spline_grid=512, device=dev)
    t64 = mace_ref.Tables64(ref_model, [0, 7], n_grid=512)
    r = torch.linspace(0.52, 5.99, 2000, dtype=torch.float64)
    for k, nW in ((0, 4), (1, 10)):
        coef = fl.tab[k].cpu().reshape(8, 1, 511, nW, 16, 4)
        x = torch.clamp((r - 0.5) * fl.inv_h, 0, 511 - 1e-4)
        kf = torch.floor(x).long()
        t = (x - kf)
        cf = coef[:, 0][:, kf]                                   # [cb, n, nW, 16, 4]
        Wg = cf[..., 0] + t[None, :, None, None] * (cf[..., 1] + t[None, :, None, None] * (cf[..., 2] + t[None, :, None, None] * cf[..., 3]))
        Wg = Wg.double().permute(1, 2, 0, 3).reshape(len(r), nW * 128)
        Wo = t64.lookup(k, r, torch.zeros(len(r), dtype=torch.long))
        err = float((Wg - Wo).abs().max() / Wo.abs().max())
        _say(f"  table layer {k + 1}: rel err {err:.2e}")
        assert err < 2e-6


# ----------------------------------------------------------------------------- end to end
@pytest.fixture(scope="module")
def water_gpu(dev):
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import System
    pos, box, Z = systems.water_box(64, seed=0)
    s = System(pos, box, Z - 1, 6.0, dev)
    s.build_neighbors()
    return s


@pytest.mark.parametrize("chunk", [48, 192])
def test_standalone_three_pass_vs_oracle(dev, model, ref_model, water_gpu, chunk):
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    s = water_gpu
    ev = ReceiverChunkMACE(model, chunk=chunk, device=dev)
    E, eat, F, PF = ev.compute(s)
    _say(f"chunk {chunk}: E={E:.8f}")
    _check(E, eat, F, _oracle_three_pass(ref_model, s, 192), s.N, rel=1e-4)


@pytest.mark.parametrize("deterministic", [False, True])
def test_low_memory_mode_vs_oracle_and_default(dev, model, ref_model, water_gpu, deterministic):
    """ReceiverChunkMACE(low_memory=True): chunk topologies rebuilt per pass and each chunk's pair forces added to F
    at once (mm_chunk_forces; the reference's _accum_forces, receiver_chunk_mace.py:272-276).  Against the oracle,
    and against the default path: the same per-edge pair forces, summed per pass instead of once, so the forces
    agree to fp32 rounding of PF_B + PF_C and the energies exactly (deterministic mode: bitwise)."""
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    s = water_gpu
    lo = ReceiverChunkMACE(model, chunk=48, device=dev, low_memory=True, deterministic=deterministic)
    E, eat, F, PF = lo.compute(s)
    assert PF is None
    _say(f"low memory (deterministic {deterministic}): E={E:.8f}")
    _check(E, eat, F, _oracle_three_pass(ref_model, s, 192), s.N, rel=1e-4)
    E1, eat1, F1, PF1 = ReceiverChunkMACE(model, chunk=48, device=dev, deterministic=deterministic).compute(s)
    dF = float((F - F1).abs().max())
    _say(f"  vs default: |dE| {abs(E - E1):.2e}, max|dF| {dF:.2e}")
    assert dF <= 1e-6 * float(F1.abs().max())
    if deterministic:
        assert torch.equal(eat, eat1)
        E2, eat2, F2, _ = lo.compute(s)
        assert torch.equal(F2, F) and torch.equal(eat2, eat)      # bitwise repeatable
    else:
        assert float((eat - eat1).abs().max()) < 1e-9


def test_chunked_atom_forces_beyond_int32_pairs(dev, model, water_gpu, monkeypatch):
    """Beyond 2^31 - 1 pairs the per-atom forces are summed chunk by chunk (mm_chunk_forces over each chunk's sender
    CSR) instead of through one sort of the whole pair list: the limit lowered to 100 pairs sends this box down
    that path, which must give the whole-list sums to fp64 rounding (same pair forces, other summation order)."""
    from mace_onegpu import receiver_chunk_mace as rcm
    s = water_gpu
    ev = rcm.ReceiverChunkMACE(model, chunk=48, device=dev, deterministic=True)
    graphs = ev.graphs(s)
    E, eat, F, PF = ev.compute(s, graphs=graphs)
    monkeypatch.setattr(rcm, "INT32_MAX", 100)
    F2 = rcm.pair_to_atom_forces(s, PF, graphs)
    d = float((F2 - F).abs().max())
    _say(f"  chunked force sums vs whole-list: max|dF| {d:.2e}")
    assert d <= 1e-12 * float(F.abs().max())
    with pytest.raises(ValueError, match="chunk topologies"):
        rcm.pair_to_atom_forces(s, PF)


def test_fp32_vs_oracle_with_same_tables(dev, model, ref_model, water_gpu):
    """Against the fp64 oracle that uses the same 512-knot tables only fp32 rounding remains."""
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    from oracle import mace_ref
    s = water_gpu
    tab = mace_ref.Tables64(ref_model, sorted(set(s.spidx.cpu().tolist())), n_grid=512)
    ev = ReceiverChunkMACE(model, chunk=96, device=dev)
    E, eat, F, PF = ev.compute(s)
    _check(E, eat, F, _oracle_three_pass(ref_model, s, 96, tables=tab), s.N, rel=2e-5)


@pytest.mark.parametrize("shuffle", [None, 3])
def test_mliap_boundary_with_ghosts(dev, model, ref_model, water_gpu, shuffle):
    """ThreePassMLIAP.compute_forces on the periodic-image data object (ghost senders, forward/reverse exchange,
    optionally unsorted pairs) gives the oracle's energies and forces."""
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    s = water_gpu
    data = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True, shuffle_pairs_seed=shuffle)
    assert data.nghost > 0
    tp = ThreePassMLIAP(model, chunk=80)
    tp.compute_forces(data)
    _check(data.energy, data.eatoms, data.atom_forces(), _oracle_three_pass(ref_model, s, 192), s.N)


def test_multispecies_fcc_vs_oracle(dev, model, ref_model):
    """Four species (Fe, Ni, Cr, Co): species-block skip, per-species symmetric contraction and readout rows."""
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    pos, box, Z = systems.fcc_alloy(n_cells=4, a=3.6)
    s = System(pos, box, Z - 1, 6.0, dev)
    s.build_neighbors()
    ev = ReceiverChunkMACE(model, chunk=100, device=dev)
    E, eat, F, PF = ev.compute(s)
    _check(E, eat, F, _oracle_three_pass(ref_model, s, 256), s.N)


def test_replica_and_translation_at_size(dev, model):
    """Size-independent properties on a 12,288-atom 4x4x4 replica: every atom's force equals its base-cell
    image's, E/N equals the base cell's, a rigid translation changes nothing, and the forces sum to zero."""
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    pos, box, Z = systems.water_box(64, seed=0)
    n = len(pos)
    g = np.stack(np.meshgrid(*[np.arange(4)] * 3, indexing="ij"), -1).reshape(-1, 3)
    rep = (g[:, None, :] * box[None, None, :] + pos[None]).reshape(-1, 3)
    Zr = np.tile(Z, len(g))
    base = System(pos, box, Z - 1, 6.0, dev)
    base.build_neighbors()
    Eb, _, Fb, _ = ReceiverChunkMACE(model, chunk=192, device=dev).compute(base)
    big = System(rep, box * 4, Zr - 1, 6.0, dev)
    big.build_neighbors()
    ev = ReceiverChunkMACE(model, chunk=4096, device=dev)
    E, eat, F, PF = ev.compute(big)
    Fb_orig = torch.empty_like(Fb)
    Fb_orig[base.perm] = Fb
    F_orig = torch.empty_like(F)
    F_orig[big.perm] = F
    dF = float((F_orig - Fb_orig.repeat(len(g), 1)).abs().max())
    _say(f"  replica: E/N {E / big.N:.10f} base {Eb / n:.10f} max|dF| {dF:.2e}")
    assert abs(E / big.N - Eb / n) < 1e-7
    assert dF < 1e-5 * float(Fb.abs().max()) + 1e-9
    assert float(F.sum(0).abs().max()) < 1e-4 * float(F.abs().max())
    shifted = System(rep + np.array([0.37, -1.3, 2.9]), box * 4, Zr - 1, 6.0, dev)
    shifted.build_neighbors()
    E2, _, F2, _ = ev.compute(shifted)
    F2o = torch.empty_like(F2)
    F2o[shifted.perm] = F2
    assert abs(E2 - E) / big.N < 1e-8
    assert float((F2o - F_orig).abs().max()) < 1e-5 * float(F.abs().max())


def test_forces_are_the_energy_gradient_below_the_table_start(dev, model):
    """A pair closer than the spline tables' first knot (r_lo = 0.5 A; such pairs occur by the tens of thousands
    in configuration 5's MD with this random-weight model, which has no short-range repulsion).  Below r_lo the
    radial weights are clamped to W(r_lo) (the clamp of spline_w._coords, spline_w.py:18-27), so the forces must
    leave out their r-derivative there; the reference's backward takes the table's slope at the clamped end
    instead, which made the full-size MD gain 318 eV over 100 steps.  The H atom of molecule 1 is put 0.3 A from
    the O atom of molecule 0, and its force is compared with a 4-point central difference of the total energy
    (h = 1e-3 A along x, y and z; both atoms stay below r_lo).  Measured: 1.2e-5 eV/A, and 3.0e-2 eV/A with the
    slope taken as the reference takes it; the bound, 2e-4 eV/A, lies between them (the difference's fp32 noise
    is about 1e-8 eV of energy over 1e-3 A)."""
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    pos, box, Z = systems.water_box(64, seed=3)
    pos = pos.copy()
    u = np.array([0.48, -0.6, 0.64])
    pos[4] = pos[0] + 0.3 * u / np.linalg.norm(u)

    def energy_forces(p):
        s = System(p, box, Z - 1, 6.0, dev)
        s.build_neighbors()
        E, eat, F, PF = ReceiverChunkMACE(model, chunk=4096, device=dev).compute(s)
        Fo = torch.empty_like(F)
        Fo[s.perm.long()] = F
        return E, Fo.cpu().numpy()

    E0, F0 = energy_forces(pos)
    h = 1e-3
    fd = np.zeros(3)
    for d in range(3):
        e = {}
        for k in (1, -1, 2, -2):
            p = pos.copy()
            p[4, d] += k * h
            e[k] = energy_forces(p)[0]
        fd[d] = -(8 * (e[1] - e[-1]) - (e[2] - e[-2])) / (12 * h)
    err = float(np.abs(fd - F0[4]).max())
    _say(f"  pair at 0.3 A: F {F0[4].tolist()}  F_fd {fd.tolist()}  max|F - F_fd| {err:.3e} eV/A")
    assert err < 2e-4


def test_md_steps_conserve_energy(dev, model):
    """Ten velocity-Verlet steps of a 1,536-atom box: the skin-filtered pair list equals a fresh build and the
    total energy drift stays far below the kinetic energy."""
    from mace_onegpu import systems
    from mace_onegpu.md import MDRunner
    from mace_onegpu.receiver_chunk_mace import System
    pos, box, Z = systems.water_box(512, seed=1)
    md = MDRunner(model, pos, box, Z, chunk=1024, device=dev)
    md.forces()
    s = System(md.pos.cpu().numpy(), box, (md.Z - 1).cpu().numpy(), 6.0, dev)
    s.build_neighbors()
    pairs_filtered = set(zip(np.repeat(np.arange(md.pairs.N), md.pairs.NN.cpu().numpy()).tolist(),
                             md.pairs.send_view.cpu().tolist()))
    perm = s.perm.cpu().numpy()            # fresh sorted index -> md slot
    pairs_fresh = set(zip(perm[np.repeat(np.arange(s.N), s.NN.cpu().numpy())].tolist(),
                          perm[s.send.cpu().numpy()].tolist()))
    assert pairs_filtered == pairs_fresh
    e_tot = []
    for _ in range(10):
        md.step()
        e_tot.append(md.E + md.kinetic())
    drift = max(e_tot) - min(e_tot)
    _say(f"  MD: E_tot range {drift:.3e} eV over 10 steps, KE {md.kinetic():.3f} eV")
    assert drift < 1e-3 * md.kinetic()


def test_layer1_cache_matches_recompute(dev, model, water_gpu):
    """Pass C reusing pass A's layer-1 message/density gives the recomputed result.  (Not bitwise: pass B's
    sender-feature gradient is scattered with fp32 atomics, so G1 differs between any two runs at the rounding
    level, as the reference's index_add_ / tl.atomic_add do.)"""
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    s = water_gpu
    a = ReceiverChunkMACE(model, chunk=64, device=dev, cache_layer1=True).compute(s)
    b = ReceiverChunkMACE(model, chunk=64, device=dev, cache_layer1=False).compute(s)
    assert abs(a[0] - b[0]) < 1e-9 * s.N
    assert float((a[3] - b[3]).abs().max()) < 1e-6 * float(b[3].abs().max())


@pytest.mark.parametrize("species", [(8, 1), (26,), (26, 28, 24), (26, 28, 24, 27)])
def test_ace_layer1_matches_conv_path(dev, model, species):
    """Layer 1 in the density-projection form (per-edge ht x Y on MFMA, folded atom-level GEMM) equals the
    spline-table convolution path (same interpolant: the spline of W is the spline of ht mapped by A3) for 1 to 4
    species."""
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    _say(f"case ace species={species}")
    if species == (8, 1):
        pos, box, Z = systems.water_box(64, seed=3)
    else:
        pos, box, Z = systems.fcc_alloy(n_cells=4, a=3.6, species=species)
    s = System(pos, box, Z - 1, 6.0, dev)
    s.build_neighbors()
    a = ReceiverChunkMACE(model, chunk=100, device=dev, ace_layer1=True)
    b = ReceiverChunkMACE(model, chunk=100, device=dev, ace_layer1=False)
    Ea, eata, Fa, PFa = a.compute(s)
    Eb, eatb, Fb, PFb = b.compute(s)
    assert a.fl.ace and not b.fl.ace
    dE = abs(Ea - Eb) / s.N
    dF = float((Fa - Fb).abs().max())
    _say(f"  |dE|/N {dE:.2e} max|dF| {dF:.2e} (max|F| {float(Fb.abs().max()):.2e})")
    assert dE < 1e-8 and dF < 1e-5 * float(Fb.abs().max())


def test_isolated_atoms_and_tiny_chunks(dev, model, ref_model):
    """Receivers without any neighbour (empty CSR rows) and chunks of one receiver: energies and forces still match
    the oracle (isolated atoms carry E0 + the readout of their empty-neighbourhood features and zero force)."""
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    O = np.array([[2.0, 2.0, 2.0], [4.5, 2.2, 2.5], [3.0, 4.5, 3.0], [2.5, 3.0, 5.0]])   # 4 molecules
    H = np.array([[0.757, 0.586, 0.0], [-0.757, 0.586, 0.0]])
    pos = np.concatenate([np.stack([o, o + H[0], o + H[1]]) for o in O])
    Z = np.tile([8, 1, 1], len(O))
    box = np.array([16.0, 15.0, 17.0])
    far = np.array([[11.0, 10.6, 11.6]])                      # ~10 A from every image of the cluster
    pos = np.concatenate([pos, far])
    Z = np.concatenate([Z, [8]])
    s = System(pos, box, Z - 1, 6.0, dev)
    s.build_neighbors()
    assert int((s.NN == 0).sum()) == 1
    ref = _oracle_three_pass(ref_model, s, 64)
    for chunk in (1, 7, 64):
        _say(f"case isolated atoms chunk={chunk}")
        E, eat, F, PF = ReceiverChunkMACE(model, chunk=chunk, device=dev).compute(s)
        _check(E, eat, F, ref, s.N)
        iso = (s.NN == 0).cpu()
        assert float(F.cpu()[iso].abs().max()) == 0.0


def test_fmax_guard_raises(dev, model, water_gpu, monkeypatch):
    """The non-finite / absurd-force guard (mliap_threepass.py:595-601) raises instead of handing LAMMPS the forces;
    forced from the host with a tiny MACE3P_FMAX_ABORT (every kernel still runs normally)."""
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    monkeypatch.setenv("MACE3P_FMAX_ABORT", "1e-12")
    s = water_gpu
    data = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True)
    tp = ThreePassMLIAP(model, chunk=96)
    with pytest.raises(RuntimeError, match="absurd"):
        tp.compute_forces(data)
    assert data.pair_forces is None


def test_md_chunks_from_skin_list_match_per_call_topology(dev, model):
    """The MD pair list's chunks (node lists from the skin list, built once per rebuild; local senders by one
    gather per step) give the energies and pair forces of the per-call chunk topology (chunk_topology) on the same
    filtered pairs, over several steps and a rebuild; only the fp32 atomic order differs."""
    from mace_onegpu import systems
    from mace_onegpu.md import MDRunner, _PairView
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    pos, box, Z = systems.water_box(512, seed=3)
    md = MDRunner(model, pos, box, Z, chunk=700, device=dev)             # 1536 atoms: 2 full chunks + a tail
    ref = ReceiverChunkMACE(model, chunk=700, device=dev)
    for step in range(4):
        if step == 2:
            md._build(md.pos.clone())                     # a neighbour-list rebuild: new skin list, new chunks
        md.step()
        view = _PairView(md.pairs)
        E1, eat1, F1, PF1 = md.ev.compute(view)
        view.chunk_graphs = None                          # the generic per-call topology on the same pairs
        E0, eat0, F0, PF0 = ref.compute(view)
        n_nodes = [g.n_nodes for g in md.pairs._tmpl]
        dP = float((PF1 - PF0).abs().max())
        _say(f"  step {step} (rebuilds {md.n_rebuild}): nodes {n_nodes}, |dE| {abs(E1 - E0):.2e}, max|dPF| {dP:.2e}")
        assert abs(E1 - E0) < 1e-9 * len(pos) and float((eat1 - eat0).abs().max()) < 1e-9
        assert dP <= 1e-6 * float(PF0.abs().max())
    assert md.n_rebuild >= 2


def test_md_skin_forces_match_sorted_sum(dev, model):
    """Per-atom forces of an MD step summed through the skin list's reverse-pair map (mm_pair_forces_skin) equal
    the receiver + sender-sorted sums of mm_pair_forces_to_atoms for the same pair forces."""
    from mace_onegpu import systems
    from mace_onegpu.md import MDRunner, _PairView
    from mace_onegpu.receiver_chunk_mace import pair_to_atom_forces
    pos, box, Z = systems.water_box(512, seed=2)
    md = MDRunner(model, pos, box, Z, chunk=1024, device=dev)
    md.step()
    md.step()
    view = _PairView(md.pairs)
    E, eat, F_skin, PF = md.ev.compute(view)
    view.atom_forces_fn = None
    F_sorted = pair_to_atom_forces(view, PF)
    d = float((F_skin - F_sorted).abs().max())
    _say(f"  skin vs sorted force sums: max|d| {d:.2e}")
    assert d <= 1e-12 * float(F_sorted.abs().max())

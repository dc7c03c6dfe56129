"""The species-pair table path on the GPU (marked gpu): a model with a radial network per ordered species pair
(the shape MACE-MPA-0's species-pair distance transform gives W(r), spline_radial.py:5-9, 116-151) evaluated
with one spline table per distinct network (n_tab = 3) and a non-trivial pair -> table map, through the
standalone evaluator and the ML-IAP plugin with HIP-graph chunks, against the fp64 oracle with the same per-pair
tables (fp32 rounding only) and with each edge's exact network (plus the tables' interpolation error).

The oracle's per-pair machinery is pinned in tests/test_oracle.py (equal networks reproduce the default model,
per-pair tables follow the per-edge networks, a transposed pair index is detected)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def pair_setup():
    assert torch.cuda.is_available(), "GPU test without a GPU"
    from mace_onegpu import model as mm, o3, systems
    from mace_onegpu.receiver_chunk_mace import System
    from oracle import mace_ref
    from test_oracle import _pair_networks
    m = mm.MaceModel(seed=0)
    m.pair_radial = _pair_networks(m, 5, [[(0, 0), (7, 7)], [(0, 7)], [(7, 0)]])
    rm = mace_ref.RefModel(m, o3.coupling)
    pos, box, Z = systems.water_box(64, seed=0)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    recv = np.repeat(np.arange(s.N), s.NN.cpu().numpy())
    args = (s.pos.cpu().numpy(), box, s.spidx.cpu().numpy(), recv, s.send.cpu().numpy())
    tab = mace_ref.Tables64(rm, [0, 7], n_grid=512)
    ref_tab = mace_ref.three_pass(rm, *args, chunk=96, tables=tab)
    ref_exact = mace_ref.three_pass(rm, *args, chunk=96)
    return m, s, ref_tab, ref_exact


def _check(what, E, eat, F, ref, N, rel):
    E0, e0, F0 = ref[0], ref[1], ref[2]
    dE = abs(E - E0) / N
    de = float((eat.cpu() - e0).abs().max())
    dF = float((F.cpu() - F0).abs().max())
    _say(f"  {what}: |dE|/N {dE:.2e} max|de_i| {de:.2e} max|dF| {dF:.2e} (max|F| {float(F0.abs().max()):.3e})")
    assert dE < 1e-5 and de < 1e-5 and dF < 1e-3 and dF < rel * float(F0.abs().max())


def test_pair_tables_standalone(pair_setup):
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    m, s, ref_tab, ref_exact = pair_setup
    ev = ReceiverChunkMACE(m, chunk=96, device="cuda")
    _say("case pair tables standalone, chunk 96")
    E, eat, F, PF = ev.compute(s)
    fl = ev.fl
    assert fl.n_tab == 3 and fl.pair_map.cpu().tolist() == [0, 1, 2, 0] and not fl.ace
    _check("vs oracle, same tables", E, eat, F, ref_tab, s.N, 2e-5)
    _check("vs oracle, exact networks", E, eat, F, ref_exact, s.N, 1e-4)


def test_pair_tables_mliap_graphs(pair_setup, monkeypatch):
    """ThreePassMLIAP with HIP-graph chunks (4 full chunks of 48, captured once and replayed over two calls) on the
    periodic-image data object, unsorted pairs."""
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    m, s, ref_tab, ref_exact = pair_setup
    monkeypatch.setenv("MACE3P_GRAPHS", "1")
    tp = ThreePassMLIAP(m, chunk=48)
    for call in range(2):
        _say(f"case pair tables mliap graphs call {call}")
        data = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True, shuffle_pairs_seed=3)
        tp.compute_forces(data)
        torch.cuda.synchronize()
        eat = data.eatoms
        _check("vs oracle, same tables", data.energy, eat, data.atom_forces(), ref_tab, s.N, 2e-5)
    assert tp._rt.gx is not None and tp._rt.gx.n_replays > 0 and tp._rt.fl.n_tab == 3


def test_pair_tables_md_conserves_energy(pair_setup):
    """Velocity Verlet with the per-pair model (the layer-1 convolution with 3 tables) on a 12,288-atom water box,
    50 steps of 0.5 fs from 300 K with HIP-graph chunks: E_pot + E_kin stays within 1 % of the range of E_pot
    (measured: 3.6e-3 eV against 8.8 eV)."""
    from mace_onegpu import systems
    from mace_onegpu.md import MDRunner
    m = pair_setup[0]
    pos, box, Z = systems.water_box(4096, seed=0)
    md = MDRunner(m, pos, box, Z, chunk=4096, skin=2.0, dt_fs=0.5, T=300.0, seed_v=4, device="cuda",
                  use_graphs=True)
    md.forces()
    e_pot, e_kin = [md.E], [md.kinetic()]
    for _ in range(50):
        md.step()
        e_pot.append(md.E)
        e_kin.append(md.kinetic())
    drift = float(np.ptp(np.array(e_pot) + np.array(e_kin)))
    _say(f"  pair-table MD: E_tot range {drift:.3e} eV, E_pot range {float(np.ptp(e_pot)):.3e} eV")
    assert drift < 0.01 * float(np.ptp(e_pot))

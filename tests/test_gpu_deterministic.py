"""Deterministic mode (MACE3P_DETERMINISTIC=1 / deterministic=True): the sender-feature gradient of pass B is summed
per sender in a fixed order instead of with float atomics (the reference's tl.atomic_add, conv_spline.py:175-180),
so two evaluations of the same input are bitwise identical -- energies, pair forces and G1 -- through the
standalone evaluator, the ML-IAP plugin (eager and HIP graphs) and the MD driver; and the result equals the oracle
(marked gpu)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def water():
    assert torch.cuda.is_available(), "GPU test without a GPU"
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import System
    pos, box, Z = systems.water_box(512, seed=4)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    return s


def test_standalone_is_bitwise_repeatable_and_matches_the_oracle(model, ref_model, water):
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE
    from oracle import mace_ref
    s = water
    outs = []
    for rep in range(2):
        ev = ReceiverChunkMACE(model, chunk=700, device="cuda", deterministic=True)
        E, eat, F, PF = ev.compute(s)
        outs.append((eat.clone(), PF.clone(), ev.G1.clone(), F.clone()))
    _say(f"case standalone deterministic: E {E:.10f}")
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # the default (atomic) path agrees to rounding
    E1, eat1, F1, PF1 = ReceiverChunkMACE(model, chunk=700, device="cuda").compute(s)
    assert abs(E1 - E) < 1e-9 * s.N and float((PF1 - outs[0][1]).abs().max()) < 1e-6 * float(PF1.abs().max())
    recv = np.repeat(np.arange(s.N), s.NN.cpu().numpy())
    E0, e0, F0, _, _ = mace_ref.three_pass(ref_model, s.pos.cpu().numpy(), s.box, s.spidx.cpu().numpy(), recv,
                                           s.send.cpu().numpy(), chunk=384)
    dF = float((F.cpu() - F0).abs().max())
    _say(f"  vs oracle: |dE|/N {abs(E - E0) / s.N:.2e} max|dF| {dF:.2e}")
    assert abs(E - E0) / s.N < 1e-5 and dF < 1e-4 * float(F0.abs().max())


@pytest.mark.parametrize("graphs", ["0", "1"])
def test_mliap_is_bitwise_repeatable(model, water, graphs, monkeypatch):
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    s = water
    monkeypatch.setenv("MACE3P_DETERMINISTIC", "1")
    monkeypatch.setenv("MACE3P_GRAPHS", graphs)
    tp = ThreePassMLIAP(model, chunk=512)                   # 3 full chunks of 512 receivers
    outs = []
    for call in range(3):                                   # graphs: capture, then two replays
        _say(f"case mliap deterministic graphs={graphs} call {call}")
        data = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True, shuffle_pairs_seed=7)
        tp.compute_forces(data)
        outs.append((data.eatoms.clone(), data.pair_forces.clone()))
    for rep in outs[1:]:
        assert torch.equal(rep[0], outs[0][0]) and torch.equal(rep[1], outs[0][1])
    if graphs == "1":
        assert tp._rt.gx is not None and tp._rt.gx.n_replays > 0


@pytest.mark.parametrize("graphs", [False, True])
def test_md_trajectory_is_bitwise_repeatable(model, graphs):
    """Eager, and with HIP graphs: chunk 512 gives 3 full chunks of the 1,536 atoms, captured once and replayed with
    the persistent MD chunk objects (their sender CSR reloaded into the graph slots on every step)."""
    from mace_onegpu import systems
    from mace_onegpu.md import MDRunner
    pos, box, Z = systems.water_box(512, seed=6)
    runs = []
    for rep in range(2):
        _say(f"case md deterministic graphs={graphs} run {rep}")
        md = MDRunner(model, pos, box, Z, chunk=512 if graphs else 700, device="cuda", deterministic=True,
                      use_graphs=graphs)
        for _ in range(4):
            md.step()
        if graphs:
            gx = md.ev._gx
            assert gx is not None and gx.n_replays > 0
        runs.append((md.pos.clone(), md.vel.clone(), md.E))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1]) and runs[0][2] == runs[1][2]

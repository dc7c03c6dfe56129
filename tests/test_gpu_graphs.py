"""HIP-graph execution of full chunks (chunk_graphs.ChunkGraphExec) against the eager path, on the GPU.

Every replay is checked against the eager result, with eager work and synchronisations between the replays (the
graphs are replayed for several chunks and over several calls).  The two paths run the same kernels; only the
order of pass B's fp32 atomic additions differs, so energies agree to 1e-9 eV/atom and pair forces to 1e-6 of
their maximum.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def water_sys():
    assert torch.cuda.is_available(), "GPU test without a GPU"
    from mace_onegpu import systems
    from mace_onegpu.receiver_chunk_mace import System
    pos, box, Z = systems.water_box(64, seed=0)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    return s


def _close(E, PF, eat, E0, PF0, eat0, N, what):
    dE = abs(E - E0) / N
    de = float((eat - eat0).abs().max())
    dP = float((PF - PF0).abs().max())
    _say(f"  {what}: |dE|/N {dE:.2e} max|de_i| {de:.2e} max|dPF| {dP:.2e} (max|PF| {float(PF0.abs().max()):.2e})")
    assert dE < 1e-9 and de < 1e-9
    assert dP <= 1e-6 * float(PF0.abs().max())


@pytest.mark.parametrize("cache_l1", ["1", "0"])
def test_mliap_graphs_match_eager(model, water_sys, cache_l1, monkeypatch):
    """ThreePassMLIAP with MACE3P_GRAPHS=1: 4 full chunks of 48 receivers (graph replays) over 3 calls,
    interleaved with eager calls, each equal to the eager result."""
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    s = water_sys
    monkeypatch.setenv("MACE3P_CACHE_L1", cache_l1)
    monkeypatch.setenv("MACE3P_GRAPHS", "0")
    eager = ThreePassMLIAP(model, chunk=48)
    monkeypatch.setenv("MACE3P_GRAPHS", "1")
    graphed = ThreePassMLIAP(model, chunk=48)
    for call in range(3):
        _say(f"case mliap graphs cache_l1={cache_l1} call {call}")
        shuffle = call if call else None          # calls 1 and 2: unsorted pair lists (same for both paths)
        d0 = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True, shuffle_pairs_seed=shuffle)
        eager.compute_forces(d0)
        torch.cuda.synchronize()
        d1 = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True, shuffle_pairs_seed=shuffle)
        graphed.compute_forces(d1)
        torch.cuda.synchronize()
        assert graphed._rt.gx is not None and graphed._rt.gx.n_replays == 12 * (call + 1)
        _close(d1.energy, d1.pair_forces, d1.eatoms, d0.energy, d0.pair_forces, d0.eatoms, s.N, f"call {call}")
    assert graphed.n_captures == 1


def test_mliap_graphs_recapture_when_a_call_outgrows_them(model, water_sys, monkeypatch):
    """A call whose chunks and ghost count exceed the captured capacities (no headroom: margin 1.0, edge capacity
    aligned to 256) recaptures once; a smaller call after it replays the larger graphs.  Every call equals the eager
    evaluation of the same input."""
    from mace_onegpu import systems
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    from mace_onegpu.receiver_chunk_mace import System
    pos, box, Z = systems.water_box(512, seed=2)
    big = System(pos, box, Z - 1, 6.0, "cuda")
    big.build_neighbors()
    monkeypatch.setenv("MACE3P_CAP_MARGIN", "1.0")
    monkeypatch.setenv("MACE3P_GRAPHS", "0")
    eager = ThreePassMLIAP(model, chunk=48, e_align=256)
    monkeypatch.setenv("MACE3P_GRAPHS", "1")
    graphed = ThreePassMLIAP(model, chunk=48, e_align=256)
    captures = []
    for call, s in enumerate((water_sys, big, water_sys)):
        _say(f"case mliap graphs recapture call {call}: {s.N} atoms")
        d0 = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True)
        eager.compute_forces(d0)
        torch.cuda.synchronize()
        d1 = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True)
        graphed.compute_forces(d1)
        torch.cuda.synchronize()
        captures.append(graphed.n_captures)
        _close(d1.energy, d1.pair_forces, d1.eatoms, d0.energy, d0.pair_forces, d0.eatoms, s.N, f"call {call}")
    assert captures == [1, 2, 2]


def test_standalone_graphs_match_eager(model, water_sys):
    """ReceiverChunkMACE(use_graphs=True): 3 full chunks of 64 receivers, two calls, and a translated copy of the
    box (same capacities, new positions) -- every call equal to the eager evaluation of the same input."""
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    s = water_sys
    ev0 = ReceiverChunkMACE(model, chunk=64, device="cuda")
    ev1 = ReceiverChunkMACE(model, chunk=64, device="cuda", use_graphs=True)
    shifted = System(s.pos.cpu().numpy() + np.array([0.4, -0.2, 1.1]), s.box, s.spidx.cpu().numpy(), 6.0, "cuda")
    shifted.build_neighbors()
    for call, sysm in enumerate((s, s, shifted)):
        _say(f"case standalone graphs call {call}")
        E0, eat0, F0, PF0 = ev0.compute(sysm)
        torch.cuda.synchronize()
        E1, eat1, F1, PF1 = ev1.compute(sysm)
        torch.cuda.synchronize()
        _close(E1, PF1, eat1, E0, PF0, eat0, s.N, f"call {call}")
    assert ev1.n_captures == 1 and ev1._gx.n_replays == 27
    # an eager call of the same evaluator runs on the executor's static rows and workspace (no second set of H1,
    # G1, layer-1 cache rows and chunk buffers) and still equals the eager evaluator; a graph call after it is
    # unaffected
    ev1.use_graphs = False
    E2, eat2, F2, PF2 = ev1.compute(s)
    assert ev1.H1.data_ptr() == ev1._gx.H1x.data_ptr() and ev1.G1.data_ptr() == ev1._gx.G1.data_ptr()
    assert ev1.fl.ws is ev1._gx.ws                                 # and its workspace
    E0, eat0, F0, PF0 = ev0.compute(s)
    _close(E2, PF2, eat2, E0, PF0, eat0, s.N, "eager call on the executor's rows")
    ev1.use_graphs = True
    E3, eat3, F3, PF3 = ev1.compute(s)
    _close(E3, PF3, eat3, E0, PF0, eat0, s.N, "graph call after it")
    assert ev1.n_captures == 1


def test_md_with_graphs_matches_eager(model):
    """Five MD steps with graphed force calls follow the eager trajectory (positions within 1e-9 A)."""
    from mace_onegpu import systems
    from mace_onegpu.md import MDRunner
    pos, box, Z = systems.water_box(512, seed=1)
    _say("case md graphs")
    a = MDRunner(model, pos, box, Z, chunk=512, device="cuda")
    b = MDRunner(model, pos, box, Z, chunk=512, device="cuda", use_graphs=True)
    for step in range(5):
        a.step()
        b.step()
        dx = float((a.pos - b.pos).abs().max())
        _say(f"  step {step}: E {a.E:.8f} / {b.E:.8f}, max|dx| {dx:.2e}")
        assert abs(a.E - b.E) < 1e-9 * len(pos)
        assert dx < 1e-9
    assert b.ev.n_captures >= 1 and b.ev._gx.n_replays > 0


def test_mliap_call_log_fields(model, water_sys, tmp_path, monkeypatch):
    """MACE3P_LOG: one JSON line per call with the reference's fields (mliap_threepass.py:433-441, 606-616): sizes,
    chunks, captures, e_cap, the phase times, peak_out (peak device GB of this call) and peak_gb (running max); a
    capture line precedes the first graphed call."""
    import json

    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    s = water_sys
    log = tmp_path / "m3p.jsonl"
    monkeypatch.setenv("MACE3P_LOG", str(log))
    monkeypatch.setenv("MACE3P_GRAPHS", "1")
    tp = ThreePassMLIAP(model, chunk=48)
    for call in range(2):
        _say(f"case mliap log call {call}")
        tp.compute_forces(PeriodicMLIAPData(s, s.spidx.long(), ghosts=True))
    tp._rt.log.flush()
    lines = [json.loads(x) for x in log.read_text().splitlines()]
    calls = [x for x in lines if "step" in x]
    assert "capture" in lines[0] and len(calls) == 2
    for c in calls:
        assert c["nlocal"] == s.N and c["chunks"] == 4 and c["graphs"] and c["captures"] == 1
        assert c["e_cap"] >= max(1, int(s.rowptr[-1]) // 4)
        assert {"A", "B", "C", "t_total"} <= set(c)
        assert 0 < c["peak_out"] <= c["peak_gb"]
    assert calls[1]["peak_gb"] == max(calls[0]["peak_gb"], calls[1]["peak_out"])

"""The command-line entry points on the GPU (marked gpu), called in-process: the evaluator's replica check and JSON
record, the evaluator on a structure file against ReceiverChunkMACE on the same atoms, and the MD driver."""
import json

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_evaluator_replica_check_and_record(tmp_path):
    """python -m mace_onegpu.receiver_chunk_mace --water 64 --rep 3 2 1 --check-replica --graphs --repeat 2: every
    atom of the 1,152-atom replica (a box of 3 x 2 x 1 base cells: cell grids of three different lengths) has its
    base image's force and energy (fp32 arithmetic in other orders), and the record holds both runs."""
    from mace_onegpu.receiver_chunk_mace import main
    assert torch.cuda.is_available(), "GPU test without a GPU"
    out = tmp_path / "r.json"
    res = main(["--water", "64", "--rep", "3", "2", "1", "--chunk", "256", "--graphs", "--repeat", "2",
                "--check-replica", "--json", str(out)])
    rc = res["replica_check"]
    assert res["N"] == 1152 and res["pairs"] > 0 and len(res["runs"]) == 2
    assert rc["max_dF"] < 1e-5 * rc["max_F"] and rc["max_de"] < 1e-6 and abs(rc["dE_per_atom"]) < 1e-9
    assert res["runs"][0]["energy"] == pytest.approx(res["runs"][1]["energy"], abs=1e-9)
    assert json.loads(out.read_text())["replica_check"] == rc


def test_evaluator_on_a_structure_file(tmp_path):
    """An extended-XYZ file read by the command line gives ReceiverChunkMACE's energy on the same atoms."""
    from mace_onegpu import model as mm, systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System, main
    pos, box, Z = systems.water_box(64, seed=5)
    f = tmp_path / "w.xyz"
    r = lambda v: repr(float(v))
    f.write_text("\n".join([str(len(pos)), f'Lattice="{r(box[0])} 0 0 0 {r(box[1])} 0 0 0 {r(box[2])}"']
                           + [f"{systems.SYMBOLS[z - 1]} {r(x)} {r(y)} {r(w)}" for z, (x, y, w) in zip(Z, pos)])
                 + "\n")
    res = main(["--structure", str(f), "--chunk", "96"])
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    E = ReceiverChunkMACE(mm.MaceModel(seed=0), chunk=96, device="cuda").compute(s)[0]
    assert res["runs"][0]["energy"] == pytest.approx(E, abs=1e-9)
    # the reference's memory layout and the deterministic mode give the same energy
    for flags in (["--low-memory"], ["--deterministic"]):
        r2 = main(["--structure", str(f), "--chunk", "96"] + flags)
        assert r2["runs"][0]["energy"] == pytest.approx(E, abs=1e-9), flags


def test_md_command_line(tmp_path):
    """python -m mace_onegpu.md --water 512 --steps 20: the record's throughput and energy drift (1,536 atoms,
    chunks of 512 replayed from HIP graphs)."""
    from mace_onegpu.md import main
    out = tmp_path / "md.json"
    res = main(["--water", "512", "--seed", "1", "--steps", "20", "--chunk", "512", "--graphs", "--every", "10",
                "--json", str(out)])
    assert res["N"] == 1536 and res["steps"] == 20 and res["atom_step_per_s"] > 0
    assert res["E_tot_range"] < 1e-3 * res["E_kin"]
    assert json.loads(out.read_text())["E_tot_range"] == res["E_tot_range"]
    assert np.isfinite(res["E_pot"])

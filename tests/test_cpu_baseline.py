"""The fp32 CPU restatement that bench.py times as its CPU baseline (oracle/cpu_fp32.py) computes the three-pass
energies and forces: it equals the fp64 oracle with the same 512-knot tables to fp32 rounding (CPU only)."""
import numpy as np
import torch

from oracle import cpu_fp32, mace_ref


def test_fp32_restatement_matches_fp64_oracle(ref_model, water192):
    w = water192
    cols = sorted(set(w["spec"].tolist()))
    t64 = mace_ref.Tables64(ref_model, cols, n_grid=512)
    E0, e0, F0, _, _ = mace_ref.three_pass(ref_model, w["pos"], w["box"], w["spec"], w["recv"], w["send"], chunk=96,
                                           tables=t64)
    E, eat, F = cpu_fp32.three_pass(ref_model.astype(torch.float32), t64.astype(torch.float32), w["pos"], w["box"],
                                    w["spec"], w["recv"], w["send"], chunk=48)
    n = len(w["pos"])
    assert abs(E - E0) / n < 1e-6
    assert float((eat - e0).abs().max()) < 1e-5
    assert float((F - F0).abs().max()) < 2e-5 * float(F0.abs().max())


def test_chunk_timing_runs_one_chunk(ref_model, water192):
    w = water192
    cols = sorted(set(w["spec"].tolist()))
    t32 = mace_ref.Tables64(ref_model, cols, n_grid=512).astype(torch.float32)
    rowptr = np.concatenate([[0], np.cumsum(w["NN"])])
    r = cpu_fp32.chunk_timing(ref_model.astype(torch.float32), t32, w["pos"], w["box"], w["spec"], rowptr,
                              w["send"], 64, 128, sub=32)
    assert r["receivers"] == 64 and r["edges"] == int(rowptr[128] - rowptr[64])
    assert all(r[k] > 0 for k in ("topology", "A", "B", "C"))

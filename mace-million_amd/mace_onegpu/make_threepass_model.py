"""Writes the LAMMPS ML-IAP model file of the three-pass evaluator (scripts/make_threepass_model.py of the
reference, :1-46):

    python -m mace_onegpu.make_threepass_model --out mace3p.pt [--seed 0 | --weights state.safetensors]
        [--chunk 16384] [--spline-grid 512] [--recipe]

The file is a pickled mace_onegpu.mliap_threepass.ThreePassMLIAP holding the fp32 model (the MACE-MPA-0-medium
architecture of mace_onegpu.model, random-init from --seed or loaded from a state_dict in safetensors / a
weights-only torch file).  Device tables, kernel constants and HIP graphs are rebuilt inside LAMMPS on the first
force call.  With --recipe the file stores (class, constructor kwargs, state_dict) instead of the module object.
LAMMPS needs mace-million_amd/ on PYTHONPATH to unpickle it:

    pair_style  mliap unified mace3p.pt 0
    pair_coeff  * * O H
"""
import argparse

import torch

from .mliap_threepass import ThreePassMLIAP
from .model import MaceModel, MaceSpec, load_weights


def make(out, seed=0, weights=None, chunk=16384, spline_grid=512, recipe=False):
    spec = MaceSpec()
    model = MaceModel(spec, seed=seed)
    if weights:
        load_weights(model, weights)
    cfg = dict(spec=spec, seed=seed) if recipe else None
    obj = ThreePassMLIAP(model.float(), chunk=chunk, spline_grid=spline_grid, rebuild_config=cfg)
    torch.save(obj, out)
    return obj


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", required=True)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--weights", default=None)
    ap.add_argument("--chunk", type=int, default=16384)
    ap.add_argument("--spline-grid", type=int, default=512)
    ap.add_argument("--recipe", action="store_true")
    a = ap.parse_args(argv)
    obj = make(a.out, a.seed, a.weights, a.chunk, a.spline_grid, a.recipe)
    print(f"saved {a.out}: chunk={obj.chunk} spline_grid={obj.spline_grid} dtype={obj.dtype} "
          f"elements={len(obj.element_types)} recipe={obj._rebuild is not None}")


if __name__ == "__main__":
    main()

"""The ML-IAP model file (mace_onegpu.make_threepass_model): pickled by module path, runtime state dropped, the
rebuild recipe reconstructs the same weights (reference behaviour: mliap_threepass.py:155-202,
scripts/make_threepass_model.py)."""
import pickle

import pytest
import torch

from mace_onegpu import make_threepass_model
from mace_onegpu.mliap_threepass import ThreePassMLIAP


def _same_weights(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    return sa.keys() == sb.keys() and all(torch.equal(sa[k], sb[k]) for k in sa)


def test_model_file_roundtrip(tmp_path):
    out = tmp_path / "m3p.pt"
    obj = make_threepass_model.make(str(out), seed=0, chunk=4096, spline_grid=256)
    # the file was written by this test: a full unpickle is what LAMMPS does with it
    back = torch.load(str(out), weights_only=False)
    assert type(back) is ThreePassMLIAP and type(back).__module__ == "mace_onegpu.mliap_threepass"
    assert back.element_types[:8] == ["H", "He", "Li", "Be", "B", "C", "N", "O"] and back.num_species == 89
    assert back.rcutfac == 3.0 and back.ndescriptors == 1 and back.nparams == 1
    assert (back.chunk, back.spline_grid, back.node_bucket, back.e_align) == (4096, 256, 8192, 65536)
    assert back.dtype == torch.float32
    assert _same_weights(back.model, obj.model)


def test_runtime_state_is_not_pickled():
    obj = ThreePassMLIAP(make_threepass_model.MaceModel(seed=1))
    obj._rt, obj.last_timings = object(), {"A": 1.0}
    d = obj.__getstate__()
    assert not {"_rt", "last_timings"} & set(d)
    back = pickle.loads(pickle.dumps(obj))
    assert back._rt is None and back.last_timings is None and _same_weights(back.model, obj.model)


def test_rebuild_recipe(tmp_path):
    out = tmp_path / "m3pr.pt"
    obj = make_threepass_model.make(str(out), seed=3, recipe=True)
    back = torch.load(str(out), weights_only=False)
    assert "model" not in back.__dict__ and back._rebuild is not None
    assert _same_weights(back._rebuild_model(), obj.model)


@pytest.mark.parametrize("key", ["_rebuild", "_recipe"])
def test_recipe_state_layouts(key):
    """A state dict with the recipe under the reference's `_rebuild` (mliap_threepass.py:173-184), or under the
    `_recipe` key an earlier file layout used, and no model: the model is rebuilt and the object pickles again."""
    src = make_threepass_model.MaceModel(seed=5)
    obj = ThreePassMLIAP(src, rebuild_config=dict(seed=5))
    state = obj.__getstate__()
    assert "model" not in state and state["_rebuild"] is not None
    state[key] = state.pop("_rebuild")
    back = ThreePassMLIAP.__new__(ThreePassMLIAP)
    back.__setstate__(state)
    assert back._rebuild is not None and "_recipe" not in back.__dict__
    assert _same_weights(back._rebuild_model(), src)
    again = pickle.loads(pickle.dumps(back))
    assert "model" not in again.__dict__ and _same_weights(again._rebuild_model(), src)


def test_missing_model_and_recipe_raises():
    obj = ThreePassMLIAP(make_threepass_model.MaceModel(seed=2))
    state = obj.__getstate__()
    state.pop("model")
    back = ThreePassMLIAP.__new__(ThreePassMLIAP)
    back.__setstate__(state)
    with pytest.raises(RuntimeError, match="neither the model nor a rebuild recipe"):
        back._rebuild_model()


def test_weights_file(tmp_path):
    from safetensors.torch import save_file
    src = make_threepass_model.MaceModel(seed=7)
    w = tmp_path / "w.safetensors"
    save_file({k: v.contiguous() for k, v in src.state_dict().items()}, str(w))
    obj = make_threepass_model.make(str(tmp_path / "m.pt"), seed=0, weights=str(w))
    assert _same_weights(obj.model, src)


@pytest.mark.gpu
def test_model_file_computes_forces(tmp_path):
    """A model file written with a rebuild recipe, unpickled, evaluates the same energies and pair forces as the
    object it was written from."""
    from mace_onegpu import systems
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.receiver_chunk_mace import System
    assert torch.cuda.is_available(), "GPU test without a GPU"
    pos, box, Z = systems.water_box(64, seed=0)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    obj = make_threepass_model.make(str(tmp_path / "m.pt"), seed=0, chunk=96, recipe=True)
    back = torch.load(str(tmp_path / "m.pt"), weights_only=False)
    d0, d1 = (PeriodicMLIAPData(s, s.spidx.long(), ghosts=True) for _ in range(2))
    obj.compute_forces(d0)
    back.compute_forces(d1)
    print(f"case model file: E {d0.energy:.10f} / {d1.energy:.10f}", flush=True)
    assert abs(d0.energy - d1.energy) < 1e-9 * s.N
    assert float((d0.pair_forces - d1.pair_forces).abs().max()) <= 1e-6 * float(d0.pair_forces.abs().max())

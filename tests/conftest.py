import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "mace-million_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


@pytest.fixture(scope="session")
def model():
    from mace_onegpu import model as mm
    return mm.MaceModel(seed=0)


@pytest.fixture(scope="session")
def ref_model(model):
    from mace_onegpu import o3
    from oracle import mace_ref
    return mace_ref.RefModel(model, o3.coupling)


@pytest.fixture(scope="session")
def water192():
    """64-molecule water box of the build's generator, Morton-sorted with its neighbour list (oracle)."""
    import numpy as np
    from mace_onegpu import systems
    from oracle import neighbors
    pos, box, Z = systems.water_box(64, seed=0)
    s = neighbors.SystemRef(pos, box, Z - 1, 6.0)
    NN, rp, send = s.build_neighbors()
    recv = np.repeat(np.arange(s.N), NN)
    return dict(pos=s.pos, box=box, spec=s.spidx, recv=recv, send=send, NN=NN, raw=(pos, box, Z), sys=s)


@pytest.fixture(scope="session")
def water_config5():
    """Configuration 5's water box (343,000 molecules, 1,029,000 atoms, L = 217.30 A, seed 0), host arrays
    (pos fp64 [N, 3], box [3], Z [N]); generated once per session (about 13 s)."""
    from mace_onegpu import systems
    print("case config5 water box: generating 343,000 molecules", flush=True)
    return systems.water_box(343000, seed=0)

"""Host-side behaviour of the ML-IAP boundary that needs no GPU: early returns, the int32 neighbour-slot guard and
the int32 column split of the ghost exchange (reference mliap_threepass.py:40-55, 444-461)."""
import pytest
import torch

from mace_onegpu import mliap_threepass
from mace_onegpu.mliap_threepass import ThreePassMLIAP, exchange_in_column_blocks


class _Data:
    """Minimal ML-IAP data object: only what compute_forces reads before it touches the device."""

    def __init__(self, nlocal, ntotal, npairs):
        self.nlocal, self.ntotal, self.npairs = nlocal, ntotal, npairs
        self.elems = torch.zeros(ntotal, dtype=torch.int64)
        self.touched = False

    def update_pair_forces_gpu(self, PF):
        self.touched = True


@pytest.fixture(scope="module")
def plugin(model):
    return ThreePassMLIAP(model, chunk=64)


@pytest.mark.parametrize("nl,P", [(0, 100), (10, 0), (10, 1)])
def test_early_return(plugin, nl, P):
    """nlocal == 0 or npairs <= 1: nothing is computed and nothing is written (mliap_threepass.py:446-447)."""
    d = _Data(nl, nl, P)
    assert plugin.compute_forces(d) is None
    assert not d.touched and plugin.step == 0


def test_int32_slot_guard(plugin, monkeypatch):
    """An estimated LAMMPS neighbour-slot count near 2^31 raises before any work (mliap_threepass.py:450-461);
    MACE3P_ALLOW_HUGE=1 lifts the guard (it then needs the GPU, so only the raising side is run here)."""
    monkeypatch.setenv("MACE3P_SKIN", "2.0")
    P = int(0.95 * 2 ** 31 / (8.0 / 6.0) ** 3) + 10
    with pytest.raises(RuntimeError, match="int32"):
        plugin.compute_forces(_Data(1000, 1000, P))
    monkeypatch.setenv("MACE3P_SKIN", "0.0")           # the same pair count passes the guard without a skin
    est = P * ((6.0 + 0.0) / 6.0) ** 3
    assert est <= 0.95 * 2 ** 31


def test_exchange_column_split(monkeypatch):
    """ntotal * D >= 2^31 elements: the exchange is called on column blocks that each stay below the limit,
    and the blocks reassemble the full result."""
    monkeypatch.setattr(mliap_threepass, "INT32_ELEMENTS", 1000)
    calls = []

    def fn(src, dst, D):
        assert src.shape[0] * D < 1000 and src.is_contiguous() and dst.shape == src.shape
        calls.append(D)
        dst.copy_(2 * src)

    src = torch.arange(40 * 64, dtype=torch.float32).view(40, 64)
    dst = torch.empty_like(src)
    exchange_in_column_blocks(fn, src, dst, 64)
    assert torch.equal(dst, 2 * src)
    assert len(calls) > 1 and sum(calls) == 64
    calls.clear()
    small = torch.ones(3, 8)
    out = torch.empty_like(small)
    exchange_in_column_blocks(fn, small, out, 8)                       # below the limit: one call on the whole array
    assert calls == [8] and torch.equal(out, 2 * small)


def test_pickle_drops_runtime_state(model):
    import pickle
    tp = ThreePassMLIAP(model, chunk=32)
    tp._rt = object()                                  # stands in for the device runtime of a used plugin
    back = pickle.loads(pickle.dumps(tp))
    assert back._rt is None and back.step == 0
    assert back.chunk == 32 and back.rcutfac == 0.5 * model.spec.r_max

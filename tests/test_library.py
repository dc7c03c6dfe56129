"""The C-ABI library builds for gfx950 and exports every symbol that include/mace_million_amd.h declares (no
compute calls: no GPU here); the generated kernel sources are what the committed generator writes."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mace_million_amd.h")
LIB = os.path.join(ROOT, "mace-million_amd", "lib", "libmace_million_amd.so")


def declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(mm_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_the_binding():
    from mace_onegpu import _lib
    assert set(declared()) == set(_lib.SIGNATURES)


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (python mace-million_amd/build.py)")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [s for s in declared() if not hasattr(lib, s)]
    assert not missing, missing
    from mace_onegpu import _lib
    assert lib.mm_version() == _lib.ABI_VERSION


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (python mace-million_amd/build.py)")
def test_binding_refuses_a_library_of_other_conventions(monkeypatch):
    """A library whose argument conventions differ from the binding's (an older build given newer buffer layouts)
    is refused when it is loaded, before any kernel can read a buffer with the wrong layout."""
    from mace_onegpu import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", _lib.ABI_VERSION + 1)
    with pytest.raises(RuntimeError, match="argument conventions version"):
        _lib.lib()
    monkeypatch.undo()
    assert _lib.lib().mm_version() == _lib.ABI_VERSION


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (python mace-million_amd/build.py)")
def test_binding_refuses_host_tensors():
    """A CPU tensor handed to a kernel entry point is refused before the call (its address is not device memory;
    the ABI's HOST arrays are ctypes objects, not tensors)."""
    import torch

    from mace_onegpu._lib import K
    x = torch.zeros(16)
    with pytest.raises(TypeError, match="argument 0 is a cpu tensor"):
        K.mm_fill_f32(x, 16, 1.0, None)
    assert not x.any()


def test_generated_sources_are_current(tmp_path):
    from mace_onegpu import codegen, model
    codegen.generate(str(tmp_path), model.Tables(model.MaceSpec()))
    gen = os.path.join(ROOT, "mace-million_amd", "csrc", "gen")
    for f in os.listdir(tmp_path):
        assert open(tmp_path / f).read() == open(os.path.join(gen, f)).read(), f


def test_codegen_term_coverage():
    """Every TP term appears exactly once per channel of a lane in the generated forward kernels (layer 2: two
    channels per lane, accumulators acc<o>a / acc<o>b; layer 1: one)."""
    from mace_onegpu import model
    t = model.Tables(model.MaceSpec())
    gen = os.path.join(ROOT, "mace-million_amd", "csrc", "gen")
    fwd2 = open(os.path.join(gen, "conv_l2.hip")).read().split("mm_conv2_bwd_kernel")[0]
    for sfx in "ab":
        assert len(re.findall(r"acc\d+" + sfx + r" = fmaf\(", fwd2)) == len(t.tp2["terms"])
    fwd1 = open(os.path.join(gen, "conv_l1.hip")).read().split("mm_conv1_bwd_kernel")[0]
    assert len(re.findall(r"acc\d+ = fmaf\(", fwd1)) == len(t.tp1["terms"])


def test_codegen_rejects_a_batch_that_is_not_a_power_of_two():
    """The forward's per-edge batch is found with masks: 48 would mix two batches' rows (results wrong, no fault)."""
    from mace_onegpu import codegen, model
    t = model.Tables(model.MaceSpec())
    for yb in (48, 128, 2):
        with pytest.raises(ValueError, match="power of two"):
            codegen.conv_source(t.tp2, 2, True, {"ybatch": yb})
    assert "yf_all[4 * 480]" in codegen.conv_source(t.tp2, 2, True, {"ybatch": 32})
    with pytest.raises(ValueError, match="cpl"):
        codegen.conv_source(t.tp2, 2, True, {"cpl": 3})


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (python mace-million_amd/build.py)")
def test_readout1_refuses_half_gradient_mode():
    """mm_readout1 computes energies only when g1r and gh are both null and the gradient when both are given; one
    without the other is refused on the host with MM_EINVAL before any launch (the pointers are never read)."""
    from mace_onegpu import _lib
    so = _lib.lib()
    fake = ctypes.c_void_p(0x1000)      # never dereferenced: the argument check returns first
    null = ctypes.c_void_p(0)
    for g1r, gh in ((null, fake), (fake, null)):
        rc = so.mm_readout1(4, fake, 512, fake, 1.0, fake, g1r, 512, gh, 512, 512, null)
        assert rc == -1
        assert "g1r and gh" in _lib.last_error()

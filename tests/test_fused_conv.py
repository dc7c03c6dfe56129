"""FusedConvTP (explicit per-edge weights): descriptor and API checks on the CPU; forward and autograd backward of
the HIP kernels against the fp64 CPU oracle (oracle.mace_ref.channelwise_tp + scatter_sum) on the GPU, for the
library's compiled tables and for tables whose kernels are built at run time (mace_onegpu.tp_jit).

Tolerance (fp32 kernels vs fp64 oracle, sums of <= 353 terms over <= 40 edges): max|d| <= 2e-5 * max|ref|.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from mace_onegpu import o3, tp_jit
from mace_onegpu.fused_conv import ChannelwiseTP, FusedConvTP

C = 128


def test_descriptor_sizes():
    # widths of the reference's two interaction blocks (D = 512 / 1280 weights, 2048 / 5120 mid) and of the
    # full l<=3 table (16 node-feature components)
    d1, d2, d3 = ChannelwiseTP([0]), ChannelwiseTP([0, 1]), ChannelwiseTP([0, 1, 2, 3])
    assert (d1.nX, d1.nW, d1.nO, len(d1.table["terms"]), d1.weight_numel) == (1, 4, 16, 16, 512)
    assert (d2.nX, d2.nW, d2.nO, len(d2.table["terms"]), d2.weight_numel) == (4, 10, 40, 86, 1280)
    assert (d3.nX, d3.nW, d3.nO, len(d3.table["terms"])) == (16, 23, 99, 353)
    assert (d1.name, d2.name, d3.name) == ("l1", "l2", "l0123")


def test_module_api_errors():
    d = ChannelwiseTP([0, 1])
    with pytest.raises(ValueError):
        FusedConvTP(d, 1000)
    with pytest.raises(TypeError):
        FusedConvTP(object(), 1280)
    m = FusedConvTP(d, 1280, irreps_out="128x0e+128x1o")
    assert m.weight_numel == 1280 and m.irreps_out == "128x0e+128x1o"
    with pytest.raises(NotImplementedError):
        ChannelwiseTP([0, 1], sh_lmax=4).kernels()         # the kernels take harmonics up to l = 3
    assert "built on first use" in repr(ChannelwiseTP([0, 2]))


def test_descriptor_from_irreps_strings():
    """The irreps strings of a MACE interaction block (what the reference's path_table reads) give the same
    descriptor as the l lists; multiplicities other than the kernels' and pseudo-parities are refused."""
    d = ChannelwiseTP.from_irreps("128x0e+128x1o", "1x0e+1x1o+1x2e+1x3o", "128x0e+128x1o+128x2e+128x3o")
    assert (d.in_ls, d.sh_lmax, d.target_ls, d.name) == ((0, 1), 3, (0, 1, 2, 3), "l2")
    d = ChannelwiseTP.from_irreps("128x0e", "0e+1o+2e", "128x0e + 128x2e")
    assert (d.in_ls, d.sh_lmax, d.target_ls, d.nY) == ((0,), 2, (0, 2), 9)
    with pytest.raises(ValueError, match="128 per irrep"):
        ChannelwiseTP.from_irreps("64x0e", "1x0e", "128x0e")
    with pytest.raises(NotImplementedError, match="parity"):
        ChannelwiseTP.from_irreps("128x1e", "1x0e+1x1o", "128x0e")
    with pytest.raises(ValueError, match="l = 0 .. L"):
        ChannelwiseTP.from_irreps("128x0e", "1x0e+1x2e", "128x0e")
    with pytest.raises(ValueError, match="cannot read"):
        ChannelwiseTP.from_irreps("128x0y", "1x0e", "128x0e")


def test_run_time_tables_are_prebuilt_and_export_their_entry_points():
    """The build makes the kernels of o3.PREBUILT_JIT_TP_TABLES ahead, from this tree's sources; their libraries
    load without a GPU and export both entry points under the table's name."""
    for a, b, c in o3.PREBUILT_JIT_TP_TABLES:
        desc = ChannelwiseTP(a, b, c)
        assert desc.name is None
        assert tp_jit.is_current(desc.table), f"{desc} not built: run __graft_entry__.build()"
        fwd, bwd = desc.kernels()
        name = tp_jit.paths(desc.table)[0]
        assert (fwd.name, bwd.name) == (f"mm_tpw_{name}_fwd", f"mm_tpw_{name}_bwd")
        assert desc.kernels()[0] is fwd                       # loaded once per process


def test_run_time_kernels_report_their_own_errors():
    """An argument error of a run-time library's entry point is raised with that library's message (its own
    mm_last_error), checked on the host before anything reaches the GPU."""
    desc = ChannelwiseTP(*o3.PREBUILT_JIT_TP_TABLES[0])
    fwd, bwd = desc.kernels()
    with pytest.raises(RuntimeError, match="row strides smaller than the path table's widths"):
        fwd(None, 1, None, None, None, 8, None, desc.nW * C, None, desc.nX * C, None, desc.nO * C, None)
    with pytest.raises(RuntimeError, match="bad sizes"):
        bwd(None, -1, None, None, None, 16, None, desc.nW * C, None, desc.nX * C, None, desc.nO * C, None, 0, None, 0,
            None, 0, None)


def test_run_time_build_of_a_new_table(tmp_path, monkeypatch):
    """A table nobody built before: its kernels are generated and compiled on first use (into a scratch directory
    here), a second request reuses the library, and a library whose recorded source differs is rebuilt."""
    monkeypatch.setattr(tp_jit, "JIT_DIR", str(tmp_path))
    t = o3.tp_table([0, 1, 2], 3, (0, 1, 2))
    assert not tp_jit.is_current(t)
    so = tp_jit.build(t)
    assert tp_jit.is_current(t) and os.path.dirname(so) == str(tmp_path)
    m0 = os.stat(so).st_mtime_ns
    assert tp_jit.build(t) == so and os.stat(so).st_mtime_ns == m0
    lib = ctypes.CDLL(so)
    name = tp_jit.paths(t)[0]
    for kind in ("fwd", "bwd"):
        assert getattr(lib, f"mm_tpw_{name}_{kind}")
    hip = tp_jit.paths(t)[1]
    with open(hip, "a") as fh:
        fh.write("// edited\n")
    assert not tp_jit.is_current(t)
    tp_jit.build(t)
    assert tp_jit.is_current(t)
    assert sorted(os.listdir(tmp_path)) == sorted(os.path.basename(p) for p in tp_jit.paths(t)[1:])


@pytest.mark.parametrize("tab", list(o3.PREBUILT_JIT_TP_TABLES) + [((0, 1, 2), 3, (0, 1, 2))])
def test_sparse_table_matches_the_dense_oracle(tab):
    """The kernels evaluate the table's sparse terms (w, k, m, o, coef); the oracle contracts the dense coupling
    tensor of each path.  Both on the CPU in fp64 for a table without a compiled kernel: a wrong component offset,
    path order or dropped term of the table fails this."""
    from oracle import mace_ref
    t = o3.tp_table(list(tab[0]), tab[1], tab[2])
    g = np.random.default_rng(3)
    E, Cc = 7, 3
    W, X, Y = g.normal(size=(E, t["nW"], Cc)), g.normal(size=(E, t["nX"], Cc)), g.normal(size=(E, t["nY"]))
    out = np.zeros((E, t["nO"], Cc))
    for (w, k, m, o, c) in t["terms"]:
        out[:, o] += c * W[:, w] * X[:, k] * Y[:, m, None]
    ref = mace_ref.channelwise_tp(torch.from_numpy(W), torch.from_numpy(X), torch.from_numpy(Y), torch.arange(E),
                                  t["paths"], t["in_ls"], o3.coupling)
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)


def _oracle(desc, X, Y, W, ei, n):
    from oracle import mace_ref
    t = desc.table
    E = W.shape[0]
    mid = mace_ref.channelwise_tp(W.reshape(E, desc.nW, C), X.reshape(n, desc.nX, C), Y, ei[0], t["paths"],
                                  t["in_ls"], o3.coupling)
    return mace_ref.scatter_sum(mid, ei[1], n).reshape(n, desc.nO * C)


def _inputs(desc, n, E, seed, sort):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n, desc.nX * C, generator=g, dtype=torch.float64)
    Y = torch.randn(E, desc.nY, generator=g, dtype=torch.float64)
    W = torch.randn(E, desc.nW * C, generator=g, dtype=torch.float64)
    send = torch.randint(0, n, (E,), generator=g)
    recv = torch.randint(0, n - 3, (E,), generator=g)      # the last 3 nodes receive nothing
    if sort:
        recv = torch.sort(recv).values
    return X, Y, W, torch.stack([send, recv])


def _check(desc, seed, sort):
    assert torch.cuda.is_available(), "GPU test without a GPU"
    n, E = 37, 400
    X, Y, W, ei = _inputs(desc, n, E, seed=seed, sort=sort)
    print(f"case {desc} sorted={sort} n={n} E={E}", flush=True)
    Xr, Yr, Wr = (t.clone().requires_grad_(True) for t in (X, Y, W))
    ref = _oracle(desc, Xr, Yr, Wr, ei, n)
    R = torch.randn(ref.shape, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    gX0, gY0, gW0 = torch.autograd.grad((ref * R).sum(), [Xr, Yr, Wr])
    m = FusedConvTP(desc, desc.weight_numel)
    Xd, Yd, Wd = (t.float().cuda().requires_grad_(True) for t in (X, Y, W))
    out = m(Xd, Yd, Wd, ei.cuda())
    gX, gY, gW = torch.autograd.grad((out * R.float().cuda()).sum(), [Xd, Yd, Wd])
    for name, a, b in (("out", out, ref), ("gX", gX, gX0), ("gY", gY, gY0), ("gW", gW, gW0)):
        a, b = a.detach().double().cpu(), b.detach()
        err, scale = float((a - b).abs().max()), float(b.abs().max())
        print(f"  {name}: max|d| {err:.3e} (max|ref| {scale:.3e})", flush=True)
        assert err <= 2e-5 * scale, name
    assert float(out.detach()[n - 3:].abs().max()) == 0.0       # rows of nodes without edges


@pytest.mark.gpu
@pytest.mark.parametrize("in_ls", [[0], [0, 1], [0, 1, 2, 3]])
@pytest.mark.parametrize("sort", [False, True])
def test_fused_conv_forward_backward(in_ls, sort):
    _check(ChannelwiseTP(in_ls), len(in_ls) * 7 + int(sort), sort)


@pytest.mark.gpu
@pytest.mark.parametrize("tab", o3.PREBUILT_JIT_TP_TABLES)
@pytest.mark.parametrize("sort", [False, True])
def test_fused_conv_run_time_tables(tab, sort):
    """Tables whose kernels are built at run time (made ahead by the build, so nothing compiles here)."""
    desc = ChannelwiseTP(*tab)
    assert desc.name is None and tp_jit.is_current(desc.table)
    _check(desc, 100 + len(tab[0]) * 7 + len(tab[2]) + int(sort), sort)


@pytest.mark.gpu
def test_fused_conv_bounds_checked_on_host():
    desc = ChannelwiseTP([0, 1])
    m = FusedConvTP(desc, desc.weight_numel)
    X = torch.zeros(5, desc.nX * C, device="cuda")
    Y = torch.zeros(3, 16, device="cuda")
    W = torch.zeros(3, desc.weight_numel, device="cuda")
    with pytest.raises(IndexError):
        m(X, Y, W, torch.tensor([[0, 1, 5], [0, 1, 2]], device="cuda"))
    with pytest.raises(IndexError):
        m(X, Y, W, torch.tensor([[0, 1, 2], [0, 1, -1]], device="cuda"))
    with pytest.raises(TypeError):
        m(X.double(), Y, W, torch.tensor([[0, 1, 2], [0, 1, 2]], device="cuda"))
    out = m(X, Y[:0], W[:0], torch.zeros(2, 0, dtype=torch.long, device="cuda"))
    assert out.shape == (5, desc.nO * C) and float(out.abs().max()) == 0.0


@pytest.mark.gpu
def test_fused_conv_fewer_harmonics_shapes():
    """A table with harmonics up to l = 2 takes [E, 9] edge attributes (padded to the kernels' 16 inside) and returns
    a [E, 9] gradient for them, also with no edges; 16 columns are refused for it."""
    desc = ChannelwiseTP((0, 1), 2, (0, 1, 2))
    assert desc.nY == 9 and tp_jit.is_current(desc.table)
    m = FusedConvTP(desc, desc.weight_numel)
    X = torch.randn(5, desc.nX * C, device="cuda", requires_grad=True)
    for E in (0, 3):
        Y = torch.randn(E, 9, device="cuda", requires_grad=True)
        W = torch.randn(E, desc.weight_numel, device="cuda", requires_grad=True)
        ei = torch.tensor([[0, 1, 4], [0, 2, 2]], device="cuda")[:, :E]
        out = m(X, Y, W, ei)
        gX, gY, gW = torch.autograd.grad(out.sum(), [X, Y, W])
        assert out.shape == (5, desc.nO * C) and gY.shape == (E, 9) and gW.shape == W.shape
    with pytest.raises(ValueError):
        m(X, torch.zeros(3, 16, device="cuda"), torch.zeros(3, desc.weight_numel, device="cuda"), ei)

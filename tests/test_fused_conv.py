"""FusedConvTP (explicit per-edge weights): descriptor and API checks on the CPU; forward and autograd backward of
the HIP kernels against the fp64 CPU oracle (oracle.mace_ref.channelwise_tp + scatter_sum) on the GPU.

Tolerance (fp32 kernels vs fp64 oracle, sums of <= 353 terms over <= 40 edges): max|d| <= 2e-5 * max|ref|.
"""
import pytest
import torch

from mace_onegpu import o3
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
        ChannelwiseTP([0, 2]).require_kernel()


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
    Y = torch.randn(E, 16, generator=g, dtype=torch.float64)
    W = torch.randn(E, desc.nW * C, generator=g, dtype=torch.float64)
    send = torch.randint(0, n, (E,), generator=g)
    recv = torch.randint(0, n - 3, (E,), generator=g)      # the last 3 nodes receive nothing
    if sort:
        recv = torch.sort(recv).values
    return X, Y, W, torch.stack([send, recv])


@pytest.mark.gpu
@pytest.mark.parametrize("in_ls", [[0], [0, 1], [0, 1, 2, 3]])
@pytest.mark.parametrize("sort", [False, True])
def test_fused_conv_forward_backward(in_ls, sort):
    assert torch.cuda.is_available(), "GPU test without a GPU"
    desc = ChannelwiseTP(in_ls)
    n, E = 37, 400
    X, Y, W, ei = _inputs(desc, n, E, seed=len(in_ls) * 7 + int(sort), sort=sort)
    print(f"case in_ls={in_ls} sorted={sort} n={n} E={E}", flush=True)
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

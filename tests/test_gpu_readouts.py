"""GPU tests: the readout kernels (mm_readout1, mm_readout2) against the oracle's readout blocks with fp64 autograd.

The reference's readouts are mace's LinearReadoutBlock (layer 1) and NonLinearReadoutBlock (layer 2), applied per
atom in every pass (fast_layers.py:200-214, mliap_threepass.py:550, 578, 589); oracle.mace_ref.readout_linear and
readout_mlp restate them.  The kernels take the weights pre-divided (w0 / sqrt(C), W1 / sqrt(C), w2 / sqrt(H)) and
the silu normalisation as an argument; the references below get the same fp32 values undivided again.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
C = 128


@pytest.mark.parametrize("n,H,stride", [(1, 16, 128), (63, 16, 128), (64, 1, 132), (65, 32, 128), (1000, 7, 256)])
def test_readout2_against_oracle(n, H, stride):
    """eat += scale R2(h2) and g_h2 = scale dR2/dh2 for node counts around the kernel's 64-node workgroups, hidden
    widths 1..32 and rows wider than the 128 features (the columns past them are left alone)."""
    from mace_onegpu._lib import K, stream
    from oracle import mace_ref
    assert torch.cuda.is_available(), "GPU test without a GPU"
    print(f"case n={n} H={H} stride={stride}", flush=True)
    g = torch.Generator().manual_seed(100 * n + H)
    h = torch.randn(n, stride, generator=g).float()
    W1k = (torch.randn(C, H, generator=g, dtype=torch.float64) / math.sqrt(C)).float()
    w2k = (torch.randn(H, generator=g, dtype=torch.float64) / math.sqrt(H)).float()
    eat0 = torch.randn(n, generator=g, dtype=torch.float64)
    scale, cst = 0.7, mace_ref.silu_norm()
    x = h[:, :C].double().requires_grad_()
    R = mace_ref.readout_mlp(x, W1k.double() * math.sqrt(C), w2k.double() * math.sqrt(H))
    (gx,) = torch.autograd.grad(scale * R.sum(), x)
    R = R.detach()
    eat = eat0.cuda()
    gh = torch.full((n, stride), float("nan"), device="cuda")
    K.mm_readout2(n, h.cuda(), stride, W1k.contiguous().cuda(), w2k.cuda(), H, cst, scale, eat, gh, stride, stream())
    torch.cuda.synchronize()
    eat, gh = eat.cpu(), gh.cpu().double()
    ref = eat0 + scale * R
    err_e = float((eat - ref).abs().max())
    err_g = float((gh[:, :C] - gx).abs().max())
    print(f"  energy max|err| {err_e:.2e} (max|R| {float(R.abs().max()):.2e}); gradient max|err| {err_g:.2e} "
          f"(max {float(gx.abs().max()):.2e})", flush=True)
    assert err_e <= 2e-6 * (1 + float(R.abs().max()))
    assert err_g <= 2e-6 * (1 + float(gx.abs().max()))
    assert bool(gh[:, C:].isnan().all())


@pytest.mark.parametrize("n,D,grad", [(1, 512, True), (5, 512, False), (257, 192, True), (64, 128, True)])
def test_readout1_against_oracle(n, D, grad):
    """eat += scale R1(h1) and, with a gradient row, g_h1 = G1r + scale dR1/dh1 (the 0e block only), for row widths
    that are and are not multiples of the wave's 64 lanes."""
    from mace_onegpu._lib import K, stream
    from oracle import mace_ref
    assert torch.cuda.is_available(), "GPU test without a GPU"
    print(f"case n={n} D={D} gradient={grad}", flush=True)
    g = torch.Generator().manual_seed(7 * n + D)
    h = torch.randn(n, D, generator=g).float()
    w0k = (torch.randn(C, generator=g, dtype=torch.float64) / math.sqrt(C)).float()
    G1r = torch.randn(n, D, generator=g).float()
    eat0 = torch.randn(n, generator=g, dtype=torch.float64)
    scale = 1.3
    R = mace_ref.readout_linear(h[:, :C].double(), w0k.double() * math.sqrt(C))
    eat = eat0.cuda()
    gh = torch.full((n, D), float("nan"), device="cuda")
    if grad:
        K.mm_readout1(n, h.cuda(), D, w0k.cuda(), scale, eat, G1r.cuda(), D, gh, D, D, stream())
    else:
        K.mm_readout1(n, h.cuda(), D, w0k.cuda(), scale, eat, None, 0, None, 0, D, stream())
    torch.cuda.synchronize()
    eat, gh = eat.cpu(), gh.cpu().double()
    err_e = float((eat - (eat0 + scale * R)).abs().max())
    print(f"  energy max|err| {err_e:.2e} (max|R| {float(R.abs().max()):.2e})", flush=True)
    assert err_e <= 2e-6 * (1 + float(R.abs().max()))
    if grad:
        ref = G1r.double().clone()
        ref[:, :C] += scale * w0k.double()
        assert float((gh - ref).abs().max()) <= 1e-6 * (1 + float(ref.abs().max()))
    else:
        assert bool(gh.isnan().all())


def test_readout_argument_checks():
    """Host-side checks: hidden width beyond 32 and a row narrower than the 128 features are refused; no nodes is a
    no-op."""
    from mace_onegpu._lib import K, stream
    assert torch.cuda.is_available(), "GPU test without a GPU"
    h = torch.zeros(4, C, device="cuda")
    eat = torch.zeros(4, dtype=torch.float64, device="cuda")
    W1 = torch.zeros(C * 33, device="cuda")
    with pytest.raises(RuntimeError):
        K.mm_readout2(4, h, C, W1, torch.zeros(33, device="cuda"), 33, 1.0, 1.0, eat, h, C, stream())
    with pytest.raises(RuntimeError):
        K.mm_readout1(4, h, C, torch.zeros(C, device="cuda"), 1.0, eat, None, 0, None, 0, 64, stream())
    K.mm_readout2(0, h, C, W1, torch.zeros(16, device="cuda"), 16, 1.0, 1.0, eat, h, C, stream())
    torch.cuda.synchronize()
    assert float(eat.abs().max()) == 0.0

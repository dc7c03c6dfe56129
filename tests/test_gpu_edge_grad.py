"""mm_edge_grad called through the C ABI on random partials, against fp64 autograd (marked gpu).

Semantics checked (the autograd step torch.autograd.grad(..., [vec]) of mliap_threepass.py:550, 580, applied to the
convolution backward's per-edge partials): with g = sum over the channel blocks of part[cb][e][0..16],
    gr = g[0] + g_rho[recv(e)] * dd(e),   L_e(v) = gr |v| + sum_m g[1 + m] Y_m(v / |v|),
    pf[e] = dL_e/dv at v = r u   (pf[e] += ... when accumulating).
Both channel-block counts of the production calls are covered (8 for layer 2, 1 for ACE layer 1).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_part,accumulate", [(8, 0), (1, 1), (5, 0)])
def test_edge_grad_against_fp64_autograd(n_part, accumulate):
    from mace_onegpu._lib import K, stream
    from oracle import mace_ref
    assert torch.cuda.is_available(), "GPU test without a GPU"
    g = torch.Generator().manual_seed(n_part * 10 + accumulate)
    E, nC = 1000, 37
    print(f"case n_part={n_part} accumulate={accumulate}: {E} edges", flush=True)
    u = torch.randn(E, 3, generator=g, dtype=torch.float64)
    u /= u.norm(dim=1, keepdim=True)
    r = 0.8 + 5.2 * torch.rand(E, generator=g, dtype=torch.float64)
    part = torch.randn(n_part, E, 17, generator=g, dtype=torch.float64)
    g_rho = torch.randn(nC, generator=g, dtype=torch.float64)
    recv = torch.randint(0, nC, (E,), generator=g)
    dd = torch.randn(E, generator=g, dtype=torch.float64)
    pf0 = torch.randn(E, 3, generator=g, dtype=torch.float64)

    # fp64 reference on the fp32 values the kernel reads
    f = lambda t: t.float().double()
    gs = f(part).sum(0)
    gr = gs[:, 0] + f(g_rho)[recv] * f(dd)
    v = (f(u) * f(r)[:, None]).requires_grad_()
    n = v.norm(dim=1)
    L = (gr * n).sum() + (gs[:, 1:] * mace_ref.sh(v / n[:, None])).sum()
    (ref,) = torch.autograd.grad(L, v)
    if accumulate:
        ref = ref + f(pf0)

    dev = "cuda"
    eu = torch.empty(E, 4, dtype=torch.float32, device=dev)
    eu[:, :3] = u.float().to(dev)
    eu[:, 3] = r.float().to(dev)
    pd = part.float().to(dev).contiguous()
    pf = pf0.float().to(dev).contiguous() if accumulate else torch.full((E, 3), float("nan"), device=dev)
    K.mm_edge_grad(E, None, pd, E * 17, n_part, g_rho.float().to(dev), recv.to(torch.int32).to(dev),
                   dd.float().to(dev), eu, pf, accumulate, stream())
    torch.cuda.synchronize()
    got = pf.double().cpu()
    err = float((got - ref).abs().max())
    scale = float(ref.abs().max())
    print(f"  pf: max|err| {err:.3e} (max|ref| {scale:.3e})", flush=True)
    assert torch.isfinite(got).all() and err <= 1e-5 * scale

    # the edge count from device memory (graph replays): a launch sized for E processes only the first E_dev edges
    E_real = E - 357
    pf2 = pf0.float().to(dev).contiguous() if accumulate else torch.full((E, 3), float("nan"), device=dev)
    before = pf2.clone()
    K.mm_edge_grad(E, torch.tensor([E_real], dtype=torch.int32, device=dev), pd, E * 17, n_part,
                   g_rho.float().to(dev), recv.to(torch.int32).to(dev), dd.float().to(dev), eu, pf2, accumulate,
                   stream())
    torch.cuda.synchronize()
    assert torch.equal(pf2[:E_real], pf[:E_real])                       # the same kernel arithmetic
    assert torch.equal(pf2[E_real:].isnan(), before[E_real:].isnan())   # nothing beyond E_dev written
    assert torch.equal(torch.nan_to_num(pf2[E_real:]), torch.nan_to_num(before[E_real:]))

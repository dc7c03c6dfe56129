"""The symmetric-contraction kernels (mm_symc{1,2}_fwd, mm_symc{1,2}_bwd) called through the C ABI on random node
features, against the fp64 restatement in the oracle with autograd (marked gpu).

Semantics checked (mace SymmetricContraction, correlation 3; the reference's capture-safe copy of the product
block, graphed_three_pass.py:41-62):
    out[n, L-block, c] = sum_nu sum_paths W[species(n), path, c] P_path(x[n, :, c])
    gx = (d out / d x)^T gout,   g_rho[n] = -sum_{comp, c} x gx / (rho[n] + 1)
(x is the density-normalised message, so g_rho is dL/drho).  Layer 1 maps 0e+1o+2e+3o to 0e+1o, layer 2 to 0e.
Node counts are odd, so the last two-node block of the kernels is half full.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

C = 128


@pytest.mark.parametrize("Z", [(1, 8), (26, 28, 24, 27)])
@pytest.mark.parametrize("layer", [1, 2])
def test_symc_kernels_against_fp64_autograd(model, ref_model, Z, layer):
    from mace_onegpu._lib import K, stream
    from mace_onegpu.fast_layers import FastLayers
    from oracle import mace_ref
    assert torch.cuda.is_available(), "GPU test without a GPU"
    cols = [z - 1 for z in Z]
    fl = FastLayers(model, cols, device="cuda")
    S, n = len(cols), 203
    g = torch.Generator().manual_seed(layer * 10 + S)
    x = torch.randn(n, 16, C, generator=g, dtype=torch.float64)
    spec = torch.randint(0, S, (n,), generator=g)
    rho = torch.rand(n, generator=g, dtype=torch.float64) * 30.0
    out_ls = [0, 1] if layer == 1 else [0]
    n_out = 4 if layer == 1 else 1
    gout = torch.randn(n, n_out, C, generator=g, dtype=torch.float64)
    print(f"case layer {layer} species {Z}: {n} nodes", flush=True)

    # fp64 reference on the fp32 values the kernels read
    xr = x.float().double().requires_grad_()
    Wts = ref_model.sym_weights(layer - 1, tuple(out_ls))
    paths = ref_model.sc1 if layer == 1 else ref_model.sc2
    sp_cols = torch.as_tensor(cols)[spec]
    out_r = mace_ref.symmetric_contraction(xr, sp_cols, Wts, paths, out_ls, [0, 1, 2, 3], ref_model.coupling)
    (out_r * gout.float().double()).sum().backward()
    gx_r = xr.grad
    grho_r = -(xr.detach() * gx_r).sum((1, 2)) / (rho.float().double() + 1.0)

    dev = dict(device="cuda")
    xd = x.float().reshape(n, 16 * C).to(**dev).contiguous()
    sd = spec.to(torch.int32).to(**dev)
    Wsc = fl.Wsc1 if layer == 1 else fl.Wsc2
    out = torch.full((n, n_out * C), float("nan"), **dev)
    go = gout.float().reshape(n, n_out * C).to(**dev).contiguous()
    gx = torch.full((n, 16 * C), float("nan"), **dev)
    rd = rho.float().to(**dev)
    grho = torch.full((n,), float("nan"), **dev)
    fwd, bwd = (K.mm_symc1_fwd, K.mm_symc1_bwd) if layer == 1 else (K.mm_symc2_fwd, K.mm_symc2_bwd)
    fwd(n, xd, 16 * C, sd, Wsc, out, n_out * C, stream())
    bwd(n, xd, 16 * C, sd, Wsc, go, n_out * C, gx, 16 * C, rd, grho, stream())
    torch.cuda.synchronize()

    def close(name, got, ref, rel):
        got = got.double().cpu()
        err = float((got - ref).abs().max())
        scale = float(ref.abs().max())
        print(f"  {name}: max|err| {err:.3e} (max|ref| {scale:.3e})", flush=True)
        assert torch.isfinite(got).all() and err <= rel * scale

    close("out", out.view(n, n_out, C), out_r.detach(), 1e-5)
    close("dL/dx", gx.view(n, 16, C), gx_r, 1e-5)
    close("dL/drho", grho, grho_r, 1e-5)

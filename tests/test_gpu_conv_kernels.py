"""The layer-2 edge-convolution kernels (mm_conv2_fwd, mm_conv2_bwd) called through the C ABI on synthetic
receiver-CSR inputs, against an fp64 autograd restatement of the channelwise tensor product (marked gpu).

Semantics checked (reference kernels K1/K2, conv_spline.py:38-94, 97-181):
    W[e, w, c]   = a0 + t (a1 + t (a2 + t a3)),   (a0..a3) = table row of edge e, path w, channel c
    out[i, o, c] = sum_{e: recv(e) = i} sum_terms coef W[e, w, c] X[send(e), k, c] Y[e, m]
    rho[i]       = sum_{e: recv(e) = i} density(e)
and, for L = sum gA * out: dL/dX, dL/dY[e, m] and inv_h * dL/dt[e] (the last two summed over the 8 channel
blocks of the per-edge partials).

The cases drive every path of the backward's accumulation of dL/dX per group of 4 receivers:
- receivers without edges;
- a last group of fewer than 4 receivers;
- groups whose distinct senders exceed the LDS slots;
- groups with more edges than the per-group edge cap;
- and local groups that share most senders.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

C = 128


def _terms():
    from mace_onegpu import model as mm
    return mm.Tables(mm.MaceSpec()).tp2


def _case(seed, nC, n_nodes, deg_max, local, NR=9, degrees=None):
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, deg_max + 1, nC) if degrees is None else rng.choice(degrees, nC)
    deg[::7] = 0
    send = []
    for i in range(nC):
        if local:      # senders in a window around the receiver: neighbouring receivers share them
            c0 = int(i * n_nodes / nC)
            lo, hi = max(0, c0 - 80), min(n_nodes, c0 + 80)
        else:          # senders anywhere: a group's distinct senders overflow the LDS slots
            lo, hi = 0, n_nodes
        d = min(int(deg[i]), hi - lo)
        deg[i] = d
        send.append(rng.choice(np.arange(lo, hi), d, replace=False))
    send = np.concatenate(send).astype(np.int32)
    rowptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    E = len(send)
    u = rng.normal(size=(E, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    r = rng.uniform(0.8, 6.0, E)
    t = rng.uniform(0.0, 1.0, E)
    row = rng.integers(0, NR, E)
    dens = rng.uniform(0.0, 1.0, E)
    X = rng.normal(size=(n_nodes, 4 * C))
    tab = rng.normal(size=(8, NR, 10, 16, 4)) * np.array([1.0, 0.5, 0.25, 0.125])
    gA = rng.normal(size=(nC, 40 * C))
    return dict(rowptr=rowptr, send=send, u=u, r=r, t=t, row=row, dens=dens, X=X, tab=tab, gA=gA, NR=NR)


def _reference(cs, tp):
    """fp64 forward and autograd backward on the CPU."""
    from oracle import mace_ref
    f64 = dict(dtype=torch.float64)
    E = len(cs["send"])
    nC = len(cs["rowptr"]) - 1
    recv = torch.repeat_interleave(torch.arange(nC), torch.from_numpy(np.diff(cs["rowptr"])).long())
    send = torch.from_numpy(cs["send"]).long()
    tab = torch.tensor(cs["tab"], **f64).float().double()          # the fp32 table values the kernel reads
    tabc = tab.permute(1, 2, 0, 3, 4).reshape(cs["NR"], 10, C, 4)  # [row, w, c, coef]
    t = torch.tensor(cs["t"], **f64).float().double().requires_grad_()
    Y = mace_ref.sh(torch.tensor(cs["u"], **f64).float().double()).detach().requires_grad_()
    X = torch.tensor(cs["X"], **f64).float().double().view(-1, 4, C).requires_grad_()
    a = tabc[torch.from_numpy(cs["row"]).long()]                    # [E, w, c, 4]
    tt = t[:, None, None]
    W = a[..., 0] + tt * (a[..., 1] + tt * (a[..., 2] + tt * a[..., 3]))
    Xs = X[send]                                                    # [E, k, c]
    by_o = {}
    for (w, k, m, o, coef) in tp["terms"]:
        by_o.setdefault(o, []).append((w, k, m, coef))
    zero = torch.zeros(E, C, **f64)
    msg = torch.stack([sum((coef * W[:, w] * Xs[:, k] * Y[:, m:m + 1] for (w, k, m, coef) in by_o[o]), zero)
                       if o in by_o else zero for o in range(40)], 1)
    out = torch.zeros(nC, 40, C, **f64).index_add(0, recv, msg)
    rho = torch.zeros(nC, **f64).index_add(0, recv, torch.tensor(cs["dens"], **f64).float().double())
    gA = torch.tensor(cs["gA"], **f64).float().double().view(nC, 40, C)
    (out * gA).sum().backward()
    return out.detach(), rho, X.grad.reshape(-1, 4 * C), Y.grad, t.grad


@pytest.mark.parametrize("name,nC,n_nodes,deg_max,local,degrees", [
    ("local", 203, 1500, 120, True, None),        # 203 = 50 groups of 4 + a group of 3
    ("scattered", 97, 4000, 240, False, None),    # distinct senders per group > slots; edges per group > cap
    ("sparse", 61, 300, 6, False, None),          # few edges, many empty receivers
    # receivers at and around the forward's 64-edge batches of harmonic factors
    ("batch_edges", 67, 1200, 0, False, [1, 3, 4, 5, 63, 64, 65, 127, 128, 129, 192]),
    # receivers with degrees around multiples of the 4-edge steps and 16-edge groups, in a local sender window
    ("tile_edges", 71, 900, 0, True, [1, 2, 15, 16, 17, 31, 32, 33, 48, 90]),
])
def test_conv2_kernels_against_fp64_autograd(name, nC, n_nodes, deg_max, local, degrees):
    from mace_onegpu._lib import K, stream
    assert torch.cuda.is_available(), "GPU test without a GPU"
    tp = _terms()
    cs = _case(7, nC, n_nodes, deg_max, local, degrees=degrees)
    E = len(cs["send"])
    print(f"case {name}: nC {nC} nodes {n_nodes} edges {E}", flush=True)
    dev = "cuda"
    f32 = dict(dtype=torch.float32, device=dev)
    pk = torch.empty(E, 4, **f32)
    pk[:, 0] = torch.tensor(cs["t"], **f32)
    pk[:, 3] = torch.tensor(cs["dens"], **f32)
    pki = pk.view(torch.int32)
    pki[:, 1] = torch.tensor(cs["row"], dtype=torch.int32, device=dev)
    pki[:, 2] = torch.tensor(cs["send"], dtype=torch.int32, device=dev)
    eu = torch.empty(E, 4, **f32)
    eu[:, :3] = torch.tensor(cs["u"], **f32)
    eu[:, 3] = torch.tensor(cs["r"], **f32)
    rowptr = torch.tensor(cs["rowptr"], dtype=torch.int32, device=dev)
    X = torch.tensor(cs["X"], **f32)
    tab = torch.tensor(cs["tab"], **f32).contiguous()
    gA = torch.tensor(cs["gA"], **f32)
    out = torch.full((nC, 40 * C), float("nan"), **f32)
    rho = torch.full((nC,), float("nan"), **f32)
    inv_h = 3.0
    part = torch.full((8, E * 17 + 5), float("nan"), **f32)
    gX = torch.zeros(n_nodes, 4 * C, **f32)
    M = cs["NR"] + 1
    K.mm_conv2_fwd(rowptr, nC, pk, eu, X, 4 * C, tab, 1, M, out, rho, stream())
    K.mm_conv2_bwd(rowptr, nC, pk, eu, X, 4 * C, tab, 1, M, inv_h, gA, part, E * 17 + 5, gX, stream())
    torch.cuda.synchronize()
    out_r, rho_r, gX_r, gY_r, gt_r = _reference(cs, tp)

    def close(name, got, ref, rel):
        got = got.double().cpu()
        err = float((got - ref).abs().max())
        scale = float(ref.abs().max())
        print(f"  {name}: max|err| {err:.3e} (max|ref| {scale:.3e})", flush=True)
        assert torch.isfinite(got).all() and err <= rel * scale + 1e-12

    # fp32 sums of at most a few thousand products against fp64: 1e-5 of the largest value (an indexing or
    # race error is of the order of the values themselves)
    close("out", out.view(nC, 40, C), out_r, 1e-5)
    close("rho", rho, rho_r, 1e-5)
    # dL/dX comes in 16-channel-block-major rows, gX[s][cb][k][16] = dL/dX[s, k, 16 cb + j]
    def comp_major(g):
        return g.view(-1, 8, 4, 16).permute(0, 2, 1, 3).reshape(-1, 4 * C)

    close("gX", comp_major(gX), gX_r, 1e-5)
    p = part[:, :E * 17].view(8, E, 17).double().sum(0).cpu()
    close("dL/dY", p[:, 1:], gY_r, 1e-5)
    close("inv_h dL/dt", p[:, 0], inv_h * gt_r, 1e-5)
    assert torch.isnan(part[:, E * 17:]).all()      # nothing written past the partials

    # the deterministic variant: per-edge dL/dX rows summed per sender in ascending edge order
    from mace_onegpu.fast_layers import sender_csr
    from mace_onegpu.receiver_chunk_mace import ChunkGraph
    g = ChunkGraph()
    g.ls, g.nE, g.n_nodes = torch.tensor(cs["send"], dtype=torch.int32, device=dev), E, n_nodes
    srp, sperm = sender_csr(g)
    results = []
    for rep in range(2):
        part2 = torch.full((8, E * 17 + 5), float("nan"), **f32)
        gXe = torch.full((max(E, 1), 4 * C), float("nan"), **f32)
        gX2 = torch.full((n_nodes, 4 * C), float("nan"), **f32)
        K.mm_conv2_bwd_det(rowptr, nC, pk, eu, X, 4 * C, tab, 1, M, inv_h, gA, part2, E * 17 + 5, gXe, stream())
        K.mm_gather_rows_csr(srp, sperm, gXe, 4 * C, 4 * C, gX2, 4 * C, n_nodes, stream())
        torch.cuda.synchronize()
        results.append((part2.clone(), gX2.clone()))
    close("gX (deterministic)", comp_major(gX2), gX_r, 1e-5)
    assert torch.equal(results[0][1], results[1][1])                # bitwise repeatable
    assert torch.equal(results[0][0][:, :E * 17], results[1][0][:, :E * 17])
    p2 = results[0][0][:, :E * 17].view(8, E, 17).double().sum(0).cpu()
    close("dL/dY (deterministic)", p2[:, 1:], gY_r, 1e-5)
    close("inv_h dL/dt (deterministic)", p2[:, 0], inv_h * gt_r, 1e-5)


def test_conv0123_kernels_against_oracle_tp():
    """mm_conv0123_fwd / _bwd (literal 0e+1o+2e+3o node features: 23 paths, 353 terms, the benchmark's V3 shape)
    against the oracle's dense channelwise TP (mace_ref.channelwise_tp over the coupling tensors, independent of
    the generated term list) with W from the same interval coefficients in fp64, and fp64 autograd for dL/dX,
    dL/dY and inv_h dL/dt (the latter two summed over the kernel's partial rows)."""
    from mace_onegpu import codegen, o3
    from mace_onegpu._lib import K, stream
    from oracle import mace_ref
    assert torch.cuda.is_available(), "GPU test without a GPU"
    t3 = codegen.tpw_tables()["l0123"]
    nX, nW, nO = t3["nX"], t3["nW"], t3["nO"]
    parts = codegen.tpw_layout(t3)["parts"]
    rng = np.random.default_rng(11)
    nC, n_nodes, NR = 45, 300, 7
    deg = rng.choice([0, 1, 2, 3, 17, 40, 65], nC)
    send = np.concatenate([rng.choice(n_nodes, d, replace=False) for d in deg]).astype(np.int32)
    rowptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    E = len(send)
    print(f"case conv0123: nC {nC} nodes {n_nodes} edges {E} parts {parts}", flush=True)
    u = rng.normal(size=(E, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    tt, row = rng.uniform(0, 1, E), rng.integers(0, NR, E)
    dens = rng.uniform(0, 1, E)
    X = rng.normal(size=(n_nodes, nX * C))
    tab = rng.normal(size=(8, NR, nW, 16, 4)) * np.array([1.0, 0.5, 0.25, 0.125])
    gA = rng.normal(size=(nC, nO * C))
    dev = "cuda"
    f32 = dict(dtype=torch.float32, device=dev)
    pk = torch.empty(E, 4, **f32)
    pk[:, 0], pk[:, 3] = torch.tensor(tt, **f32), torch.tensor(dens, **f32)
    pk.view(torch.int32)[:, 1] = torch.tensor(row, dtype=torch.int32, device=dev)
    pk.view(torch.int32)[:, 2] = torch.tensor(send, dtype=torch.int32, device=dev)
    eu = torch.empty(E, 4, **f32)
    eu[:, :3], eu[:, 3] = torch.tensor(u, **f32), 1.0
    rp = torch.tensor(rowptr, dtype=torch.int32, device=dev)
    Xd, tabd, gAd = torch.tensor(X, **f32), torch.tensor(tab, **f32).contiguous(), torch.tensor(gA, **f32)
    out = torch.full((nC, nO * C), float("nan"), **f32)
    rho = torch.full((nC,), float("nan"), **f32)
    part = torch.full((parts, E * 17 + 3), float("nan"), **f32)
    gX = torch.zeros(n_nodes, nX * C, **f32)
    inv_h = 2.5
    K.mm_conv0123_fwd(rp, nC, pk, eu, Xd, nX * C, tabd, 1, NR + 1, out, rho, stream())
    K.mm_conv0123_bwd(rp, nC, pk, eu, Xd, nX * C, tabd, 1, NR + 1, inv_h, gAd, part, E * 17 + 3, gX, stream())
    torch.cuda.synchronize()
    f64 = dict(dtype=torch.float64)
    tabc = torch.tensor(tab, **f64).float().double().permute(1, 2, 0, 3, 4).reshape(NR, nW, C, 4)
    a = tabc[torch.from_numpy(row).long()]
    t = torch.tensor(tt, **f64).float().double().requires_grad_()
    tq = t[:, None, None]
    W = a[..., 0] + tq * (a[..., 1] + tq * (a[..., 2] + tq * a[..., 3]))
    Y = mace_ref.sh(torch.tensor(u, **f64).float().double()).detach().requires_grad_()
    Xr = torch.tensor(X, **f64).float().double().view(n_nodes, nX, C).requires_grad_()
    recv = torch.repeat_interleave(torch.arange(nC), torch.from_numpy(deg).long())
    mid = mace_ref.channelwise_tp(W, Xr, Y, torch.from_numpy(send).long(), t3["paths"], t3["in_ls"], o3.coupling)
    ref = mace_ref.scatter_sum(mid, recv, nC)
    G = torch.tensor(gA, **f64).float().double().view(nC, nO, C)
    (ref * G).sum().backward()
    rho_r = torch.zeros(nC, **f64).index_add(0, recv, torch.tensor(dens, **f64).float().double())

    def close(name, got, want, rel):
        got = got.double().cpu()
        err, scale = float((got - want).abs().max()), float(want.abs().max())
        print(f"  {name}: max|err| {err:.3e} (max|ref| {scale:.3e})", flush=True)
        assert torch.isfinite(got).all() and err <= rel * scale + 1e-12

    close("out", out.view(nC, nO, C), ref.detach(), 1e-5)
    close("rho", rho, rho_r, 1e-5)
    close("gX", gX.view(n_nodes, nX, C), Xr.grad, 1e-5)
    p = part[:, :E * 17].view(parts, E, 17).double().sum(0).cpu()
    close("dL/dY", p[:, 1:], Y.grad, 1e-5)
    close("inv_h dL/dt", p[:, 0], inv_h * t.grad, 1e-5)
    assert torch.isnan(part[:, E * 17:]).all()

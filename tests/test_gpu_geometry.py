"""mm_edge_geom_rij called through the C ABI on random pair vectors, against the fp64 oracle (marked gpu).

Semantics checked (fast_layers.py:154-156, 179-183, 190-192; spline_w._coords, spline_w.py:18-27):
    e_u[e]  = (v / |v|, |v|),  v = rij[e] rounded to fp32 (rij.to(dtype), mliap_threepass.py:326)
    e_pk[e] = (t, table(pair) * (M - 1) + k, sender feature row, d(|v|)),  x = clamp((r - r_lo) / h, 0, M - 1 - 1e-4),
              k = floor(x), t = x - k (t = -0 below r_lo), pair = (species(send), species(recv)),
              d(r) = tanh((B(r) . w)^2) f_cut(r)
    e_dd[e] = d'(r),  e_recv[e] = pair_i[e] - a
Lengths are drawn away from the knots (t in [0.05, 0.95]) so that the interval is the same in fp32 and fp64.
"""
import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("x_from_spec", [0, 1])
def test_edge_geometry_against_fp64(x_from_spec):
    from mace_onegpu._lib import K, stream
    from oracle import mace_ref
    assert torch.cuda.is_available(), "GPU test without a GPU"
    g = torch.Generator().manual_seed(7 + x_from_spec)
    E, n_nodes, S, nb, p, M, r_lo, r_max = 3000, 200, 2, 8, 5, 512, 0.5, 6.0
    h = (r_max - r_lo) / (M - 1)
    print(f"case x_from_spec={x_from_spec}: {E} edges", flush=True)
    k = torch.randint(0, M - 1, (E,), generator=g)
    t = 0.05 + 0.9 * torch.rand(E, generator=g, dtype=torch.float64)
    r = r_lo + (k + t) * h
    r = r.clamp(max=r_max - 0.05 * h)
    u = torch.randn(E, 3, generator=g, dtype=torch.float64)
    u /= u.norm(dim=1, keepdim=True)
    rij = u * r[:, None]
    a = 17
    recv = torch.randint(0, n_nodes, (E,), generator=g)
    send = torch.randint(0, n_nodes, (E,), generator=g)
    spec = torch.randint(0, S, (n_nodes,), generator=g)
    pair_map = torch.tensor([2, 0, 3, 1])                            # distinct table per ordered pair
    w = torch.randn(nb, generator=g, dtype=torch.float64) * 0.3

    # fp64 reference on the fp32 values the kernel reads
    v = rij.float().double()
    rr = v.norm(dim=1).requires_grad_()
    wf = w.float().double()
    d = torch.tanh((mace_ref.bessel(rr, r_max, nb) @ wf) ** 2) * mace_ref.poly_cutoff(rr, r_max, p)
    (dd,) = torch.autograd.grad(d.sum(), rr)
    d, rr = d.detach(), rr.detach()
    x = ((rr - r_lo) / h).clamp(0.0, M - 1 - 1e-4)
    kk = torch.floor(x)
    row = pair_map[spec[send] * S + spec[recv]] * (M - 1) + kk.long()
    xsrc = spec[send] if x_from_spec else send

    dev = "cuda"
    i32 = dict(dtype=torch.int32, device=dev)
    e_u = torch.full((E, 4), float("nan"), device=dev)
    e_pk = torch.full((E, 4), float("nan"), device=dev)
    e_recv = torch.full((E,), -7, **i32)
    e_dd = torch.full((E,), float("nan"), device=dev)
    dens_w = (ctypes.c_float * nb)(*w.tolist())
    K.mm_edge_geom_rij(E, None, rij.to(dev), (recv + a).to(**i32), a, send.to(**i32), spec.to(**i32), S,
                       pair_map.to(**i32), dens_w, nb, r_max, p, M, r_lo, 1.0 / h, x_from_spec, e_u, None, e_pk,
                       e_recv, e_dd, stream())
    # the edge count from device memory (graph replays): the same launch writes only the first E_dev edges
    E_real = E // 3
    pk2 = torch.full((E, 4), float("nan"), device=dev)
    K.mm_edge_geom_rij(E, torch.tensor([E_real], **i32), rij.to(dev), (recv + a).to(**i32), a, send.to(**i32),
                       spec.to(**i32), S, pair_map.to(**i32), dens_w, nb, r_max, p, M, r_lo, 1.0 / h, x_from_spec,
                       torch.empty_like(e_u), None, pk2, torch.empty_like(e_recv), torch.empty_like(e_dd), stream())
    torch.cuda.synchronize()
    assert torch.equal(pk2[:E_real].view(torch.int32), e_pk[:E_real].view(torch.int32))
    assert bool(pk2[E_real:].isnan().all())
    e_u, e_pk, e_recv, e_dd = e_u.cpu().double(), e_pk.cpu(), e_recv.cpu(), e_dd.cpu().double()
    pki = e_pk.view(torch.int32)

    def close(name, got, ref, tol):
        err = float((got - ref).abs().max())
        print(f"  {name}: max|err| {err:.3e} (max|ref| {float(ref.abs().max()):.3e})", flush=True)
        assert torch.isfinite(got).all() and err <= tol

    close("unit vector", e_u[:, :3], v / rr[:, None], 3e-7)
    close("r", e_u[:, 3], rr, 2e-7 * r_max)
    close("t", e_pk[:, 0].double(), x - kk, 1e-4)
    # the Bessel sines come from one fp64 sincos and an fp64 rotation: the remaining error is fp32 arithmetic
    # (measured on these seeds: 3e-7 / 6e-7 of max|d|, 2.4e-7 / 8.7e-7 of max|d'|)
    close("density", e_pk[:, 3].double(), d, 1e-6 * float(d.abs().max()) + 2e-8)
    close("d density / dr", e_dd, dd, 2e-6 * float(dd.abs().max()) + 2e-8)
    assert torch.equal(pki[:, 1].long(), row)
    assert torch.equal(pki[:, 2].long(), xsrc)
    assert torch.equal(e_recv.long(), recv)


@pytest.mark.parametrize("M", [512, 4096, 8192])
def test_spline_interval_stays_inside_the_table(M):
    """Lengths at the top of the table and beyond r_max land in the last interval (k = M - 2, t in [0, 1]) for
    every knot count: the fp32 clamp M - 1 - 1e-4 rounds to M - 1 for M >= 4096, and the interval index is clamped
    separately so that no row points past the n_tab (M - 1) intervals of the table."""
    from mace_onegpu._lib import K, stream
    assert torch.cuda.is_available(), "GPU test without a GPU"
    S, nb, p, r_lo, r_max = 1, 8, 5, 0.5, 6.0
    h = (r_max - r_lo) / (M - 1)
    r = torch.tensor([r_max - 0.5 * h, r_max - 1e-6, r_max, r_max + 0.3, 7.5, r_lo + 0.25 * h, 0.3],
                     dtype=torch.float64)
    E = r.numel()
    print(f"case M={M}: {E} edges", flush=True)
    rij = torch.stack([r, torch.zeros_like(r), torch.zeros_like(r)], 1)
    dev = "cuda"
    i32 = dict(dtype=torch.int32, device=dev)
    e_u = torch.empty(E, 4, device=dev)
    e_pk = torch.empty(E, 4, device=dev)
    e_recv = torch.empty(E, **i32)
    e_dd = torch.empty(E, device=dev)
    dens_w = (ctypes.c_float * nb)(*([0.1] * nb))
    K.mm_edge_geom_rij(E, None, rij.to(dev), torch.zeros(E, **i32), 0, torch.zeros(E, **i32), torch.zeros(1, **i32), S,
                       torch.zeros(1, **i32), dens_w, nb, r_max, p, M, r_lo, 1.0 / h, 0, e_u, None, e_pk, e_recv,
                       e_dd, stream())
    torch.cuda.synchronize()
    pk = e_pk.cpu()
    row = pk.view(torch.int32)[:, 1].long()
    t = pk[:, 0].double()
    print(f"  rows {row.tolist()} t {[round(float(x), 4) for x in t]}", flush=True)
    assert int(row.max()) <= M - 2 and int(row.min()) >= 0
    assert bool(((t >= 0) & (t <= 1)).all())
    assert row[:5].tolist() == [M - 2] * 5                        # r >= r_max - h/2: the last interval
    assert row[5:].tolist() == [0, 0]                             # r <= r_lo + h/4: the first interval
    assert float(t[6]) == 0.0                                     # below r_lo: clamped to the first knot
    # a length below r_lo is marked by the sign of t = -0 (its spline derivative is zero); r_lo + h/4 is not
    assert math.copysign(1.0, float(t[6])) == -1.0 and math.copysign(1.0, float(t[5])) == 1.0

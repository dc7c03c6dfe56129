"""The layer-1 ACE kernels (mm_ace1_fwd, mm_ace1_bwd) called through the C ABI on synthetic receiver-CSR inputs,
against an fp64 restatement (marked gpu).

Semantics checked (the density-projection form of layer 1, reference ace_layer1.py:58-85):
    h_q(e)        = a0 + t (a1 + t (a2 + t a3)),  (a0..a3) = table row of edge e, feature q (64 features)
    B[i, m, s, q] = sum_{e: recv(e) = i, species(e) = s} h_q(e) Y_m(u_e),    rho[i] = sum_e density(e)
    part[e, 1+m]  = sum_q h_q(e) gB[i, m, s_e, q],   part[e, 0] = inv_h sum_m Y_m(u_e) sum_q h'_q(e) gB[i, m, s_e, q]
(the backward takes gB with its columns in the kernel's MFMA operand order, fast_layers.ace_gb_order)
Receiver degrees sit at and around the kernels' 64-slot harmonic batches, 16-edge backward tiles (8-slot forward step
pairs), 224-edge species-grouped forward segments and 256-edge backward segments; every special degree occurs.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H = 64


def _case(seed, nC, S, S_pad, NR=11):
    rng = np.random.default_rng(seed)
    special = [0, 1, 3, 7, 8, 9, 15, 16, 17, 63, 64, 65, 80, 128, 129, 223, 224, 225, 255, 256, 257, 300, 449, 513]
    deg = np.concatenate([special, rng.choice(special, nC - len(special))])
    rng.shuffle(deg)
    rowptr = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    E = int(rowptr[-1])
    u = rng.normal(size=(E, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    return dict(rowptr=rowptr, u=u, r=rng.uniform(0.8, 6.0, E), t=rng.uniform(0.0, 1.0, E),
                row=rng.integers(0, NR, E), spec=rng.integers(0, S, E), dens=rng.uniform(0.0, 1.0, E),
                tab=rng.normal(size=(NR, H, 4)) * np.array([1.0, 0.5, 0.25, 0.125]),
                gB=rng.normal(size=(nC, 16, S_pad, H)), S=S, S_pad=S_pad)


def _reference(cs):
    from oracle import mace_ref
    f = lambda a: torch.tensor(a, dtype=torch.float32).double()      # the fp32 values the kernels read
    nC = len(cs["rowptr"]) - 1
    recv = torch.repeat_interleave(torch.arange(nC), torch.from_numpy(np.diff(cs["rowptr"])).long())
    Y = mace_ref.sh(f(cs["u"]))                                       # [E, 16]
    a = f(cs["tab"])[torch.from_numpy(cs["row"]).long()]             # [E, 64, 4]
    t = f(cs["t"])[:, None]
    h = a[..., 0] + t * (a[..., 1] + t * (a[..., 2] + t * a[..., 3]))
    hp = a[..., 1] + t * (2 * a[..., 2] + 3 * t * a[..., 3])
    s = torch.from_numpy(cs["spec"]).long()
    B = torch.zeros(nC, 16, cs["S_pad"], H, dtype=torch.float64)
    for e in range(len(recv)):
        B[recv[e], :, s[e], :] += Y[e][:, None] * h[e][None, :]
    rho = torch.zeros(nC, dtype=torch.float64).index_add(0, recv, f(cs["dens"]))
    gB = f(cs["gB"])
    gsel = gB[recv, :, s, :]                                          # [E, 16, 64]
    dY = torch.einsum("eq,emq->em", h, gsel)
    dr = torch.einsum("em,eq,emq->e", Y, hp, gsel)
    return B, rho, dY, dr


@pytest.mark.parametrize("S,S_pad", [(1, 2), (2, 2), (3, 4), (4, 4)])
def test_ace_kernels_against_fp64(S, S_pad):
    from mace_onegpu._lib import K, stream
    assert torch.cuda.is_available(), "GPU test without a GPU"
    nC = 45
    cs = _case(11, nC, S, S_pad)
    E = len(cs["t"])
    print(f"case S={S} S_pad={S_pad}: nC {nC} edges {E}", flush=True)
    dev = "cuda"
    f32 = dict(dtype=torch.float32, device=dev)
    pk = torch.empty(E, 4, **f32)
    pk[:, 0] = torch.tensor(cs["t"], **f32)
    pk[:, 3] = torch.tensor(cs["dens"], **f32)
    pki = pk.view(torch.int32)
    pki[:, 1] = torch.tensor(cs["row"], dtype=torch.int32, device=dev)
    pki[:, 2] = torch.tensor(cs["spec"], dtype=torch.int32, device=dev)
    eu = torch.empty(E, 4, **f32)
    eu[:, :3] = torch.tensor(cs["u"], **f32)
    eu[:, 3] = torch.tensor(cs["r"], **f32)
    rowptr = torch.tensor(cs["rowptr"], dtype=torch.int32, device=dev)
    tab = torch.tensor(cs["tab"], **f32).contiguous()
    from mace_onegpu.fast_layers import ace_gb_order
    gB = torch.tensor(cs["gB"], **f32).reshape(nC, 16, S_pad * H)[:, :, ace_gb_order(S_pad)].contiguous()
    B = torch.full((nC, 16 * S_pad * H), float("nan"), **f32)
    rho = torch.full((nC,), float("nan"), **f32)
    part = torch.full((E * 17 + 9,), float("nan"), **f32)
    inv_h = 2.5
    K.mm_ace1_fwd(rowptr, nC, pk, eu, tab, S, S_pad, B, rho, stream())
    K.mm_ace1_bwd(rowptr, nC, pk, eu, tab, S, S_pad, gB, inv_h, part, stream())
    torch.cuda.synchronize()
    B_r, rho_r, dY_r, dr_r = _reference(cs)

    def close(name, got, ref, rel):
        got = got.double().cpu()
        err = float((got - ref).abs().max())
        scale = float(ref.abs().max())
        print(f"  {name}: max|err| {err:.3e} (max|ref| {scale:.3e})", flush=True)
        assert torch.isfinite(got).all() and err <= rel * scale + 1e-12

    close("B", B.view(nC, 16, S_pad, H), B_r, 1e-5)     # pad species blocks are written as 0
    close("rho", rho, rho_r, 1e-5)
    p = part[:E * 17].view(E, 17)
    close("dL/dY", p[:, 1:], dY_r, 1e-5)
    close("inv_h dL/dr", p[:, 0], inv_h * dr_r, 1e-5)
    assert torch.isnan(part[E * 17:]).all()                # nothing written past the partials

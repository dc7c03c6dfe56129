"""Pins of the oracle's scalar conventions (CPU only).

mace-torch / e3nn are not installed, so the oracle's radial basis, cutoff, activation constant and layer
normalisations are restated from their published definitions (oracle/mace_ref.py).  Each test here checks one of
them against what the mathematics fixes, chosen so that a plausible slip fails:
  * Bessel basis sqrt(2/r_max) sin(k pi r / r_max) / r: orthonormal on [0, r_max] with weight r^2 (a wrong
    prefactor, k offset or power of r breaks it);
  * polynomial cutoff (p = 5): the unique polynomial 1 + a x^p + b x^(p+1) + c x^(p+2) with f(1) = f'(1) = f''(1)
    = 0 (a wrong coefficient breaks a boundary condition), and 0 beyond r_max;
  * silu_n = normalize2mom(silu): unit second moment under N(0, 1), by Gauss-Hermite quadrature (independent of
    the adaptive quadrature the oracle uses) and the product's constant;
  * e3nn normalisation (every weight ~ N(0, 1)): each Linear, the one-hot skip tensor product, the node
    embedding, the readouts, the radial MLP and each channelwise-TP path keep the second moment of unit-variance
    inputs (a dropped or doubled 1/sqrt(fan_in), sqrt(2 l + 1) or silu_n constant changes it by a large factor);
  * the density normalisation: message = linear(A) / (rho + 1) with rho = sum_e tanh(z_e^2) f_cut(r_e), checked
    in the two limits that reduce it to closed forms (w = 0: rho = 0; saturated tanh: rho = sum_e f_cut);
  * the oracle's harmonics equal the scipy-pinned table of mace_onegpu.o3;
  * energy bookkeeping E_i = e0[Z_i] + shift + scale (R1 + R2): affine in the model's scale / shift / E0.
"""
import math

import numpy as np
import pytest
import torch
from scipy.integrate import quad

from oracle import mace_ref

F64 = torch.float64


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _second_moment(fn, n_in, n_draws, n_samples, seed, x_sampler=None):
    """Mean of y^2 over weight draws (fn(x, gen) draws its own N(0, 1) weights) and unit-variance inputs."""
    g = _g(seed)
    acc = []
    for _ in range(n_draws):
        x = torch.randn(n_samples, *n_in, generator=g, dtype=F64) if x_sampler is None else x_sampler(g)
        y = fn(x, g)
        acc.append(float((y ** 2).mean()))
    return float(np.mean(acc))


# ----------------------------------------------------------------------------- radial basis and cutoff
@pytest.mark.parametrize("r_max", [5.0, 6.0])
def test_bessel_basis_is_orthonormal_with_weight_r2(r_max):
    n = 8

    def b(r):
        return mace_ref.bessel(torch.tensor([r], dtype=F64), r_max, n)[0].numpy()
    G = np.zeros((n, n))
    for i in range(n):
        for j in range(i, n):
            v, _ = quad(lambda r: b(r)[i] * b(r)[j] * r * r, 1e-12, r_max, limit=200, epsabs=1e-13)
            G[i, j] = G[j, i] = v
    np.testing.assert_allclose(G, np.eye(n), atol=1e-10)
    # the first function is sqrt(2/r_max) sin(pi r / r_max) / r: its limit at r -> 0 is sqrt(2/r_max) pi / r_max
    b0 = float(mace_ref.bessel(torch.tensor([1e-9], dtype=F64), r_max, 1)[0, 0])
    assert abs(b0 - math.sqrt(2 / r_max) * math.pi / r_max) < 1e-8


@pytest.mark.parametrize("p", [5, 6])
def test_polynomial_cutoff_boundary_conditions(p):
    r_max = 6.0
    x = torch.linspace(0, 0.999, 400, dtype=F64)
    f = mace_ref.poly_cutoff(x * r_max, r_max, p).numpy()
    # a polynomial of degree p + 2 in x (exact fit), equal to 1 + a x^p + b x^(p+1) + c x^(p+2)
    V = np.vander(x.numpy(), p + 3, increasing=True)
    coef, *_ = np.linalg.lstsq(V, f, rcond=None)
    assert np.abs(V @ coef - f).max() < 1e-12
    assert abs(coef[0] - 1) < 1e-9 and np.abs(coef[1:p]).max() < 1e-7
    # f(1) = f'(1) = f''(1) = 0: the three conditions that fix a, b, c
    P = np.polynomial.Polynomial(coef)
    for d in range(3):
        assert abs(P.deriv(d)(1.0) if d else P(1.0)) < 1e-7, d
    assert abs(P.deriv(3)(1.0)) > 1.0                     # not identically flat: the degree is p + 2
    # zero at and beyond r_max; one at r = 0; monotone in between
    out = mace_ref.poly_cutoff(torch.tensor([r_max, r_max + 1e-9, 7.5, 100.0], dtype=F64), r_max, p)
    assert torch.all(out == 0)
    assert float(mace_ref.poly_cutoff(torch.tensor([0.0], dtype=F64), r_max, p)[0]) == 1.0
    assert np.all(np.diff(f) <= 1e-15)


# ----------------------------------------------------------------------------- activation constant
def test_silu_normalisation_constant():
    from mace_onegpu import model as mm
    z, w = np.polynomial.hermite_e.hermegauss(300)          # weight exp(-z^2/2); sum(w) = sqrt(2 pi)
    silu = z / (1 + np.exp(-z))
    m2 = float((w * silu ** 2).sum() / w.sum())
    c = 1 / math.sqrt(m2)
    assert abs(c - mace_ref.silu_norm()) < 1e-10
    assert abs(c - mm.SILU_NORM) < 1e-12
    # Monte-Carlo: silu_n has unit second moment under N(0, 1)
    zz = torch.randn(2_000_000, generator=_g(3), dtype=F64)
    assert abs(float((mace_ref.silu_n(zz) ** 2).mean()) - 1) < 5e-3


# ----------------------------------------------------------------------------- layer normalisations
def _w(g, *shape):
    return torch.randn(*shape, generator=g, dtype=F64)


@pytest.mark.parametrize("dims,tol", [([64, 64, 64, 64, 512], 0.06), ([8, 64, 64, 64, 512], 0.25)])
def test_radial_mlp_keeps_unit_second_moment(dims, tol):
    """Every hidden layer and the output of the radial MLP have unit second moment for unit-variance inputs.
    normalize2mom makes silu_n exact for N(0, 1) pre-activations; with a finite fan-in n the pre-activation
    variance of a column is chi2_n / n, and the convexity of silu^2 raises the mean by about 1 % per layer at
    n = 64 and 6 % at n = 8 (the first layer of the real MLP), compounding over the layers.  The slips this must
    catch change it by a factor 8 or 64 (a dropped 1/sqrt(fan_in)) or 0.36 per layer (a dropped silu_n
    constant)."""

    def layers(depth):
        def fn(x, g):
            Ws = [_w(g, dims[j], dims[j + 1]) for j in range(depth)]
            return mace_ref.radial_mlp(x, Ws)
        return fn
    for depth in range(1, len(dims)):
        m2 = _second_moment(layers(depth), (dims[0],), 30, 2000, 10 + depth)
        assert abs(m2 - 1) < tol, (depth, m2)


@pytest.mark.parametrize("ls", [[0], [0, 1], [0, 1, 2, 3]])
def test_per_l_linear_keeps_unit_second_moment(ls):
    C = 128
    n = sum(2 * l + 1 for l in ls)
    m2 = _second_moment(lambda x, g: mace_ref.per_l_linear(x, ls, _w(g, len(ls), C, C), C), (n, C), 8, 200, 1)
    assert abs(m2 - 1) < 0.03


@pytest.mark.parametrize("n_src", [1, 2, 3])
def test_multi_source_linear_keeps_unit_second_moment(n_src):
    C = 128

    def fn(x, g):
        return mace_ref.multi_source_linear([x[:, j] for j in range(n_src)], [_w(g, C, C) for _ in range(n_src)])
    m2 = _second_moment(fn, (n_src, 3, C), 8, 200, 2)
    assert abs(m2 - 1) < 0.03


def test_skip_tp_and_node_embedding_normalisation():
    """FullyConnectedTensorProduct(x, attrs): unit second moment for unit-variance x and attrs; with one-hot
    attrs (second moment 1/n_el per component) the output has second moment 1/n_el, and the one-hot fast path
    equals the general contraction."""
    C, ne = 128, 89
    g = _g(4)
    m2 = _second_moment(lambda x, gg: mace_ref.skip_tp(x[:, :, :C], x[:, 0, C:C + ne], _w(gg, C, ne, C)),
                        (3, C + ne), 6, 300, 5)
    assert abs(m2 - 1) < 0.05
    x = torch.randn(300, 3, C, generator=g, dtype=F64)
    s = torch.randint(0, ne, (300,), generator=g)
    W = _w(g, C, ne, C)
    oh = torch.nn.functional.one_hot(s, ne).to(F64)
    a, b = mace_ref.skip_tp(x, s, W), mace_ref.skip_tp(x, oh, W)
    assert float((a - b).abs().max()) < 1e-12
    assert abs(float((a ** 2).mean()) * ne - 1) < 0.1
    # node embedding (e3nn Linear n_el x 0e -> C x 0e): unit second moment for unit-variance attributes
    m2 = _second_moment(lambda x, gg: mace_ref.node_embedding(x, _w(gg, ne, C)), (ne,), 8, 300, 6)
    assert abs(m2 - 1) < 0.03


def test_readouts_keep_unit_second_moment():
    C = 128
    m2 = _second_moment(lambda x, g: mace_ref.readout_linear(x, _w(g, C)), (C,), 400, 100, 7)
    assert abs(m2 - 1) < 0.06
    m2 = _second_moment(lambda x, g: mace_ref.readout_mlp(x, _w(g, C, 16), _w(g, 16)), (C,), 400, 100, 8)
    assert abs(m2 - 1) < 0.1


@pytest.mark.parametrize("layer", [1, 2])
def test_tp_paths_keep_unit_second_moment(layer):
    """Each channelwise-TP path (component irrep normalisation, element path normalisation, one instruction per
    output segment): with W, X ~ N(0, 1) and Y the harmonics of a uniform direction, every output component has
    unit second moment."""
    from mace_onegpu import model as mm, o3
    tab = mm.Tables(mm.MaceSpec()).tp1 if layer == 1 else mm.Tables(mm.MaceSpec()).tp2
    g = _g(20 + layer)
    E, C = 40000, 4
    nX = sum(2 * l + 1 for l in tab["in_ls"])
    u = torch.randn(E, 3, generator=g, dtype=F64)
    Y = mace_ref.sh(u)
    W = _w(g, E, tab["nW"], C)
    X = _w(g, E, nX, C)
    out = mace_ref.channelwise_tp(W, X, Y, torch.arange(E), tab["paths"], tab["in_ls"], o3.coupling)
    m2 = (out ** 2).mean((0, 2))                                    # per output component
    assert out.shape[1] == tab["nO"]
    assert float((m2 - 1).abs().max()) < 0.06, m2


def test_oracle_harmonics_match_the_scipy_pinned_table():
    from mace_onegpu import o3
    u = torch.randn(500, 3, generator=_g(9), dtype=F64)
    np.testing.assert_allclose(mace_ref.sh(u).numpy(), o3.spherical_harmonics(u.numpy()), atol=1e-12)
    # component normalisation: mean of Y_m^2 over the sphere is 1 for every m
    v = torch.randn(400000, 3, generator=_g(10), dtype=F64)
    m2 = (mace_ref.sh(v) ** 2).mean(0)
    assert float((m2 - 1).abs().max()) < 0.02


# ----------------------------------------------------------------------------- density normalisation
def _cluster(seed=0):
    from mace_onegpu import systems
    pos, box, Z = systems.water_box(64, seed=seed)
    keep = np.nonzero(((pos - pos[0]) ** 2).sum(1) < 5.0 ** 2)[0][:30]
    p = torch.as_tensor(pos[keep] - pos[keep].mean(0))
    d = ((p[:, None] - p[None]) ** 2).sum(-1)
    recv, send = torch.nonzero((d < 36.0) & ~torch.eye(len(p), dtype=torch.bool), as_tuple=True)
    return p, torch.as_tensor(Z[keep] - 1), recv, send


def test_message_is_divided_by_density_plus_one(ref_model):
    """Density weight w = 0 gives rho = 0 (tanh 0 = 0); a huge w saturates tanh(z^2) -> 1 so rho = sum_e f_cut.
    The two messages differ by exactly the factor (sum_e f_cut + 1) per receiver."""
    import copy
    p, spec, recv, send = _cluster()
    n = len(p)
    vec = p[recv] - p[send]
    m0, m1 = copy.copy(ref_model), copy.copy(ref_model)
    m0.P = dict(ref_model.P)
    m1.P = dict(ref_model.P)
    m0.P["i0_dens"] = torch.zeros_like(ref_model.P["i0_dens"])
    # only the first Bessel function, sqrt(2/r_max) sin(pi r/r_max)/r > 0 on (0, r_max): z^2 is huge except within
    # ~1e-6 A of r_max, where f_cut ~ (1 - r/r_max)^3 vanishes
    w1 = torch.zeros_like(ref_model.P["i0_dens"])
    w1[0] = 1e6
    m1.P["i0_dens"] = w1
    with torch.no_grad():
        M0 = mace_ref.layer1_message(m0, spec, n, send, recv, vec)
        M1 = mace_ref.layer1_message(m1, spec, n, send, recv, vec)
    r = torch.linalg.vector_norm(vec, dim=1)
    fsum = mace_ref.scatter_sum(mace_ref.poly_cutoff(r, ref_model.r_max, ref_model.p), recv, n)
    ratio = M0 / M1
    np.testing.assert_allclose(ratio.numpy(), (fsum + 1)[:, None, None].expand_as(ratio).numpy(), rtol=1e-9)


def test_density_preactivation_has_unit_second_moment():
    m2 = _second_moment(lambda x, g: mace_ref.density_z(x, _w(g, 8, 1)), (8,), 400, 100, 11)
    assert abs(m2 - 1) < 0.06


# ----------------------------------------------------------------------------- energy bookkeeping
def test_scale_shift_e0_enter_affinely(model):
    """E_i = e0[Z_i] + shift + scale (R1_i + R2_i): with scale s, shift t and per-species E0 the per-atom energies
    are e0 + t + s e_i(identity) and the forces are s F(identity); this fails for a missing or doubled scale in
    either readout or in the G1 chain of the three-pass evaluation."""
    from mace_onegpu import model as mm, o3
    p, spec, recv, send = _cluster(1)
    box = np.array([60.0, 60.0, 60.0])
    p = p + 30.0
    base = mace_ref.RefModel(model, o3.coupling)
    sp = mm.MaceSpec(scale=1.7, shift=-0.35)
    mdl = mm.MaceModel(sp, seed=0)
    mdl.e0.copy_(torch.linspace(-2.0, 1.5, sp.num_elements, dtype=F64))
    m = mace_ref.RefModel(mdl, o3.coupling)
    E0, e0, F0 = mace_ref.three_pass(base, p, box, spec, recv, send, chunk=11)[:3]
    E1, e1, F1 = mace_ref.three_pass(m, p, box, spec, recv, send, chunk=11)[:3]
    expect = mdl.e0[spec] - 0.35 + 1.7 * e0
    np.testing.assert_allclose(e1.numpy(), expect.numpy(), atol=1e-12)
    np.testing.assert_allclose(F1.numpy(), 1.7 * F0.numpy(), atol=1e-13)
    Ef, ef, Ff = mace_ref.energy_forces_full(m, p, box, spec, recv, send)
    np.testing.assert_allclose(ef.numpy(), e1.numpy(), atol=1e-11)
    np.testing.assert_allclose(Ff.numpy(), F1.numpy(), atol=1e-11)

"""Pins of the O(3) building blocks shared by the oracle and the kernels (CPU)."""
import math

import numpy as np
import pytest

from mace_onegpu import o3


def _rot(seed):
    q = np.random.default_rng(seed).normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([[a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
                     [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
                     [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d]])


def test_sh_matches_scipy_complex_harmonics():
    """Y_real = sqrt(4 pi) U_l Y_complex with scipy's Condon-Shortley harmonics (textbook check of the table)."""
    from scipy.special import sph_harm_y
    rng = np.random.default_rng(0)
    u = rng.normal(size=(200, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    theta = np.arccos(u[:, 2])
    phi = np.arctan2(u[:, 1], u[:, 0])
    Y = o3.spherical_harmonics(u)
    for l in range(4):
        Yc = np.stack([sph_harm_y(l, m, theta, phi) for m in range(-l, l + 1)], -1)
        Yr = math.sqrt(4 * math.pi) * (Yc @ o3.real_basis(l).T)
        assert np.abs(Yr.imag).max() < 1e-12
        np.testing.assert_allclose(Y[:, l * l:(l + 1) ** 2], Yr.real, atol=1e-12)


def test_sh_component_normalisation_and_harmonic():
    rng = np.random.default_rng(1)
    u = rng.normal(size=(500, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    Y = o3.spherical_harmonics(u)
    for l in range(4):
        np.testing.assert_allclose((Y[:, l * l:(l + 1) ** 2] ** 2).sum(1), 2 * l + 1, rtol=1e-12)
    # r^l Y_lm are harmonic polynomials: the Laplacian by central differences vanishes
    x = rng.normal(size=(50, 3))
    h = 1e-3
    lap = np.zeros((50, 16))
    for k in range(3):
        e = np.zeros(3)
        e[k] = h
        f = lambda p: np.stack(o3.sh_cartesian(p[:, 0], p[:, 1], p[:, 2]), -1)
        lap += (f(x + e) - 2 * f(x) + f(x - e)) / h ** 2
    assert np.abs(lap).max() < 1e-4


@pytest.mark.parametrize("l1,l2,l3", [(l1, l2, l3) for l1 in range(4) for l2 in range(4)
                                       for l3 in range(abs(l1 - l2), min(l1 + l2, 3) + 1)])
def test_coupling_is_equivariant(l1, l2, l3):
    """C(D1 a, D2 b) = D3 C(a, b) with D from the harmonics themselves: fails for a transposed tensor, a wrong
    sign pattern or a basis mismatch."""
    R = _rot(11)
    D = [o3.wigner_d_from_sh(R, l) for l in range(4)]
    C = o3.w3j(l1, l2, l3)
    assert abs(np.linalg.norm(C) - 1) < 1e-12
    rng = np.random.default_rng(2)
    a, b = rng.normal(size=2 * l1 + 1), rng.normal(size=2 * l2 + 1)
    lhs = np.einsum("ijk,i,j->k", C, D[l1] @ a, D[l2] @ b)
    rhs = D[l3] @ np.einsum("ijk,i,j->k", C, a, b)
    np.testing.assert_allclose(lhs, rhs, atol=1e-12)


def test_cg_orthogonality():
    """Racah CG: sum_{m1 m2} <j1 m1 j2 m2|J M><j1 m1 j2 m2|J' M'> = delta (closed-form identity)."""
    for j1, j2 in [(1, 1), (2, 1), (3, 2), (2, 2)]:
        for J in range(abs(j1 - j2), j1 + j2 + 1):
            for Jp in range(abs(j1 - j2), j1 + j2 + 1):
                s = sum(o3.su2_cg(j1, m1, j2, M - m1, J, M) * o3.su2_cg(j1, m1, j2, M - m1, Jp, M)
                        for M in range(-min(J, Jp), min(J, Jp) + 1) for m1 in range(-j1, j1 + 1)) / (2 * J + 1)
                assert abs(s - (1.0 if J == Jp else 0.0)) < 1e-12


def test_tp_tables_match_reference_widths():
    """nW / nO / terms of the two channelwise TPs: D = 512 / 1280 weights (spline_radial.py:8) and
    2048 -> 5120 messages (scripts/flop_budget.py:68,72) of the reference's MPA-0 layers."""
    t1, t2 = o3.tp_table([0]), o3.tp_table([0, 1])
    assert (t1["nX"], t1["nW"], t1["nO"], len(t1["terms"])) == (1, 4, 16, 16)
    assert (t2["nX"], t2["nW"], t2["nO"], len(t2["terms"])) == (4, 10, 40, 86)
    assert t2["mid_ls"] == [0, 0, 1, 1, 1, 2, 2, 2, 3, 3]
    assert all(abs(abs(c) - 1) < 1e-12 for *_, c in t1["terms"])


def _equivariant_dim(nu, L):
    """Dimension of the degree-nu O(3)-equivariant polynomial maps 0e+1o+2e+3o -> L, by a null-space count."""
    import itertools
    mono = list(itertools.combinations_with_replacement(range(16), nu))
    par = np.array([(-1) ** l for l in range(4) for _ in range(2 * l + 1)], float)
    rng = np.random.default_rng(1)
    X = rng.normal(size=(60 if nu < 3 else 320, 16))
    nM = 2 * L + 1
    rows = []
    for seed in (3, 4, -1):
        if seed < 0:
            D, DL = np.diag(par), np.eye(nM) * (-1) ** L
        else:
            R = _rot(seed)
            D = np.zeros((16, 16))
            for l in range(4):
                D[l * l:(l + 1) ** 2, l * l:(l + 1) ** 2] = o3.wigner_d_from_sh(R, l)
            DL = D[L * L:(L + 1) ** 2, L * L:(L + 1) ** 2]
        A = np.stack([np.prod((X @ D.T)[:, list(m)], 1) for m in mono], 1)
        B = np.stack([np.prod(X[:, list(m)], 1) for m in mono], 1)
        for M in range(nM):
            r = np.zeros((len(X), nM, len(mono)))
            r[:, M, :] += A
            for Mp in range(nM):
                r[:, Mp, :] -= DL[M, Mp] * B
            rows.append(r.reshape(len(X), -1))
    s = np.linalg.svd(np.concatenate(rows), compute_uv=False)
    return int((s < 1e-9 * s[0]).sum())


@pytest.mark.parametrize("L", [0, 1])
def test_symmetric_contraction_basis_spans_the_equivariant_space(L):
    paths = o3.symmetric_contraction_paths([0, 1, 2, 3], L, 3)
    for nu in (1, 2, 3):
        assert len(paths[nu]) == _equivariant_dim(nu, L), (L, nu)


def test_unnormalised_harmonic_polynomials():
    """The backward edge convolution evaluates P_m (mm_shp16) and folds c_m into its coefficients:
    c_m P_m(u) = Y_m(u) on unit vectors, and the generated 1 / c_m table matches."""
    import re
    from mace_onegpu import codegen
    rng = np.random.default_rng(5)
    u = rng.normal(size=(200, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    Y = np.stack(o3.sh_cartesian(u[:, 0], u[:, 1], u[:, 2]), 1)
    P = np.stack(codegen._sh_poly(u[:, 0], u[:, 1], u[:, 2]), 1)
    assert np.abs(P * np.asarray(codegen.SH_NORM) - Y).max() < 1e-12
    inv = [float(v) for v in re.findall(r"r = m == \d+ \? ([0-9.e+-]+)f", codegen.sh_header())]
    assert np.allclose(inv, 1.0 / np.asarray(codegen.SH_NORM)[1:], rtol=1e-15)

"""O(3) building blocks of the MACE layers, restated from their mathematical definitions.

* Real spherical harmonics for l <= 3 in component normalisation (sum_m Y_lm(u)^2 = 2l + 1 on the unit
  sphere), z-polar real basis, components ordered m = -l .. l.  The reference reaches the same functions through
  ``model.spherical_harmonics`` of mace-torch / e3nn (receiver_chunk_mace.py:230-234); e3nn uses a y-polar real
  basis, which is an orthogonal change of basis inside every l and therefore gives the same model class.
* Real coupling coefficients for any (l1, l2, l3): the complex Clebsch-Gordan coefficients from Racah's formula,
  carried into the real basis above, normalised to unit Frobenius norm (the Wigner-3j convention of e3nn).
* The path table of MACE's channelwise ("uvu") tensor product: what the reference reads from the cuEquivariance
  descriptor in ``fused_edge_conv.path_table`` (fused_edge_conv.py:43-68), i.e. terms (w, k, m, o, coef) with
  out[o, c] += coef * W[w, c] * X[k, c] * Y[m], coef = sqrt(2 l3 + 1) * w3j (e3nn "component" irrep
  normalisation, "element" path normalisation with one instruction per output segment).
* The coupling paths of the correlation-3 symmetric contraction (MACE's ``SymmetricContraction``), reduced to a
  linearly independent subset.

Irreps here are the natural-parity ones l = 0e, 1o, 2e, 3o; a feature vector of ``C`` channels over a list of
irreps is stored component-major, channel-minor ("ir_mul"): element (component j, channel c) at j * C + c.
"""
import math
from fractions import Fraction
from functools import lru_cache

import numpy as np

LMAX_SH = 3
N_SH = (LMAX_SH + 1) ** 2          # 16 components: l=0 (1), 1 (3), 2 (5), 3 (7)


def sh_index(l, m):
    """Component index of (l, m) inside the concatenated l = 0..3 vector."""
    return l * l + (m + l)


# ----------------------------------------------------------------------------- spherical harmonics (numpy, fp64)
_S3, _S5, _S7 = math.sqrt(3.0), math.sqrt(5.0), math.sqrt(7.0)
_S15, _S42, _S70, _S105 = math.sqrt(15.0), math.sqrt(42.0), math.sqrt(70.0), math.sqrt(105.0)


def sh_cartesian(x, y, z):
    """Y_lm of a UNIT vector (x, y, z), l = 0..3, component normalisation, as a list of 16 arrays.

    Homogeneous polynomials of degree l (r^2 = x^2 + y^2 + z^2 is written out, so the same expressions are the
    solid harmonics r^l Y_lm for non-unit arguments)."""
    one = np.ones_like(x)
    x2, y2, z2 = x * x, y * y, z * z
    return [
        one,
        _S3 * y, _S3 * z, _S3 * x,
        _S15 * x * y, _S15 * y * z, 0.5 * _S5 * (2 * z2 - x2 - y2), _S15 * x * z, 0.5 * _S15 * (x2 - y2),
        0.25 * _S70 * y * (3 * x2 - y2),
        _S105 * x * y * z,
        0.25 * _S42 * y * (4 * z2 - x2 - y2),
        0.5 * _S7 * z * (2 * z2 - 3 * x2 - 3 * y2),
        0.25 * _S42 * x * (4 * z2 - x2 - y2),
        0.5 * _S105 * z * (x2 - y2),
        0.25 * _S70 * x * (x2 - 3 * y2),
    ]


def spherical_harmonics(vec):
    """[..., 3] -> [..., 16]; the vectors are normalised first."""
    v = np.asarray(vec, dtype=np.float64)
    u = v / np.linalg.norm(v, axis=-1, keepdims=True)
    return np.stack(sh_cartesian(u[..., 0], u[..., 1], u[..., 2]), -1)


def wigner_d_from_sh(R, l, n_samples=64, seed=1234):
    """Real Wigner-D of degree l <= 3 for rotation matrix R, defined by Y_l(R u) = D Y_l(u) (least squares)."""
    rng = np.random.default_rng(seed)
    u = rng.normal(size=(n_samples, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    sl = slice(l * l, (l + 1) ** 2)
    A = spherical_harmonics(u)[:, sl]                 # [n, 2l+1]
    B = spherical_harmonics(u @ R.T)[:, sl]           # rows Y(R u)
    D, *_ = np.linalg.lstsq(A, B, rcond=None)         # A D^T = B
    return D.T


# ----------------------------------------------------------------------------- Clebsch-Gordan coefficients
def _f(n):
    return math.factorial(n)


@lru_cache(maxsize=None)
def su2_cg(j1, m1, j2, m2, j3, m3):
    """Complex-basis Clebsch-Gordan <j1 m1; j2 m2 | j3 m3> for integer j (Racah's closed formula, exact rationals)."""
    if m3 != m1 + m2 or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    if j3 < abs(j1 - j2) or j3 > j1 + j2:
        return 0.0
    pref = Fraction((2 * j3 + 1) * _f(j3 + j1 - j2) * _f(j3 - j1 + j2) * _f(j1 + j2 - j3), _f(j1 + j2 + j3 + 1))
    pref *= _f(j3 + m3) * _f(j3 - m3) * _f(j1 - m1) * _f(j1 + m1) * _f(j2 - m2) * _f(j2 + m2)
    s = Fraction(0)
    for k in range(0, j1 + j2 - j3 + 1):
        d = (k, j1 + j2 - j3 - k, j1 - m1 - k, j2 + m2 - k, j3 - j2 + m1 + k, j3 - j1 - m2 + k)
        if min(d) < 0:
            continue
        den = 1
        for t in d:
            den *= _f(t)
        s += Fraction((-1) ** k, den)
    if s == 0:
        return 0.0
    return math.copysign(math.sqrt(pref * s * s), float(s))


@lru_cache(maxsize=None)
def real_basis(l):
    """U_l (rows: real m = -l..l, columns: complex mu = -l..l) with Y^real_m = sum_mu U[m, mu] Y^complex_mu
    (Condon-Shortley complex harmonics; real harmonics as in the Cartesian table above)."""
    U = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    r2 = 1.0 / math.sqrt(2.0)
    for m in range(-l, l + 1):
        if m > 0:
            U[m + l, -m + l] = r2
            U[m + l, m + l] = (-1) ** m * r2
        elif m == 0:
            U[l, l] = 1.0
        else:
            U[m + l, m + l] = 1j * r2
            U[m + l, -m + l] = -1j * (-1) ** m * r2
    return U


@lru_cache(maxsize=None)
def w3j(l1, l2, l3):
    """Real coupling tensor [2l1+1, 2l2+1, 2l3+1], unit Frobenius norm, such that
    c_M = sum C[m1, m2, M] a_m1 b_m2 maps (V_l1 x V_l2) -> V_l3 equivariantly in the real basis.
    Sign convention: the first entry (C order) with |value| > 1e-9 is positive.  Zero tensor if the triangle
    condition fails."""
    if l3 < abs(l1 - l2) or l3 > l1 + l2:
        return np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    cg = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for a in range(-l1, l1 + 1):
        for b in range(-l2, l2 + 1):
            if abs(a + b) <= l3:
                cg[a + l1, b + l2, a + b + l3] = su2_cg(l1, a, l2, b, l3, a + b)
    U1, U2, U3 = real_basis(l1), real_basis(l2), real_basis(l3)
    # complex coefficients of a real vector a: a^C = U^T a ;  real coefficients of the result: c^R = conj(U) c^C
    C = np.einsum("ia,jb,abk,mk->ijm", U1, U2, cg, np.conj(U3))
    re, im = np.abs(C.real).max(), np.abs(C.imag).max()
    C = C.real if re >= im else C.imag
    C = C / np.linalg.norm(C)
    flat = C.reshape(-1)
    first = flat[np.argmax(np.abs(flat) > 1e-9)]
    if first < 0:
        C = -C
    C[np.abs(C) < 1e-15] = 0.0
    return C


def coupling(l1, l2, l3):
    """Component-normalised coupling coefficients sqrt(2 l3 + 1) * w3j (what e3nn's TensorProduct applies for a
    single "uvu" instruction per output segment with component / element normalisation)."""
    return math.sqrt(2 * l3 + 1) * w3j(l1, l2, l3)


# ----------------------------------------------------------------------------- irreps lists
class Irreps:
    """A list of natural-parity irreps (each of multiplicity C) with component offsets."""

    def __init__(self, ls):
        self.ls = list(ls)
        self.offsets = []
        o = 0
        for l in self.ls:
            self.offsets.append(o)
            o += 2 * l + 1
        self.dim = o                               # number of components (times C floats per node)

    def __repr__(self):
        return "+".join(f"{l}{'e' if l % 2 == 0 else 'o'}" for l in self.ls)


def tp_paths(in_ls, sh_lmax, target_ls):
    """Instructions of MACE's ``tp_out_irreps_with_instructions``: for every input irrep l1 (in order), every SH l2
    (0..sh_lmax) and every l3 in |l1-l2| .. l1+l2 with natural parity that is in target_ls, one output segment;
    segments are then sorted by l3 (stable), which fixes both the mid layout and the weight order.
    Returns a list of (l1_index, l1, l2, l3) in mid order."""
    raw = []
    for i1, l1 in enumerate(in_ls):
        for l2 in range(sh_lmax + 1):
            for l3 in range(abs(l1 - l2), l1 + l2 + 1):
                if (l1 + l2 + l3) % 2 == 0 and l3 in target_ls:
                    raw.append((i1, l1, l2, l3))
    return sorted(raw, key=lambda p: p[3])   # Python's sort is stable


def tp_table(in_ls, sh_lmax=LMAX_SH, target_ls=(0, 1, 2, 3), tol=1e-12):
    """Path table of the channelwise TP (node feats in_ls x SH 0..sh_lmax -> mid): dict with
    nX (input components), nW (paths = weight segments), nO (mid components), nY, terms [(w, k, m, o, coef)],
    paths [(i1, l1, l2, l3)], mid_ls, in_ls."""
    xin = Irreps(in_ls)
    paths = tp_paths(in_ls, sh_lmax, target_ls)
    mid = Irreps([p[3] for p in paths])
    terms = []
    for w, (i1, l1, l2, l3) in enumerate(paths):
        C = coupling(l1, l2, l3)
        for a in range(2 * l1 + 1):
            for b in range(2 * l2 + 1):
                for M in range(2 * l3 + 1):
                    c = C[a, b, M]
                    if abs(c) > tol:
                        terms.append((w, xin.offsets[i1] + a, l2 * l2 + b, mid.offsets[w] + M, float(c)))
    return dict(nX=xin.dim, nW=len(paths), nO=mid.dim, nY=(sh_lmax + 1) ** 2, terms=terms, paths=paths,
                mid_ls=mid.ls, in_ls=list(in_ls))


# Channelwise-TP path tables that have a compiled explicit-weight kernel (mm_tpw_<name>_{fwd,bwd}, used by
# FusedConvTP): name -> (node-feature ls, SH lmax, target ls).  The two interaction blocks of the MACE-MPA-0
# architecture and the full l<=3 table (node features 0e+1o+2e+3o) of the edge-convolution microbenchmark.
COMPILED_TP_TABLES = {"l1": ((0,), 3, (0, 1, 2, 3)),
                      "l2": ((0, 1), 3, (0, 1, 2, 3)),
                      "l0123": ((0, 1, 2, 3), 3, (0, 1, 2, 3))}

# Tables without a kernel in the library whose kernels the build makes ahead (mace_onegpu.tp_jit; any other table
# gets its kernels built on first use): one of each backward layout the generator has besides the compiled
# tables' -- one channel per lane with two edges in flight (1o input), two path groups (0e+2e input, 145 terms),
# two channels per lane (0e+1o -> 0e+1o, 21 terms) -- and a table with harmonics up to l = 2 (9 components).
PREBUILT_JIT_TP_TABLES = (((1,), 3, (0, 1, 2, 3)),
                          ((0, 2), 3, (0, 1, 2, 3)),
                          ((0, 1), 3, (0, 1)),
                          ((0, 1), 2, (0, 1, 2)))


# ----------------------------------------------------------------------------- symmetric contraction paths
def _sym_monomials(nvar, deg):
    """All sorted index tuples (i1 <= ... <= i_deg) -> position."""
    out = {}

    def rec(start, cur):
        if len(cur) == deg:
            out[tuple(cur)] = len(out)
            return
        for i in range(start, nvar):
            rec(i, cur + [i])
    rec(0, [])
    return out


def _ls_of(in_ls):
    xin = Irreps(in_ls)
    return xin, [(l, xin.offsets[i]) for i, l in enumerate(in_ls)]


def path_tensor(path, in_ls, L):
    """Dense tensor U[M, i1, ..., i_nu] (components of the input irreps list) of one coupling path:
    nu=1: ('1', l1) ; nu=2: ('2', l1, l2) ; nu=3: ('3', l1, l2, J, l3)."""
    xin = Irreps(in_ls)
    d = xin.dim
    off = {l: xin.offsets[i] for i, l in enumerate(in_ls)}
    kind = path[0]
    if kind == "1":
        l1 = path[1]
        U = np.zeros((2 * L + 1, d))
        for M in range(2 * L + 1):
            U[M, off[l1] + M] = 1.0
        return U
    if kind == "2":
        _, l1, l2 = path
        C = coupling(l1, l2, L)
        U = np.zeros((2 * L + 1, d, d))
        U[:, off[l1]:off[l1] + 2 * l1 + 1, off[l2]:off[l2] + 2 * l2 + 1] = C.transpose(2, 0, 1)
        return U
    _, l1, l2, J, l3 = path
    C1 = coupling(l1, l2, J)                       # [a, b, j]
    C2 = coupling(J, l3, L)                        # [j, c, M]
    T = np.einsum("abj,jcM->Mabc", C1, C2)
    U = np.zeros((2 * L + 1, d, d, d))
    U[:, off[l1]:off[l1] + 2 * l1 + 1, off[l2]:off[l2] + 2 * l2 + 1, off[l3]:off[l3] + 2 * l3 + 1] = T
    return U


def _sym_vector(U, mono):
    """Coefficients of the polynomial M -> sum U[M, i..] x_i.. in the symmetric monomial basis (flattened over M)."""
    nu = U.ndim - 1
    nM = U.shape[0]
    v = np.zeros((nM, len(mono)))
    it = np.nditer(U[0], flags=["multi_index"])
    idx = np.argwhere(np.abs(U) > 0)
    for row in idx:
        M, key = row[0], tuple(sorted(row[1:].tolist()))
        v[M, mono[key]] += U[tuple(row)]
    del it
    return v.reshape(-1), nu


def symmetric_contraction_paths(in_ls, L, correlation=3, tol=1e-9):
    """Linearly independent coupling paths of degree 1..correlation mapping the input irreps (each multiplicity 1
    per channel) to the natural-parity output irrep L.  Enumeration order: nu ascending; nu=2: l1 <= l2;
    nu=3: (l1 <= l2, J, l3) lexicographic; a path is kept if its polynomial is not in the span of the kept ones
    of the same degree.  Returns {nu: [path, ...]}."""
    xin = Irreps(in_ls)
    out = {}
    for nu in range(1, correlation + 1):
        cands = []
        if nu == 1:
            if L in in_ls:
                cands.append(("1", L))
        elif nu == 2:
            for i, l1 in enumerate(in_ls):
                for l2 in in_ls[i:]:
                    if abs(l1 - l2) <= L <= l1 + l2 and (l1 + l2 + L) % 2 == 0:
                        cands.append(("2", l1, l2))
        else:
            for i, l1 in enumerate(in_ls):
                for l2 in in_ls[i:]:
                    for J in range(abs(l1 - l2), l1 + l2 + 1):
                        for l3 in in_ls:
                            if abs(J - l3) <= L <= J + l3 and (l1 + l2 + l3 + L) % 2 == 0:
                                cands.append(("3", l1, l2, J, l3))
        mono = _sym_monomials(xin.dim, nu)
        basis = []
        kept = []
        for p in cands:
            v, _ = _sym_vector(path_tensor(p, in_ls, L), mono)
            if np.linalg.norm(v) < tol:
                continue
            r = v.copy()
            for q in basis:
                r -= (q @ r) * q
            if np.linalg.norm(r) > tol * max(1.0, np.linalg.norm(v)):
                basis.append(r / np.linalg.norm(r))
                kept.append(p)
        out[nu] = kept
    return out

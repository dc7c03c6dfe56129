"""fp64 PyTorch-CPU oracle of the MACE three-pass energy+force path (TEST INFRASTRUCTURE ONLY; see __init__.py).

What it restates (reference file:line):
  * the layer functions  receiver_chunk_mace.layer1 / layer2_energy (:237-256) and FastLayers (fast_layers.py:
    168-222): edge embedding, radial MLP x cutoff, channelwise TP summed on receivers, density normalisation,
    linear, skip_tp, symmetric contraction, product linear, readouts; the model's arithmetic is mace-torch's
    (third-party, not installed: see mace_onegpu/model.py for the restated definition);
  * the full-graph energy and autograd forces (what tests/gpu/test_threepass.py:66-71 compares against);
  * ReceiverChunkMACE.compute (receiver_chunk_mace.py:278-386): passes A (H1), B (layer-2 energy, forces,
    G1 = dE2/dh1), C (layer 1 with grad, loss scale*R1 + G1.h1), force accumulation (:272-276);
  * the tabulated radial weights: spline_radial._sample (spline_radial.py:116-151, fp64, central differences,
    eps = 1e-5 (r_hi - r_lo), ordered pairs sender-major), conv_spline.build_tables (conv_spline.py:230-249,
    TG = h dW/dr) and the cubic-Hermite lookup of spline_w._w_fwd (spline_w.py:18-50, clamp to M - 1 - 1e-4).
The TP and the symmetric contraction are evaluated densely from the coupling tensors (einsum), independently of
the sparse term lists that the GPU kernels are generated from.
Pinned by (tests/test_oracle.py, tests/test_oracle_conventions.py, tests/test_o3.py):
  * rotation/translation/permutation invariance of E and covariance of F (fails for a wrong coupling sign, a
    transposed coupling or a wrong SH), finite differences of E against F, three-pass == full graph and chunk
    invariance (the reference's own criteria, test_threepass.py:66-88);
  * the SH against scipy.special, the coupling tensors' equivariance, the symmetric-contraction basis against the
    dimension of the equivariant space;
  * bessel: orthonormality on [0, r_max] with weight r^2 (quadrature); poly_cutoff: the unique degree-(p+2)
    polynomial with f(0) = 1 and f = f' = f'' = 0 at r_max; silu_n: Gauss-Hermite quadrature;
  * the e3nn normalisations of radial_mlp, per_l_linear, multi_source_linear, skip_tp, node_embedding, the
    readouts, density_z and every channelwise-TP path: unit second moment for unit-variance inputs (Monte Carlo);
  * the density normalisation: the closed forms rho = 0 (w = 0) and rho = sum f_cut (saturated tanh);
  * E_i = e0 + shift + scale (R1 + R2): affine in scale / shift / E0, three-pass and full graph alike.
Parity unpinned: absolute values against mace-torch itself (not installed); the basis of the real harmonics
(z-polar here) and of the symmetric contraction are reparametrisations of random-init weights.
"""
import math

import numpy as np
import torch

F64 = torch.float64
SILU_NORM_QUAD = None     # computed lazily by quadrature (independent of the product's constant)


def silu_norm():
    global SILU_NORM_QUAD
    if SILU_NORM_QUAD is None:
        import warnings
        from scipy.integrate import quad
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            v, _ = quad(lambda z: (z / (1 + math.exp(-z))) ** 2 * math.exp(-z * z / 2) / math.sqrt(2 * math.pi),
                        -40, 40, epsabs=1e-15, epsrel=1e-14, limit=500)
        SILU_NORM_QUAD = 1.0 / math.sqrt(v)
    return SILU_NORM_QUAD


# ----------------------------------------------------------------------------- edge embedding
def sh(vec):
    """Real SH l<=3, component normalisation, z-polar, m = -l..l; vec [E, 3] -> [E, 16] (differentiable)."""
    u = vec / torch.linalg.vector_norm(vec, dim=-1, keepdim=True)
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    x2, y2, z2 = x * x, y * y, z * z
    s = math.sqrt
    return torch.stack([
        torch.ones_like(x),
        s(3) * y, s(3) * z, s(3) * x,
        s(15) * x * y, s(15) * y * z, s(5) / 2 * (2 * z2 - x2 - y2), s(15) * x * z, s(15) / 2 * (x2 - y2),
        s(70) / 4 * y * (3 * x2 - y2), s(105) * x * y * z, s(42) / 4 * y * (4 * z2 - x2 - y2),
        s(7) / 2 * z * (2 * z2 - 3 * x2 - 3 * y2), s(42) / 4 * x * (4 * z2 - x2 - y2), s(105) / 2 * z * (x2 - y2),
        s(70) / 4 * x * (x2 - 3 * y2)], -1)


def bessel(r, r_max, n):
    """mace BesselBasis: sqrt(2/r_max) sin(k pi r / r_max) / r, k = 1..n; r [E] -> [E, n]."""
    k = torch.arange(1, n + 1, dtype=r.dtype)
    return math.sqrt(2.0 / r_max) * torch.sin(k[None, :] * math.pi * r[:, None] / r_max) / r[:, None]


def poly_cutoff(r, r_max, p):
    """mace PolynomialCutoff: 1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2) for x = r/r_max < 1."""
    x = r / r_max
    env = 1.0 - (p + 1) * (p + 2) / 2.0 * x ** p + p * (p + 2.0) * x ** (p + 1) - p * (p + 1) / 2.0 * x ** (p + 2)
    return env * (x < 1.0).to(r.dtype)


def silu_n(z):
    """e3nn normalize2mom(silu): silu scaled to unit second moment under z ~ N(0, 1)."""
    return silu_norm() * torch.nn.functional.silu(z)


def radial_mlp(B, Ws):
    """e3nn FullyConnectedNet (mace's conv_tp_weights, receiver_chunk_mace.py:230-234 via
    fast_layers.py:150-156): hidden h <- silu_n(h @ W / sqrt(fan_in)); the last layer is linear."""
    h = B
    for j, W in enumerate(Ws):
        h = h @ W / math.sqrt(W.shape[0])
        if j < len(Ws) - 1:
            h = silu_n(h)
    return h


def density_z(B, w):
    """Pre-activation of mace's density_fn (a one-layer FullyConnectedNet, fast_layers.py:179-185):
    z = B @ w / sqrt(n_bessel); B [E, nb], w [nb, 1] -> [E]."""
    return (B @ w / math.sqrt(B.shape[1]))[:, 0]


def edge_density(B, w, f):
    """Edge density d_e = tanh(z_e^2) * f_cut(r_e) (fast_layers.py:181-183, cutoff branch :190-192)."""
    return torch.tanh(density_z(B, w) ** 2) * f


# ----------------------------------------------------------------------------- equivariant operations
def comp_offsets(ls):
    out, o = [], 0
    for l in ls:
        out.append(o)
        o += 2 * l + 1
    return out, o


def channelwise_tp(W, X, Y, send, paths, in_ls, coupling):
    """Per edge: mid[e, seg w, M, c] = sum_{a,b} coupling(l1,l2,l3)[a,b,M] W[e,w,c] X[send_e, l1 a, c] Y[e, l2 b].
    W [E, nW, C], X [n, nX, C], Y [E, 16] -> [E, nO, C] (mid components in path order)."""
    xo, _ = comp_offsets(in_ls)
    outs = []
    Xs = X[send]
    for w, (i1, l1, l2, l3) in enumerate(paths):
        Cw = torch.as_tensor(coupling(l1, l2, l3), dtype=W.dtype)
        xa = Xs[:, xo[i1]:xo[i1] + 2 * l1 + 1, :] * W[:, w, None, :]
        cy = torch.einsum("abM,eb->eaM", Cw, Y[:, l2 * l2:(l2 + 1) ** 2])
        outs.append(torch.einsum("eaM,eac->eMc", cy, xa))
    return torch.cat(outs, 1)


def scatter_sum(x, idx, n):
    out = torch.zeros((n,) + tuple(x.shape[1:]), dtype=x.dtype)
    return out.index_add(0, idx, x)


def sym_path_poly(x, path, L, in_ls, coupling):
    """x [n, 16, C] -> P [n, 2L+1, C] for one coupling path (see mace_onegpu.o3.path_tensor)."""
    xo, _ = comp_offsets(in_ls)
    off = {l: xo[i] for i, l in enumerate(in_ls)}

    def seg(l):
        return x[:, off[l]:off[l] + 2 * l + 1, :]
    if path[0] == "1":
        return seg(path[1])
    if path[0] == "2":
        _, l1, l2 = path
        C = torch.as_tensor(coupling(l1, l2, L), dtype=x.dtype)
        return torch.einsum("abM,nac,nbc->nMc", C, seg(l1), seg(l2))
    _, l1, l2, J, l3 = path
    C1 = torch.as_tensor(coupling(l1, l2, J), dtype=x.dtype)
    C2 = torch.as_tensor(coupling(J, l3, L), dtype=x.dtype)
    Z = torch.einsum("abj,nac,nbc->njc", C1, seg(l1), seg(l2))
    return torch.einsum("jdM,njc,ndc->nMc", C2, Z, seg(l3))


def symmetric_contraction(x, species, weights, paths, out_ls, in_ls, coupling):
    """mace SymmetricContraction (correlation = max nu): out[n, L-block, c] = sum_nu sum_k W[s_n, k, c] P_k(x)."""
    outs = []
    for L in out_ls:
        acc = 0
        for nu, plist in paths[L].items():
            Wt = weights[(L, nu)][species]                     # [n, K, C]
            for k, path in enumerate(plist):
                acc = acc + Wt[:, k, :].unsqueeze(1) * sym_path_poly(x, path, L, in_ls, coupling)
        outs.append(acc)
    return torch.cat(outs, 1)


def per_l_linear(x, ls, Wl, C):
    """e3nn Linear between equal irreps (one weight [C, C] per irrep l in ls, in order; x [n, comps, C]):
    y = x_l @ W_l / sqrt(C) (mace's linear_up, products[k].linear)."""
    offs, _ = comp_offsets(ls)
    return torch.cat([x[:, o:o + 2 * l + 1, :] @ Wl[i] / math.sqrt(C) for i, (o, l) in enumerate(zip(offs, ls))], 1)


def multi_source_linear(blocks, Ws):
    """e3nn Linear into one output irrep fed by several input segments of that irrep (layer 2's interaction
    linear, mid irreps -> target): y = sum_j x_j @ W_j / sqrt(C * n_src); blocks [n, 2l+1, C] each."""
    fan_in = blocks[0].shape[-1] * len(blocks)
    acc = 0
    for x, W in zip(blocks, Ws):
        acc = acc + x @ W
    return acc / math.sqrt(fan_in)


def node_embedding(attrs, emb):
    """mace LinearNodeEmbeddingBlock, an e3nn Linear n_el x 0e -> C x 0e: attrs [n, n_el] @ emb / sqrt(n_el)."""
    return attrs @ emb / math.sqrt(emb.shape[0])


def skip_tp(x, y, W):
    """e3nn FullyConnectedTensorProduct(x irreps, n_el x 0e, x irreps) (mace's skip_tp, fast_layers.py:41-105):
    out[n, m, d] = sum_{c, s} x[n, m, c] y[n, s] W[c, s, d] / sqrt(C * n_el).  y is either the node attributes
    [n, n_el] (float) or, for one-hot attributes, the species index per node [n] (long)."""
    C, ne = W.shape[0], W.shape[1]
    if y.dtype == torch.long:
        Wn = W[:, y, :].permute(1, 0, 2)                       # [n, C_in, C_out]
    else:
        Wn = torch.einsum("ns,csd->ncd", y, W)
    return torch.einsum("nmc,ncd->nmd", x, Wn) / math.sqrt(C * ne)


def readout_linear(h0, w):
    """mace LinearReadoutBlock (layer 1): h[0e] @ w / sqrt(C)."""
    return h0 @ w / math.sqrt(w.shape[0])


def readout_mlp(h0, W1, w2):
    """mace NonLinearReadoutBlock (layer 2): silu_n(h @ W1 / sqrt(C)) @ w2 / sqrt(n_hidden)."""
    return silu_n(h0 @ W1 / math.sqrt(W1.shape[0])) @ w2 / math.sqrt(w2.shape[0])


# ----------------------------------------------------------------------------- model access
class RefModel:
    """fp64 view of a mace_onegpu.model.MaceModel: parameters, architecture numbers and coupling tables."""

    def __init__(self, model, coupling):
        sp = model.spec
        self.C, self.ne, self.nb = sp.C, sp.num_elements, sp.num_bessel
        self.r_max, self.p, self.scale, self.shift = sp.r_max, sp.p_cutoff, sp.scale, sp.shift
        self.P = {k: v.detach().to("cpu", F64) for k, v in model.p.items()}
        self.e0 = model.e0.detach().to("cpu", F64)
        t = model.tables
        self.tp1, self.tp2, self.sc1, self.sc2, self.lin2_src = t.tp1, t.tp2, t.sc1, t.sc2, t.lin2_src
        self.coupling = coupling
        self.nlayers_r = len(sp.radial_mlp) + 1
        # optional radial networks per ordered element pair (sender column, receiver column) -> {block k: weight
        # list}; pairs not listed use the model's own networks (mace_onegpu.model.MaceModel.pair_radial)
        pr = getattr(model, "pair_radial", None)
        self.pair_radial = None if pr is None else {
            (int(a), int(b)): {k: [w.detach().to("cpu", F64) for w in ws] for k, ws in d.items()}
            for (a, b), d in pr.items()}

    def astype(self, dtype):
        """A copy whose parameters are held in `dtype` (the fp32 CPU baseline evaluates the same functions)."""
        import copy
        m = copy.copy(self)
        m.P = {k: v.to(dtype) for k, v in self.P.items()}
        m.e0 = self.e0.to(dtype)
        return m

    def radial_W(self, k, send_col=None, recv_col=None):
        """Radial-network weights of block k; with element columns, those of the ordered pair (sender, receiver)."""
        if self.pair_radial is not None and send_col is not None:
            d = self.pair_radial.get((int(send_col), int(recv_col)))
            if d is not None and k in d:
                return d[k]
        return [self.P[f"i{k}_r{j}"] for j in range(self.nlayers_r)]

    def sym_weights(self, k, Ls):
        return {(L, nu): self.P[f"p{k}_w_L{L}_nu{nu}"] for L in Ls for nu in (1, 2, 3)
                if f"p{k}_w_L{L}_nu{nu}" in self.P}


class Tables64:
    """fp64 Hermite tables of W(r; ordered pair) per interaction block, restating conv_spline.build_tables."""

    def __init__(self, m, species_cols, n_grid=512, r_lo=0.5):
        self.M, self.r_lo, self.r_hi = n_grid, r_lo, m.r_max
        self.h = (self.r_hi - r_lo) / (n_grid - 1)
        self.inv_h = 1.0 / self.h
        S = len(species_cols)
        self.S = S
        col2s = torch.zeros(m.ne, dtype=torch.long)
        col2s[torch.as_tensor(species_cols)] = torch.arange(S)
        self.col2s = col2s
        r = torch.linspace(r_lo, self.r_hi, n_grid, dtype=F64)
        eps = 1e-5 * (self.r_hi - r_lo)
        self.TV, self.TG = [], []
        for k in range(2):
            tv, tg = [], []
            # ordered pairs p = a * S + b, sender species a outer, receiver b inner (spline_radial._sample,
            # spline_radial.py:121-151); without per-pair networks every pair holds the same function
            for a in range(S):
                for b in range(S):
                    Ws = m.radial_W(k, species_cols[a], species_cols[b])

                    def f(rr):
                        return radial_mlp(bessel(rr, m.r_max, m.nb), Ws) * poly_cutoff(rr, m.r_max, m.p)[:, None]
                    v0, vp, vm = f(r), f(r + eps), f(r - eps)
                    tv.append(v0)
                    tg.append((vp - vm) / (2 * eps) * self.h)
            self.TV.append(torch.cat(tv, 0))                       # [P*M, D]
            self.TG.append(torch.cat(tg, 0))

    def astype(self, dtype):
        import copy
        t = copy.copy(self)
        t.TV = [v.to(dtype) for v in self.TV]
        t.TG = [v.to(dtype) for v in self.TG]
        return t

    def lookup(self, k, r, pair):
        """spline_w._w_fwd in fp64: x = clamp((r - r_lo) inv_h, 0, M - 1 - 1e-4), Hermite on [k, k+1]."""
        x = torch.clamp((r - self.r_lo) * self.inv_h, 0.0, (self.M - 1) - 1e-4)
        kf = torch.floor(x.detach())
        t = (x - kf)[:, None]
        row = pair * self.M + kf.long()
        TV, TG = self.TV[k], self.TG[k]
        t2, t3 = t * t, t * t * t
        return ((2 * t3 - 3 * t2 + 1) * TV[row] + (t3 - 2 * t2 + t) * TG[row]
                + (-2 * t3 + 3 * t2) * TV[row + 1] + (t3 - t2) * TG[row + 1])


# ----------------------------------------------------------------------------- layers on a local graph
def _edge(m, vec):
    r = torch.linalg.vector_norm(vec, dim=-1)
    Y = sh(vec)
    B = bessel(r, m.r_max, m.nb)
    f = poly_cutoff(r, m.r_max, m.p)
    return r, Y, B, f


def _weights_density(m, k, r, B, f, tables, pair, cs=None, cr=None):
    """Radial weights W [E, nW C] (table lookup, or the radial network of each edge's ordered element pair
    (cs[e], cr[e]) = (sender, receiver) column) and the edge density."""
    if tables is not None:
        W = tables.lookup(k, r, pair)
    elif m.pair_radial is None:
        W = radial_mlp(B, m.radial_W(k)) * f[:, None]
    else:
        code = cs * m.ne + cr
        W = None
        for c in torch.unique(code).tolist():
            sel = code == c
            w = radial_mlp(B[sel], m.radial_W(k, c // m.ne, c % m.ne)) * f[sel][:, None]
            if W is None:
                W = torch.zeros(B.shape[0], w.shape[1], dtype=w.dtype)
            W = W.index_put((torch.nonzero(sel).squeeze(1),), w)
        if W is None:
            W = torch.zeros(0, m.P[f"i{k}_r{m.nlayers_r - 1}"].shape[1], dtype=B.dtype)
    return W, edge_density(B, m.P[f"i{k}_dens"], f)


def layer1_message(m, spec_nodes, nC, send, recv, vec, tables=None, pair=None):
    """Layer-1 interaction (RealAgnosticDensityInteractionBlock, fast_layers.py:168-200) up to the message
    before skip_tp: linear(sum_e TP(W_e, X[send_e], Y_e)) / (rho + 1) [nC, 16, C], rho = sum_e d_e."""
    C = m.C
    r, Y, B, f = _edge(m, vec)
    W, d = _weights_density(m, 0, r, B, f, tables, pair, spec_nodes[send], spec_nodes[recv])
    W = W.reshape(-1, m.tp1["nW"], C)
    onehot = torch.nn.functional.one_hot(spec_nodes, m.ne).to(m.P["emb"].dtype)
    X = per_l_linear(node_embedding(onehot, m.P["emb"])[:, None, :], [0], m.P["i0_up"], C)
    mji = channelwise_tp(W, X, Y, send, m.tp1["paths"], m.tp1["in_ls"], m.coupling)
    A = scatter_sum(mji, recv, nC)
    rho = scatter_sum(d, recv, nC)
    return per_l_linear(A, m.tp1["mid_ls"], m.P["i0_lin"], C) / (rho[:, None, None] + 1)


def layer1(m, spec_nodes, nC, send, recv, vec, tables=None, pair=None):
    """h1 [nC, 4, C] of the receivers (local nodes 0..nC-1); spec_nodes: model element index per local node."""
    M = layer1_message(m, spec_nodes, nC, send, recv, vec, tables, pair)
    s = spec_nodes[:nC]
    offs, _ = comp_offsets(m.tp1["mid_ls"])
    M = torch.cat([skip_tp(M[:, o:o + 2 * l + 1, :], s, m.P["i0_skip"][i])
                   for i, (o, l) in enumerate(zip(offs, m.tp1["mid_ls"]))], 1)
    Bsc = symmetric_contraction(M, s, m.sym_weights(0, (0, 1)), m.sc1, [0, 1], [0, 1, 2, 3], m.coupling)
    return per_l_linear(Bsc, [0, 1], m.P["p0_lin"], m.C)


def readout1(m, h1):
    return readout_linear(h1[:, 0, :], m.P["r0"])


def layer2_energy(m, spec_nodes, nC, send, recv, vec, h1_nodes, tables=None, pair=None):
    """Per-receiver layer-2 energy R2(h2) [nC]; h1_nodes [n_nodes, 4, C] for every local node."""
    C = m.C
    s = spec_nodes[:nC]
    sc = skip_tp(h1_nodes[:nC, 0:1, :], s, m.P["i1_skip"])[:, 0, :]
    X = per_l_linear(h1_nodes, [0, 1], m.P["i1_up"], C)
    r, Y, B, f = _edge(m, vec)
    W, d = _weights_density(m, 1, r, B, f, tables, pair, spec_nodes[send], spec_nodes[recv])
    W = W.reshape(-1, m.tp2["nW"], C)
    mji = channelwise_tp(W, X, Y, send, m.tp2["paths"], m.tp2["in_ls"], m.coupling)
    A = scatter_sum(mji, recv, nC)
    rho = scatter_sum(d, recv, nC)
    mo, _ = comp_offsets(m.tp2["mid_ls"])
    outs = []
    for l in [0, 1, 2, 3]:
        src = m.lin2_src[l]
        Wl = m.P[f"i1_lin_l{l}"]
        outs.append(multi_source_linear([A[:, mo[w]:mo[w] + 2 * l + 1, :] for w in src],
                                        [Wl[j] for j in range(len(src))]))
    M2 = torch.cat(outs, 1) / (rho[:, None, None] + 1)
    B2 = symmetric_contraction(M2, s, m.sym_weights(1, (0,)), m.sc2, [0], [0, 1, 2, 3], m.coupling)
    h2 = per_l_linear(B2, [0], m.P["p1_lin"], C)[:, 0, :] + sc
    return readout_mlp(h2, m.P["r1_w1"], m.P["r1_w2"])


# ----------------------------------------------------------------------------- full graph
def min_image(v, box):
    return v - box * torch.round(v / box)


def energy_full(m, pos, box, spec, recv, send, tables=None, species_cols=None):
    """Per-atom energies [N] of the whole periodic system (every atom a receiver and a node).
    pos [N, 3] fp64 (may require grad), box [3], spec [N] element index, recv/send [E] edge endpoints."""
    box = torch.as_tensor(box, dtype=F64)
    # the periodic image shift is a constant of the configuration: taken from the detached positions
    raw = (pos[recv] - pos[send]).detach()
    vec = pos[recv] - pos[send] + (min_image(raw, box) - raw)
    N = pos.shape[0]
    pair = None
    if tables is not None:
        c2s = tables.col2s[spec]
        pair = c2s[send] * tables.S + c2s[recv]
    h1 = layer1(m, spec, N, send, recv, vec, tables, pair)
    e1 = readout1(m, h1)
    e2 = layer2_energy(m, spec, N, send, recv, vec, h1, tables, pair)
    return m.e0[spec] + m.shift + m.scale * (e1 + e2)


def energy_forces_full(m, pos, box, spec, recv, send, tables=None):
    pos = torch.as_tensor(pos, dtype=F64).clone().requires_grad_(True)
    spec = torch.as_tensor(spec, dtype=torch.long)
    recv = torch.as_tensor(recv, dtype=torch.long)
    send = torch.as_tensor(send, dtype=torch.long)
    e = energy_full(m, pos, box, spec, recv, send, tables)
    E = e.sum()
    (g,) = torch.autograd.grad(E, [pos])
    return float(E.detach()), e.detach(), (-g).detach()


# ----------------------------------------------------------------------------- three-pass (ReceiverChunkMACE)
def local_graph(a, b, recv, send, loc):
    """LocalGraph (receiver_chunk_mace.py:175-193) without padding: nodes = [a, b) + unique outside senders."""
    sel = (recv >= a) & (recv < b)
    rg, sg = recv[sel], send[sel]
    nC = b - a
    C_ = torch.arange(a, b)
    loc[C_] = torch.arange(nC)
    su = torch.unique(sg)
    new = su[loc[su] < 0]
    loc[new] = torch.arange(nC, nC + new.numel())
    nodes = torch.cat([C_, new])
    ei_send, ei_recv = loc[sg].clone(), loc[rg].clone()
    loc[nodes] = -1
    return nodes, ei_send, ei_recv, rg, sg


def atom_energy_local(m, pos, box, spec, i, tables=None):
    """Energy of atom i (e0 + shift + scale (R1 + R2), eV) from its own neighbourhood only: layer 1 on i and its
    neighbours (the receivers whose h1 layer 2 of i reads), layer 2 on i.  Every atom within r_max of one of those
    receivers is within 2 r_max of i, so only that ball of the periodic system is read; the edge vectors are the
    fp64 minimum images x_recv - x_send and the neighbour test is the reference's dd < r_max^2, j != i
    (receiver_chunk_mace.py:114-165).  Equal to the whole-system evaluation (three_pass, energy_full) to fp64
    rounding, for any box larger than 2 r_max.  pos [N, 3] fp64 numpy, box [3], spec [N] element index."""
    pos = np.asarray(pos, dtype=np.float64)
    L = np.asarray(box, dtype=np.float64)
    rc2 = m.r_max ** 2

    def mic(v):
        return v - L * np.round(v / L)

    d = mic(pos - pos[i])
    ball = np.nonzero((d * d).sum(1) < (2 * m.r_max + 1e-6) ** 2)[0]           # includes i

    def neighbours(r):
        v = mic(pos[r] - pos[ball])
        keep = ((v * v).sum(1) < rc2) & (ball != r)
        return ball[keep]

    n1 = np.sort(neighbours(i))
    recv1 = np.concatenate([[i], n1])                                          # layer-1 receivers, i first
    loc = {int(a): k for k, a in enumerate(recv1)}
    rg, sg = [], []
    for r in recv1:
        for sj in neighbours(int(r)):
            rg.append(int(r))
            sg.append(int(sj))
    outside = sorted(set(sg) - set(loc))
    for a in outside:
        loc[a] = len(loc)
    nodes = torch.as_tensor(np.concatenate([recv1, np.asarray(outside, dtype=np.int64)]), dtype=torch.long)
    rg, sg = np.asarray(rg), np.asarray(sg)
    P = torch.as_tensor(pos, dtype=F64)
    Lt = torch.as_tensor(L, dtype=F64)
    spec_t = torch.as_tensor(np.asarray(spec), dtype=torch.long)
    lr = torch.as_tensor([loc[int(a)] for a in rg], dtype=torch.long)
    ls = torch.as_tensor([loc[int(a)] for a in sg], dtype=torch.long)
    vec1 = min_image(P[rg] - P[sg], Lt)
    pair1 = pair2 = None
    if tables is not None:
        c2s = tables.col2s[spec_t]
        pair1 = c2s[torch.as_tensor(sg)] * tables.S + c2s[torch.as_tensor(rg)]
    with torch.no_grad():
        h1 = layer1(m, spec_t[nodes], len(recv1), ls, lr, vec1, tables, pair1)
        sel = lr == 0                                                          # the edges received by i
        if tables is not None:
            pair2 = pair1[sel]
        e2 = layer2_energy(m, spec_t[nodes[:len(recv1)]], 1, ls[sel], lr[sel], vec1[sel], h1, tables, pair2)
        e1 = readout1(m, h1[:1])
    return float(m.e0[spec_t[i]] + m.shift + m.scale * (e1[0] + e2[0]))


def three_pass(m, pos, box, spec, recv, send, chunk, tables=None):
    """ReceiverChunkMACE.compute (receiver_chunk_mace.py:278-386) in fp64: returns (E, per-atom E, F)."""
    box = torch.as_tensor(box, dtype=F64)
    pos = torch.as_tensor(pos, dtype=F64)
    spec = torch.as_tensor(spec, dtype=torch.long)
    recv = torch.as_tensor(recv, dtype=torch.long)
    send = torch.as_tensor(send, dtype=torch.long)
    N = pos.shape[0]
    loc = torch.full((N,), -1, dtype=torch.long)
    F = torch.zeros(N, 3, dtype=F64)
    eat = m.e0[spec] + m.shift
    c2s = tables.col2s[spec] if tables is not None else None
    H1 = torch.zeros(N, 4, m.C, dtype=F64)
    graphs = []
    for a in range(0, N, chunk):
        b = min(a + chunk, N)
        nodes, ls, lr, rg, sg = local_graph(a, b, recv, send, loc)
        vec = min_image(pos[rg] - pos[sg], box)
        pair = None if tables is None else c2s[sg] * tables.S + c2s[rg]
        graphs.append((a, b, nodes, ls, lr, rg, sg, vec, pair))
    with torch.no_grad():                                              # pass A
        for (a, b, nodes, ls, lr, rg, sg, vec, pair) in graphs:
            H1[a:b] = layer1(m, spec[nodes], b - a, ls, lr, vec, tables, pair)
    G1 = torch.zeros_like(H1)
    for (a, b, nodes, ls, lr, rg, sg, vec, pair) in graphs:             # pass B
        v = vec.clone().requires_grad_(True)
        h1l = H1[nodes].clone().requires_grad_(True)
        e = layer2_energy(m, spec[nodes], b - a, ls, lr, v, h1l, tables, pair)
        eb = m.scale * e.sum()
        gv, gh = torch.autograd.grad(eb, [v, h1l])
        G1.index_add_(0, nodes, gh)
        F.index_add_(0, rg, -gv)
        F.index_add_(0, sg, gv)
        eat[a:b] += m.scale * e.detach()
    for (a, b, nodes, ls, lr, rg, sg, vec, pair) in graphs:             # pass C
        v = vec.clone().requires_grad_(True)
        h1 = layer1(m, spec[nodes], b - a, ls, lr, v, tables, pair)
        r1 = readout1(m, h1)
        loss = m.scale * r1.sum() + (G1[a:b] * h1).sum()
        (gv,) = torch.autograd.grad(loss, [v])
        F.index_add_(0, rg, -gv)
        F.index_add_(0, sg, gv)
        eat[a:b] += m.scale * r1.detach()
    return float(eat.sum()), eat, F, H1, G1

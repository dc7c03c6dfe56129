"""Per-chunk layer pipelines of the three-pass evaluation on the MI355X kernels.

Mirrors the reference's FastLayers (fast_layers.py:108-222): the exact node-level speed-ups (species-block
skip_tp, receiver-only node operations, tabulated radial weights) and the layer functions used by the three passes.
Here every pass is an explicit sequence of HIP kernels with a hand-derived backward (no autograd):

  layer 1 (pass A, and pass C with its backward):
    geometry -> conv1 (spline W x TP x receiver sum, density) -> [linear o skip_tp] per species / (rho + 1)
    -> symmetric contraction -> product linear -> (pass C) readout 1 and g_h1 = scale dR1/dh1 + G1r
    -> backward through the same chain -> per-edge dL/dv
  layer 2 (pass B):
    skip_tp(h1) per species, linear_up(H1[nodes]) -> conv2 -> linear / (rho + 1) -> symmetric contraction
    -> product linear + sc -> readout 2 -> backward -> per-edge dL/dv, G1[nodes] += dL/dh1

linear and skip_tp of layer 1 are both linear per (l, species) and act back to back, so they are applied as one
128x128 block per (l, species) (W_lin_l @ W_skip_l,s); the result is the same map.
"""
import ctypes
import math

import torch

from . import codegen, model as mm
from ._lib import K, stream

C = 128
NCB = 8
SRC = 3                         # max K-chunks of one linear output component (mm_linear)
NODE_KERNELS = ("linear", "symc1_fwd", "symc1_bwd", "symc2_fwd", "symc2_bwd")
ACE_H = 64                      # hidden features of the layer-1 ACE kernels (csrc/ace.hip)
ACE_MAX_S = 4                   # species per system of the layer-1 ACE kernels


def ace_gb_order(n_species):
    """Column order of dL/dB that mm_ace1_bwd reads (its MFMA operand order): position s * 64 + 16 g + k holds
    feature q = 4 k + g of species block s (g < 4, k < 16), so that each lane's 16 operands are contiguous."""
    p = torch.arange(n_species * ACE_H)
    s, g, k = p // ACE_H, (p % ACE_H) // 16, p % 16
    return s * ACE_H + 4 * k + g


def split3_bf16(W):
    """fp32 W -> (W0, W1, W2) bf16 with W0 = bf16(W), W1 = bf16(W - W0), W2 = bf16(W - W0 - W1) (round to nearest
    even; the differences are exact in fp32): |W - W0 - W1 - W2| <= 2^-27 |W|."""
    W = W.to(torch.float32)
    w0 = W.to(torch.bfloat16)
    r1 = W - w0.float()
    w1 = r1.to(torch.bfloat16)
    w2 = (r1 - w1.float()).to(torch.bfloat16)
    return w0, w1, w2


def mfma_block(W):
    """[128, 128] (k, n) -> flat bf16 [3 * 16384]: the three planes of split3_bf16(W), each in the LDS order of
    mm_linear's B operand: W[k][n] with k = 32 t + 8 g + u, n = 16 nt + i at (((t * 8 + nt) * 4 + g) * 16 + i) * 8
    + u, so that the 16 lanes (i, g) of one 16-byte LDS read take 256 consecutive bytes (no bank conflicts)."""
    def order(P):
        return P.reshape(4, 4, 8, 8, 16).permute(0, 3, 1, 4, 2).reshape(-1)   # [t, g, u, nt, i] -> [t, nt, g, i, u]
    return torch.cat([order(p) for p in split3_bf16(W.reshape(128, 128))]).contiguous()


def host_ints(vals):
    arr = (ctypes.c_int * len(vals))(*vals)
    return arr


class LinPlan:
    """Component table of one mm_linear launch."""

    def __init__(self, comps):
        # comps: list of (out_off, [(in_off, w_idx), ...])
        self.n = len(comps)
        nsrc, inoff, widx, outoff = [], [], [], []
        for out_off, srcs in comps:
            assert 1 <= len(srcs) <= SRC
            nsrc.append(len(srcs))
            for q in range(SRC):
                io, wi = srcs[q] if q < len(srcs) else (0, 0)
                inoff.append(io)
                widx.append(wi)
            outoff.append(out_off)
        self.nsrc, self.inoff = host_ints(nsrc), host_ints(inoff)
        self.widx, self.outoff = host_ints(widx), host_ints(outoff)
        # work of one launch per row: 128 x 128 products, distinct input blocks read, distinct weight blocks
        self.k_sum = sum(nsrc)
        self.n_in = len({io for _, srcs in comps for io, _ in srcs})
        self.n_w = len({wi for _, srcs in comps for _, wi in srcs})


def comp_of(ls):
    out, o = [], 0
    for l in ls:
        out.append(o)
        o += 2 * l + 1
    return out, o


def sender_csr(g):
    """(rowptr int32 [n_nodes + 1], edge index int32 [nE]) of chunk g's edges grouped by local sender, ascending edge
    index within a sender: the fixed summation order of the deterministic sender-feature gradient.  A chunk that
    carries them (the graph executor's static chunk) is used as is."""
    if getattr(g, "sender_rowptr", None) is not None:
        return g.sender_rowptr, g.sender_perm
    ls = g.ls[:g.nE].long()
    perm = torch.argsort(ls, stable=True).to(torch.int32)
    rp = torch.zeros(g.n_nodes + 1, dtype=torch.int32, device=ls.device)
    rp[1:] = torch.cumsum(torch.bincount(ls, minlength=g.n_nodes), 0).to(torch.int32)
    return rp, perm


class FastLayers:
    """Device constants of the model for a set of present species (model element columns) and the layer pipelines.

    species_cols: sorted model element indices present in the system (the reference's `cols`,
    mliap_threepass.py:217); spline_grid: knots M of the radial-weight tables (reference default 512)."""

    def __init__(self, model, species_cols, spline_grid=512, r_lo=0.5, device="cuda", ace_layer1=True,
                 deterministic=False):
        self.dev = torch.device(device)
        # deterministic=True: pass B sums the sender-feature gradient per sender in a fixed order (mm_conv2_bwd_det
        # + mm_gather_rows_csr) instead of with float atomics, so repeated evaluations are bitwise identical; it
        # costs a [edges, 512] fp32 buffer per chunk workspace and the per-chunk sender sort
        self.deterministic = bool(deterministic)
        sp = model.spec
        self.spec = sp
        self.cols = [int(c) for c in species_cols]
        S = len(self.cols)
        self.S = S
        ne = sp.num_elements
        P = {k: v.detach().to("cpu", torch.float64) for k, v in model.p.items()}
        self.tables = model.tables
        dev = self.dev
        f32 = dict(dtype=torch.float32, device=dev)
        col2s = torch.full((ne,), -1, dtype=torch.int32)
        col2s[torch.as_tensor(self.cols)] = torch.arange(S, dtype=torch.int32)
        self.col2s = col2s.to(dev)
        # -------- layer 1 node features per species: linear_up(node_embedding(onehot))
        emb = P["emb"][self.cols] / math.sqrt(ne)
        self.Xs1 = (emb @ P["i0_up"][0] / math.sqrt(C)).to(**f32).contiguous()
        # -------- GEMM weight blocks
        def blocks(mats):
            return torch.cat([mfma_block(m.to(torch.float32)) for m in mats]).to(dev)
        comb = [P["i0_lin"][l] / math.sqrt(C) @ (P["i0_skip"][l][:, c, :] / math.sqrt(C * ne))
                for c in self.cols for l in range(4)]                                   # block s*4 + l
        self.W_l1 = blocks(comb)
        self.W_l1T = blocks([m.T for m in comb])
        pl1 = [P["p0_lin"][l] / math.sqrt(C) for l in range(2)]
        self.W_p1, self.W_p1T = blocks(pl1), blocks([m.T for m in pl1])
        up2 = [P["i1_up"][l] / math.sqrt(C) for l in range(2)]
        self.W_up2, self.W_up2T = blocks(up2), blocks([m.T for m in up2])
        sk1 = [P["i1_skip"][:, c, :] / math.sqrt(C * ne) for c in self.cols]
        self.W_sk1, self.W_sk1T = blocks(sk1), blocks([m.T for m in sk1])
        src = self.tables.lin2_src
        lin2, self.lin2_block = [], {}
        for l in range(4):
            for j, w in enumerate(src[l]):
                self.lin2_block[(l, w)] = len(lin2)
                lin2.append(P[f"i1_lin_l{l}"][j] / math.sqrt(C * len(src[l])))
        self.W_lin2, self.W_lin2T = blocks(lin2), blocks([m.T for m in lin2])
        pl2 = [P["p1_lin"][0] / math.sqrt(C)]
        self.W_p2, self.W_p2T = blocks(pl2), blocks([m.T for m in pl2])
        # -------- symmetric contraction weights [S, paths, C] in the generated kernels' order
        def symc_w(k, paths, out_ls):
            rows = []
            for (L, nu, pth) in codegen.symc_path_order(paths, out_ls):
                j = paths[L][nu].index(pth)
                rows.append(P[f"p{k}_w_L{L}_nu{nu}"][:, j, :])                     # [ne, C]
            return torch.stack(rows, 1)[self.cols].to(**f32).contiguous()
        self.Wsc1 = symc_w(0, self.tables.sc1, [0, 1])
        self.Wsc2 = symc_w(1, self.tables.sc2, [0])
        # -------- readouts, density, energy constants
        self.r0s = (P["r0"] / math.sqrt(C)).to(**f32).contiguous()
        self.r1W1 = (P["r1_w1"] / math.sqrt(C)).to(**f32).contiguous()
        self.r1w2 = (P["r1_w2"] / math.sqrt(P["r1_w2"].shape[0])).to(**f32).contiguous()
        self.H_ro = P["r1_w2"].shape[0]
        self.dens = [(ctypes.c_float * sp.num_bessel)(*(P[f"i{k}_dens"][:, 0] / math.sqrt(sp.num_bessel)).tolist())
                     for k in range(2)]
        self.scale, self.shift = sp.scale, sp.shift
        # pass C's loss scale R1 + G1r . h1 has the h1-gradient G1r + scale w0 on the 0e block; through p0_lin^T the
        # constant part is the row scale w0 p0_lin[0]^T, added to gB after the linear has read G1r itself
        self.ro1_gB = (self.scale * (P["r0"] / math.sqrt(C)) @ pl1[0].T).to(**f32).contiguous()
        self.e0 = model.e0.detach().to(dev, torch.float64)
        # -------- spline tables (fp64 sampling on the GPU)
        self.M, self.r_lo, self.r_hi = int(spline_grid), float(r_lo), sp.r_max
        self.h = (self.r_hi - self.r_lo) / (self.M - 1)
        self.inv_h = 1.0 / self.h
        # one spline table per distinct radial network of the ordered pairs (sender s outer, receiver r inner):
        # pair_map[s * S + r] -> table.  This architecture has one network per block (every pair -> table 0); a
        # model with per-pair networks (model.pair_radial) gets one table per distinct network
        self.radial_sets, pm = self._pair_radial_sets(model, P)
        self.n_tab = len(self.radial_sets)
        self.pair_map = torch.tensor(pm, dtype=torch.int32, device=dev)
        self.tab = [self._build_table(P, k) for k in range(2)]
        # -------- layer 1 in the exact density-projection (ACE) form: per-edge ht x Y outer products on MFMA,
        # one GEMM per atom with the folded weights G[l, s_recv] (up to 4 species).  It factors W = ht(r) A3 with
        # one ht for all pairs, so per-pair networks take the spline-convolution path
        self.ace = bool(ace_layer1) and S <= ACE_MAX_S and self.n_tab == 1
        if self.ace:
            self._build_ace(P, comb)
        # -------- linear plans
        o1, _ = comp_of([0, 1, 2, 3])
        self.plan_l1 = LinPlan([((o1[l] + m) * C, [((o1[l] + m) * C, l)]) for l in range(4) for m in range(2 * l + 1)])
        self.plan_p1 = LinPlan([(j * C, [(j * C, 0 if j == 0 else 1)]) for j in range(4)])
        self.plan_sk1 = LinPlan([(0, [(0, 0)])])
        self.plan_p2 = LinPlan([(0, [(0, 0)])])
        mo, _ = comp_of(self.tables.tp2["mid_ls"])
        mid_ls = self.tables.tp2["mid_ls"]
        self.plan_lin2 = LinPlan([((o1[l] + m) * C, [((mo[w] + m) * C, self.lin2_block[(l, w)]) for w in src[l]])
                                  for l in range(4) for m in range(2 * l + 1)])
        self.plan_lin2T = LinPlan([((mo[w] + m) * C, [((o1[mid_ls[w]] + m) * C, self.lin2_block[(mid_ls[w], w)])])
                                   for w in range(len(mid_ls)) for m in range(2 * mid_ls[w] + 1)])
        self.nO1, self.nO2 = self.tables.tp1["nO"], self.tables.tp2["nO"]
        self.ws = None
        self.ktimer = None        # list of (name, units, start event, end event) while kernel timing is on
        self.ktimer_nodes = False

    # ------------------------------------------------------------------ per-launch timing (HIP events)
    def start_kernel_timing(self, node_kernels=False):
        """Time the edge kernels' launches with HIP events; node_kernels=True also times the linears and the
        symmetric contractions (many short launches: their events are kept out of a headline timing)."""
        self.ktimer = []
        self.ktimer_nodes = node_kernels

    def stop_kernel_timing(self):
        """{name: dict(launches, ms_total, units)} of the timed launches; synchronises."""
        torch.cuda.synchronize()
        out = {}
        for name, units, e0, e1 in self.ktimer or []:
            d = out.setdefault(name, dict(launches=0, ms_total=0.0, units=[]))
            d["launches"] += 1
            d["ms_total"] += e0.elapsed_time(e1)
            d["units"].append(units)
        self.ktimer = None
        return out

    def _timed(self, name, units, fn, *args):
        if self.ktimer is None or (name in NODE_KERNELS and not self.ktimer_nodes):
            return fn(*args)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn(*args)
        e1.record()
        self.ktimer.append((name, units, e0, e1))

    # ------------------------------------------------------------------ tables
    def _pair_radial_sets(self, model, P):
        """Distinct radial networks of the ordered species pairs of this system and the pair -> table map: a list
        of {k: [r0..r3] fp64} (table order) and pair_map[s * S + r] (s sender, r receiver; the reference's ordered
        pair index, spline_w.py:18-27)."""
        default = {k: [P[f"i{k}_r{j}"] for j in range(4)] for k in range(2)}
        pr = getattr(model, "pair_radial", None)
        sets, pm = [], []
        for a in self.cols:
            for b in self.cols:
                d = pr.get((a, b)) if pr is not None else None
                ws = {k: [w.detach().to("cpu", torch.float64) for w in d[k]] if d is not None and k in d
                      else default[k] for k in range(2)}
                for t, other in enumerate(sets):
                    if all(torch.equal(x, y) for k in range(2) for x, y in zip(ws[k], other[k])):
                        pm.append(t)
                        break
                else:
                    pm.append(len(sets))
                    sets.append(ws)
        return sets, pm

    def _build_table(self, P, k):
        """conv_spline.build_tables / spline_radial._sample on the GPU in fp64, then per-interval coefficients, one
        table per distinct radial network (self.radial_sets)."""
        dev = self.dev
        nW = self.tables.tp1["nW"] if k == 0 else self.tables.tp2["nW"]
        D = nW * C
        M = self.M
        r = torch.linspace(self.r_lo, self.r_hi, M, dtype=torch.float64, device=dev)
        eps = 1e-5 * (self.r_hi - self.r_lo)
        pts = torch.cat([r, r + eps, r - eps]).contiguous()
        coef = torch.empty(NCB * self.n_tab * (M - 1) * nW * 16 * 4, dtype=torch.float32, device=dev)
        for tb, ws in enumerate(self.radial_sets):
            Ws = [w.to(dev).contiguous() for w in ws[k]]
            samples = torch.empty(3 * M, D, dtype=torch.float64, device=dev)
            K.mm_radial_mlp_f64(3 * M, pts, Ws[0], Ws[1], Ws[2], Ws[3], self.spec.num_bessel, Ws[1].shape[0], D,
                                self.spec.r_max, self.spec.p_cutoff, mm.SILU_NORM, samples, stream())
            K.mm_spline_coeffs(samples, M, nW, eps, self.h, tb, self.n_tab, coef, stream())
        return coef

    def _build_ace(self, P, comb):
        """Table of ht(r) = h3(r) f_cut(r) (the last hidden layer of layer 1's radial MLP times the cutoff) and the
        folded weights G[l, s_recv][(s, q), c'] = coef_l sum_c A3[q, l, c] Xs[s, c] Wcomb[s_recv, l][c, c']."""
        dev, S = self.dev, self.S
        H = P["i0_r1"].shape[0]
        assert H == ACE_H, "the ACE kernels are built for 64 hidden features"
        Ws = [P[f"i0_r{j}"].to(dev).contiguous() for j in range(3)]
        eye = (math.sqrt(H) * torch.eye(H, dtype=torch.float64, device=dev)).contiguous()
        M = self.M
        r = torch.linspace(self.r_lo, self.r_hi, M, dtype=torch.float64, device=dev)
        eps = 1e-5 * (self.r_hi - self.r_lo)
        pts = torch.cat([r, r + eps, r - eps]).contiguous()
        samples = torch.empty(3 * M, H, dtype=torch.float64, device=dev)
        K.mm_radial_mlp_f64(3 * M, pts, Ws[0], Ws[1], Ws[2], eye, self.spec.num_bessel, H, H, self.spec.r_max,
                            self.spec.p_cutoff, mm.SILU_NORM, samples, stream())
        self.tab_h = torch.empty((M - 1) * H * 4, dtype=torch.float32, device=dev)
        K.mm_spline_coeffs_flat(samples, M, H, eps, self.h, 0, self.tab_h, stream())
        # coupling of layer 1: node features 0e, so path w = l couples Y_m (m in l) to message component m
        coef = {}
        for (w, k, m, o, c) in self.tables.tp1["terms"]:
            l = self.tables.tp1["paths"][w][2]
            assert k == 0 and o == m and l * l <= m < (l + 1) ** 2 and self.tables.tp1["paths"][w][3] == l
            assert abs(coef.setdefault(l, c) - c) < 1e-12
        A3 = (P["i0_r3"] / math.sqrt(H)).view(H, 4, C)                                  # [q, l, c]
        emb = P["emb"][self.cols] / math.sqrt(self.spec.num_elements)
        Xs = emb @ P["i0_up"][0] / math.sqrt(C)                                          # [s, c]
        self.S_pad = S + (S % 2)
        nJ = self.S_pad // 2
        self.ace_nJ = nJ
        Gs, GTs = [], []
        for sr in range(S):
            for l in range(4):
                Wc = comb[sr * 4 + l]                                                    # [c, c']
                full = torch.zeros(self.S_pad * H, C, dtype=torch.float64)
                for s in range(S):
                    full[s * H:(s + 1) * H] = coef[l] * (A3[:, l, :] * Xs[s][None, :]) @ Wc
                for j in range(nJ):
                    blk = full[j * 128:(j + 1) * 128]
                    Gs.append(blk)
                    GTs.append(blk.T[:, ace_gb_order(2)])   # gB columns in mm_ace1_bwd's operand order
        self.W_ace = torch.cat([mfma_block(m.to(torch.float32)) for m in Gs]).to(dev)
        self.W_aceT = torch.cat([mfma_block(m.to(torch.float32)) for m in GTs]).to(dev)
        Kp = self.S_pad * H
        self.ace_Kp = Kp
        lm = [l for l in range(4) for _ in range(2 * l + 1)]
        self.plan_ace = LinPlan([(m * C, [(m * Kp + j * 128, lm[m] * nJ + j) for j in range(nJ)]) for m in range(16)])
        self.plan_aceT = LinPlan([(m * Kp + j * 128, [(m * C, lm[m] * nJ + j)]) for m in range(16) for j in range(nJ)])

    def layer1_cache(self, n_atoms):
        """Pass-A cache of the layer-1 message and density for n_atoms receivers (8 KiB per atom)."""
        return dict(M=torch.empty(n_atoms, 16 * C, dtype=torch.float32, device=self.dev),
                    rho=torch.empty(n_atoms, dtype=torch.float32, device=self.dev))

    # ------------------------------------------------------------------ workspace
    def workspace(self, nC, n_nodes, E):
        ws = self.ws
        if ws is not None and ws["nC"] >= nC and ws["nN"] >= n_nodes and ws["E"] >= E:
            return ws
        nC = max(nC, ws["nC"] if ws else 0)
        n_nodes = max(n_nodes, ws["nN"] if ws else 0)
        E = max(E, ws["E"] if ws else 0)
        self.ws = None
        torch.cuda.empty_cache()
        dev = self.dev
        f = dict(dtype=torch.float32, device=dev)
        i = dict(dtype=torch.int32, device=dev)
        ws = dict(nC=nC, nN=n_nodes, E=E)
        ws.update(e_u=torch.empty(E, 4, **f), e_pk=torch.empty(E, 4, **f),
                  e_recv=torch.empty(E, **i), e_dd=torch.empty(E, **f), part=torch.empty(NCB * E * 17, **f))
        if self.deterministic:
            ws["gXe"] = torch.empty(E, 4 * C, **f)       # per-edge dL/dX rows of mm_conv2_bwd_det
        # A (a layer's message, read by the linear after its convolution) and gA (its cotangent, written by the
        # transposed linear and read by the backward convolution) are never live together in a pass: one buffer
        A = torch.empty(nC * self.nO2 * C, **f)
        ws.update(A=A, gA=A,
                  rho=torch.empty(nC, **f), g_rho=torch.empty(nC, **f),
                  M=torch.empty(nC * 16 * C, **f), gM=torch.empty(nC * 16 * C, **f),
                  B=torch.empty(nC * 4 * C, **f), gB=torch.empty(nC * 4 * C, **f),
                  h=torch.empty(nC * 4 * C, **f), gh=torch.empty(nC * 4 * C, **f),
                  Xh=torch.empty(n_nodes * 4 * C, **f), gXh=torch.empty(n_nodes * 4 * C, **f))
        self.ws = ws
        return ws

    # ------------------------------------------------------------------ helpers
    def _lin(self, plan, inp, in_stride, out, out_stride, W, rows, in_rows=None, out_rows=None, scale=None,
             scale_mode=0, species=False, accumulate=0, w_group_stride=0, count_dev=None, in_cb=0):
        """count_dev (optional device int32 [1]): the row count read by the kernel, rows only sizing the launch.
        in_cb: input rows in 16-channel-block-major order with in_cb components (mm_conv2_bwd's dL/dX)."""
        ws = self.ws
        units = (rows, plan.k_sum, plan.n_in, plan.n, accumulate, plan.n_w * (self.S if species else 1))
        if species:
            self._timed("linear", units, K.mm_linear, inp, in_stride, in_rows, out, out_stride, out_rows, W, scale,
                        scale_mode, ws["lists"], ws["counts"], ws["lists_stride"], self.S, w_group_stride, rows,
                        accumulate, plan.n, plan.nsrc, plan.inoff, plan.widx, plan.outoff, in_cb, stream())
        else:
            self._timed("linear", units, K.mm_linear, inp, in_stride, in_rows, out, out_stride, out_rows, W, scale,
                        scale_mode, None, count_dev, 0, 1, 0, rows, accumulate, plan.n, plan.nsrc, plan.inoff,
                        plan.widx, plan.outoff, in_cb, stream())

    def _geometry(self, k, g):
        """Edge geometry of chunk g for interaction block k (LAMMPS pair vectors or positions)."""
        ws = self.ws
        sp = self.spec
        x_from_spec = 1 if k == 0 else 0          # layer-1 sender features depend on the species only
        if g.rij is not None:
            K.mm_edge_geom_rij(g.nE, g.E_dev, g.rij, g.pair_i, g.a, g.ls, ws["spec"], self.S, self.pair_map, self.dens[k],
                               sp.num_bessel, sp.r_max, sp.p_cutoff, self.M, self.r_lo, self.inv_h, x_from_spec,
                               ws["e_u"], None, ws["e_pk"], ws["e_recv"], ws["e_dd"], stream())
        else:
            K.mm_edge_geom_pos(g.nE, g.E_dev, g.pos, g.box_host, g.recv_local, g.a, g.ls, g.nodes, ws["spec"], self.S,
                               self.pair_map, self.dens[k], sp.num_bessel, sp.r_max, sp.p_cutoff, self.M, self.r_lo,
                               self.inv_h, x_from_spec, ws["e_u"], None, ws["e_pk"], ws["e_recv"],
                               ws["e_dd"], stream())

    def prepare(self, g):
        """Per-chunk node species and per-species receiver lists (g.node_spec: compact species of local nodes)."""
        ws = self.workspace(g.nC, g.n_nodes, g.nE)
        ws["spec"] = g.node_spec
        # per-species receiver lists of the chunk: built once per chunk object and shared by the three passes (the
        # HIP-graph executor loads them into its static chunk with the topology)
        if getattr(g, "lists", None) is None:
            g.lists = torch.empty(self.S * g.nC, dtype=torch.int32, device=self.dev)
            g.list_counts = torch.empty(self.S, dtype=torch.int32, device=self.dev)
            K.mm_species_lists(g.node_spec, g.nC, self.S, g.lists, g.nC, g.list_counts, stream())
        ws["lists"], ws["counts"], ws["lists_stride"] = g.lists, g.list_counts, g.nC
        return ws

    # ------------------------------------------------------------------ layer 1
    def _layer1_forward(self, g, h1_out, M_out, rho_out):
        """h1 of the chunk's receivers; M_out / rho_out receive the density-normalised message (symmetric
        contraction input) and the density."""
        ws = self.ws
        self._geometry(0, g)
        if self.ace:
            Kp = self.ace_Kp
            self._timed("ace1_fwd", (g.nE, g.nC, g.n_nodes), K.mm_ace1_fwd, g.rowptr, g.nC, ws["e_pk"], ws["e_u"],
                        self.tab_h, self.S, self.S_pad, ws["A"], rho_out, stream())
            self._lin(self.plan_ace, ws["A"], 16 * Kp, M_out, 16 * C, self.W_ace, g.nC, scale=rho_out, scale_mode=1,
                      species=True, w_group_stride=4 * self.ace_nJ)
        else:
            self._timed("conv1_fwd", (g.nE, g.nC, g.n_nodes), K.mm_conv1_fwd, g.rowptr, g.nC, ws["e_pk"],
                        ws["e_u"], self.Xs1, C, self.tab[0], self.n_tab, self.M, ws["A"], rho_out, stream())
            self._lin(self.plan_l1, ws["A"], 16 * C, M_out, 16 * C, self.W_l1, g.nC, scale=rho_out, scale_mode=1,
                      species=True, w_group_stride=4)
        self._timed("symc1_fwd", (g.nC,), K.mm_symc1_fwd, g.nC, M_out, 16 * C, ws["spec"], self.Wsc1, ws["B"], 4 * C,
                    stream())
        self._lin(self.plan_p1, ws["B"], 4 * C, h1_out, 4 * C, self.W_p1, g.nC)

    def pass_a(self, g, H1, cache=None):
        """H1[a:b] = h1 of the chunk's receivers (pass A, mliap_threepass.py:504-519).  With cache (dict of
        M [N, 16*128] and rho [N]) the layer-1 message and density of the chunk are kept for pass C."""
        ws = self.prepare(g)
        if cache is None:
            self._layer1_forward(g, H1[g.a:g.b], ws["M"], ws["rho"])
        else:
            self._layer1_forward(g, H1[g.a:g.b], cache["M"][g.a:g.b], cache["rho"][g.a:g.b])

    def _chunk_pair_forces(self, g, PF, forces):
        """Where the chunk's pair forces go: PF[e0:e1] of the whole system, or (forces = per-atom F, fp64 [N, 3])
        the chunk's own buffer, added to F by mm_chunk_forces after the pass."""
        if forces is None:
            return PF[g.e0:g.e1]
        ws = self.ws
        if ws.get("pf") is None or ws["pf"].shape[0] < ws["E"]:
            ws["pf"] = torch.empty(ws["E"], 3, dtype=torch.float32, device=self.dev)
        return ws["pf"][:g.nE]

    def _add_chunk_forces(self, g, pf, forces):
        srp, sperm = sender_csr(g)
        K.mm_chunk_forces(g.n_nodes, g.nC, g.rowptr, srp, sperm, g.nodes, pf, forces, stream())

    def pass_c(self, g, G1r, PF, eat, H1=None, cache=None, forces=None):
        """Layer 1 with gradient: eat[a:b] += scale R1(h1); PF[e0:e1] += d(scale R1 + G1r . h1)/dv
        (mliap_threepass.py:564-582).  With the pass-A cache (and H1), the layer-1 forward is not recomputed: the
        stored message, density and h1 are exactly what the recomputation would produce.  With forces (per-atom
        F, fp64 [N, 3]) the chunk's pair forces are added to F instead (PF unused)."""
        ws = self.prepare(g)
        if cache is None:
            h1, Mc, rho = ws["h"], ws["M"], ws["rho"]
            self._layer1_forward(g, h1, Mc, rho)
        else:
            h1, Mc, rho = H1[g.a:g.b], cache["M"][g.a:g.b], cache["rho"][g.a:g.b]
            self._geometry(0, g)
        D1 = 4 * C
        K.mm_readout1(g.nC, h1, D1, self.r0s, self.scale, eat[g.a:g.b], None, 0, None, 0, D1, stream())
        self._lin(self.plan_p1, G1r[g.a:g.b], D1, ws["gB"], D1, self.W_p1T, g.nC)
        ws["gB"].view(-1, D1)[:g.nC, :C].add_(self.ro1_gB)
        self._timed("symc1_bwd", (g.nC,), K.mm_symc1_bwd, g.nC, Mc, 16 * C, ws["spec"], self.Wsc1, ws["gB"], D1,
                    ws["gM"], 16 * C, rho, ws["g_rho"], stream())
        if self.ace:
            Kp = self.ace_Kp
            self._lin(self.plan_aceT, ws["gM"], 16 * C, ws["gA"], 16 * Kp, self.W_aceT, g.nC, scale=rho,
                      scale_mode=1, species=True, w_group_stride=4 * self.ace_nJ)
            self._timed("ace1_bwd", (g.nE, g.nC, g.n_nodes), K.mm_ace1_bwd, g.rowptr, g.nC, ws["e_pk"], ws["e_u"],
                        self.tab_h, self.S, self.S_pad, ws["gA"], self.inv_h, ws["part"], stream())
            n_part = 1
        else:
            self._lin(self.plan_l1, ws["gM"], 16 * C, ws["gA"], 16 * C, self.W_l1T, g.nC, scale=rho, scale_mode=1,
                      species=True, w_group_stride=4)
            self._timed("conv1_bwd", (g.nE, g.nC, g.n_nodes), K.mm_conv1_bwd, g.rowptr, g.nC, ws["e_pk"],
                        ws["e_u"], self.Xs1, C, self.tab[0], self.n_tab, self.M, self.inv_h, ws["gA"], ws["part"],
                        ws["E"] * 17, None, stream())
            n_part = NCB
        pf = self._chunk_pair_forces(g, PF, forces)
        K.mm_edge_grad(g.nE, g.E_dev, ws["part"], ws["E"] * 17, n_part, ws["g_rho"], ws["e_recv"], ws["e_dd"], ws["e_u"],
                       pf, 0 if forces is not None else 1, stream())
        if forces is not None:
            self._add_chunk_forces(g, pf, forces)

    # ------------------------------------------------------------------ layer 2
    def pass_b(self, g, H1x, G1, PF, eat, forces=None):
        """Layer-2 energy with gradient: eat[a:b] += scale R2(h2); PF[e0:e1] = dE2/dv; G1[nodes] += dE2/dh1
        (mliap_threepass.py:531-553).  With forces (per-atom F, fp64 [N, 3]) the chunk's pair forces are added to
        F instead (PF unused)."""
        ws = self.prepare(g)
        D1 = 4 * C
        h2, gh2, B2, gB2 = ws["h"], ws["gh"], ws["B"], ws["gB"]       # [nC, 128] views of the wider buffers
        # sc = skip_tp(h1_recv) per species (0e part only), written into h2; the receivers are g.nodes[:nC]
        self._lin(self.plan_sk1, H1x, D1, h2, C, self.W_sk1, g.nC, in_rows=g.nodes, species=True, w_group_stride=1)
        # node features of every local node: linear_up(H1x[nodes])
        self._lin(self.plan_p1, H1x, D1, ws["Xh"], D1, self.W_up2, g.n_nodes, in_rows=g.nodes, count_dev=g.N_dev)
        self._geometry(1, g)
        self._timed("conv2_fwd", (g.nE, g.nC, g.n_nodes), K.mm_conv2_fwd, g.rowptr, g.nC, ws["e_pk"], ws["e_u"],
                    ws["Xh"], D1, self.tab[1], self.n_tab, self.M, ws["A"], ws["rho"], stream())
        self._lin(self.plan_lin2, ws["A"], self.nO2 * C, ws["M"], 16 * C, self.W_lin2, g.nC, scale=ws["rho"],
                  scale_mode=1)
        self._timed("symc2_fwd", (g.nC,), K.mm_symc2_fwd, g.nC, ws["M"], 16 * C, ws["spec"], self.Wsc2, B2, C,
                    stream())
        self._lin(self.plan_p2, B2, C, h2, C, self.W_p2, g.nC, accumulate=1)
        K.mm_readout2(g.nC, h2, C, self.r1W1, self.r1w2, self.H_ro, mm.SILU_NORM, self.scale, eat[g.a:g.b], gh2, C,
                      stream())
        # ---- backward
        self._lin(self.plan_p2, gh2, C, gB2, C, self.W_p2T, g.nC)
        self._timed("symc2_bwd", (g.nC,), K.mm_symc2_bwd, g.nC, ws["M"], 16 * C, ws["spec"], self.Wsc2, gB2, C,
                    ws["gM"], 16 * C, ws["rho"], ws["g_rho"], stream())
        self._lin(self.plan_lin2T, ws["gM"], 16 * C, ws["gA"], self.nO2 * C, self.W_lin2T, g.nC, scale=ws["rho"],
                  scale_mode=1)
        if self.deterministic:
            srp, sperm = sender_csr(g)
            self._timed("conv2_bwd", (g.nE, g.nC, g.n_nodes), K.mm_conv2_bwd_det, g.rowptr, g.nC, ws["e_pk"],
                        ws["e_u"], ws["Xh"], D1, self.tab[1], self.n_tab, self.M, self.inv_h, ws["gA"], ws["part"],
                        ws["E"] * 17, ws["gXe"], stream())
            K.mm_gather_rows_csr(srp, sperm, ws["gXe"], D1, D1, ws["gXh"], D1, g.n_nodes, stream())
        else:
            K.mm_fill_f32(ws["gXh"], g.n_nodes * D1, 0.0, stream())
            self._timed("conv2_bwd", (g.nE, g.nC, g.n_nodes), K.mm_conv2_bwd, g.rowptr, g.nC, ws["e_pk"], ws["e_u"],
                        ws["Xh"], D1, self.tab[1], self.n_tab, self.M, self.inv_h, ws["gA"], ws["part"],
                        ws["E"] * 17, ws["gXh"], stream())
        pf = self._chunk_pair_forces(g, PF, forces)
        K.mm_edge_grad(g.nE, g.E_dev, ws["part"], ws["E"] * 17, NCB, ws["g_rho"], ws["e_recv"], ws["e_dd"], ws["e_u"],
                       pf, 0, stream())
        if forces is not None:
            self._add_chunk_forces(g, pf, forces)
        # gXh holds dL/dX in 16-channel-block-major rows (as mm_conv2_bwd / mm_conv2_bwd_det write it)
        self._lin(self.plan_p1, ws["gXh"], D1, G1, D1, self.W_up2T, g.n_nodes, out_rows=g.nodes, accumulate=1,
                  count_dev=g.N_dev, in_cb=4)
        self._lin(self.plan_sk1, gh2, C, G1, D1, self.W_sk1T, g.nC, out_rows=g.nodes, species=True, w_group_stride=1,
                  accumulate=1)

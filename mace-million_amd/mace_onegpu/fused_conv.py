"""FusedConvTP: gather(sender) -> channelwise tensor product -> scatter_sum(receiver), one HIP kernel each way.

Same module path, class, constructor and forward signature as the reference's mace_onegpu/fused_conv.py:20-37:

    FusedConvTP(segmented_polynomial, weight_numel, irreps_out=None)
    forward(node_feats [n, nX*128], edge_attrs [E, 16], tp_weights [E, nW*128], edge_index [2, E]) -> [n, nO*128]
    out[i, o, c] = sum_{e: edge_index[1, e] = i} sum_terms coef * W[e, w, c] * X[edge_index[0, e], k, c] * Y[e, m]

(row 0 of edge_index = sender, row 1 = receiver; rows of nodes that receive no edge are 0; layout ir_mul).
The reference hands the three inputs to a cuEquivariance SegmentedPolynomial built from
cue.descriptors.channelwise_tensor_product(...).flatten_coefficient_modes().squeeze_modes()
(fused_edge_conv.py:43-68); here the descriptor is ChannelwiseTP (the same term list, from
mace_onegpu.o3.tp_table) and the arithmetic runs in the generated kernels mm_tpw_<table>_{fwd,bwd}
(receiver-CSR over a stable receiver order, so edges may arrive in any order; tables without a kernel in the
library get theirs built on first use, tp_jit).  Backward (autograd) gives
d node_feats (atomic adds on senders), d edge_attrs and d tp_weights.  fp32 only, as the reference's fused
kernels.
"""
import re

import torch

from . import codegen, o3
from ._lib import K, stream

C = 128


class ChannelwiseTP:
    """Channelwise TP descriptor: node-feature irreps in_ls (C channels each) x spherical harmonics 0..sh_lmax ->
    mid irreps (l3 in target_ls), e3nn/MACE path order (o3.tp_paths).  The tables of o3.COMPILED_TP_TABLES run
    the library's kernels; any other table with harmonics up to l = 3 runs kernels generated and built for it on
    first use (tp_jit).  The kernels read 16 harmonic components per edge: edge attributes of a table with
    sh_lmax < 3 ((sh_lmax + 1)^2 components) are zero-padded to 16 on the way in."""

    def __init__(self, in_ls, sh_lmax=3, target_ls=(0, 1, 2, 3)):
        self.in_ls, self.sh_lmax, self.target_ls = tuple(in_ls), int(sh_lmax), tuple(target_ls)
        self.table = o3.tp_table(list(self.in_ls), self.sh_lmax, self.target_ls)
        self.name = None
        for name, key in o3.COMPILED_TP_TABLES.items():
            if (tuple(key[0]), key[1], tuple(key[2])) == (self.in_ls, self.sh_lmax, self.target_ls):
                self.name = name
        t = self.table
        self.nX, self.nW, self.nO, self.nY = t["nX"], t["nW"], t["nO"], t["nY"]
        self.weight_numel = self.nW * C
        # the backward kernel returns dL/dY as this many partial rows per edge (one per channel half of a wave)
        self.gy_parts = codegen.tpw_layout(t)["parts"]

    @classmethod
    def from_irreps(cls, edge_irreps, edge_attrs_irreps, target_irreps):
        """The descriptor of the reference's path_table(block) (fused_edge_conv.py:43-68) from the block's irreps
        strings, e3nn notation: node features "128x0e+128x1o" (every irrep 128 channels), edge attributes
        "1x0e+1x1o+1x2e+1x3o" (the harmonics l = 0 .. L, one copy each) and target irreps "128x0e+128x1o+...".
        Irreps of the other parity than (-1)^l are not supported (NotImplementedError)."""
        node, sh, target = (_parse_irreps(x) for x in (edge_irreps, edge_attrs_irreps, target_irreps))
        for name, irr, mul in (("edge_irreps", node, C), ("target_irreps", target, C), ("edge_attrs_irreps", sh, 1)):
            for (m, l, p) in irr:
                if m != mul:
                    raise ValueError(f"{name}: {m}x{l}{p}, but the kernels take {mul} per irrep")
                if p != ("e" if l % 2 == 0 else "o"):
                    raise NotImplementedError(f"{name}: {l}{p} (only the parity (-1)^l of the spherical harmonics)")
        ls = [l for (_, l, _) in sh]
        if ls != list(range(len(ls))):
            raise ValueError(f"edge_attrs_irreps must be the harmonics l = 0 .. L in order, not {edge_attrs_irreps!r}")
        return cls([l for (_, l, _) in node], len(ls) - 1, tuple(l for (_, l, _) in target))

    def kernels(self):
        """(forward, backward) entry points of this table (arguments of mm_tpw_l1_fwd / _bwd): the library's for a
        compiled table, else those built for the table (tp_jit; the first use builds them)."""
        if self.nY > 16:
            raise NotImplementedError("the kernels take spherical harmonics up to l = 3 (16 components), "
                                      f"not {self.nY} (sh_lmax = {self.sh_lmax})")
        if self.name is not None:
            return getattr(K, f"mm_tpw_{self.name}_fwd"), getattr(K, f"mm_tpw_{self.name}_bwd")
        from . import tp_jit
        return tp_jit.kernels(self.table)

    def __repr__(self):
        kern = self.name if self.name is not None else "built on first use"
        return (f"ChannelwiseTP(in_ls={self.in_ls}, sh_lmax={self.sh_lmax}, target_ls={self.target_ls}; nX={self.nX}, "
                f"nW={self.nW}, nO={self.nO}, terms={len(self.table['terms'])}, kernel={kern})")


def _parse_irreps(text):
    """[(multiplicity, l, parity)] of an e3nn irreps string such as "128x0e+128x1o" (a bare "1o" means 1x1o)."""
    out = []
    for part in str(text).replace(" ", "").split("+"):
        m = re.fullmatch(r"(?:(\d+)x)?(\d+)([eo])", part)
        if not m:
            raise ValueError(f"cannot read irreps {text!r} (at {part!r})")
        out.append((int(m.group(1) or 1), int(m.group(2)), m.group(3)))
    return out


def receiver_csr(edge_index, n_nodes, n_send_rows):
    """(rowptr int32 [n+1], eid int32 [E] or None when already receiver-sorted, send int32 [E]) with bounds checks
    of both index rows (one device->host read)."""
    if edge_index.dim() != 2 or edge_index.shape[0] != 2:
        raise ValueError(f"edge_index must be [2, E], got {tuple(edge_index.shape)}")
    E = edge_index.shape[1]
    if E >= 2 ** 31:
        raise ValueError("more than 2^31 - 1 edges")
    dev = edge_index.device
    send = edge_index[0].to(torch.int32).contiguous()
    recv = edge_index[1].long()
    if E == 0:
        return torch.zeros(n_nodes + 1, dtype=torch.int32, device=dev), None, send
    stats = torch.stack([send.min().long(), send.max().long(), recv.min(), recv.max(),
                         (recv[1:] >= recv[:-1]).all().long() if E > 1 else torch.ones((), dtype=torch.long,
                                                                                        device=dev)]).tolist()
    smin, smax, rmin, rmax, is_sorted = stats
    if smin < 0 or smax >= n_send_rows:
        raise IndexError(f"sender index out of range [0, {n_send_rows}): min {smin}, max {smax}")
    if rmin < 0 or rmax >= n_nodes:
        raise IndexError(f"receiver index out of range [0, {n_nodes}): min {rmin}, max {rmax}")
    counts = torch.bincount(recv, minlength=n_nodes)
    rowptr = torch.zeros(n_nodes + 1, dtype=torch.int64, device=dev)
    torch.cumsum(counts, 0, out=rowptr[1:])
    eid = None if is_sorted else torch.argsort(recv, stable=True).to(torch.int32)
    return rowptr.to(torch.int32), eid, send


def _check(t, name, cols):
    if not t.is_cuda:
        raise TypeError(f"{name} must be a GPU tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (the fused kernels are fp32), got {t.dtype}")
    if t.dim() != 2 or t.shape[1] != cols:
        raise ValueError(f"{name} must be [rows, {cols}], got {tuple(t.shape)}")
    return t.contiguous()


class _FusedConvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, X, Y, W, edge_index, desc):
        fwd, bwd = desc.kernels()
        X = _check(X, "node_feats", desc.nX * C)
        Y = _check(Y, "edge_attrs", desc.nY)
        W = _check(W, "tp_weights", desc.nW * C)
        E = edge_index.shape[1]
        if Y.shape[0] != E or W.shape[0] != E:
            raise ValueError(f"edge_attrs / tp_weights rows ({Y.shape[0]}, {W.shape[0]}) != number of edges {E}")
        if desc.nY < 16:                       # the kernels read 16 components; the table uses the first nY
            Y = torch.nn.functional.pad(Y, (0, 16 - desc.nY))
        n = X.shape[0]
        rowptr, eid, send = receiver_csr(edge_index, n, n)
        out = torch.empty(n, desc.nO * C, dtype=torch.float32, device=X.device)
        fwd(rowptr, n, eid, send, Y, Y.stride(0), W, W.stride(0), X, X.stride(0), out, out.stride(0), stream())
        ctx.save_for_backward(X, Y, W, rowptr, send, eid if eid is not None else torch.empty(0))
        ctx.has_eid = eid is not None
        ctx.desc, ctx.bwd = desc, bwd
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, gO):
        X, Y, W, rowptr, send, eid = ctx.saved_tensors
        eid = eid if ctx.has_eid else None
        desc = ctx.desc
        gO = gO.contiguous()
        n, E = X.shape[0], Y.shape[0]
        nx, ny, nw = ctx.needs_input_grad[:3]
        gX = torch.zeros_like(X) if nx else None
        gYp = torch.empty(desc.gy_parts, E, 16, dtype=torch.float32, device=X.device) if (ny and E) else None
        gW = torch.empty_like(W) if nw else None
        if E and (nx or ny or nw):
            ctx.bwd(rowptr, n, eid, send, Y, Y.stride(0), W, W.stride(0), X, X.stride(0), gO, gO.stride(0), gW,
                    W.stride(0), gYp, E * 16, gX, X.stride(0), stream())
        gY = None
        if ny:
            gY = gYp.sum(0)[:, :desc.nY] if E else torch.zeros(0, desc.nY, dtype=Y.dtype, device=Y.device)
        if nw and not E:
            gW = torch.zeros_like(W)
        return gX, gY, gW, None, None


class FusedConvTP(torch.nn.Module):
    """gather(sender) -> channelwise tensor product -> scatter_add(receiver), fused in one HIP kernel.

    forward(node_feats [n_nodes, in1], edge_attrs [E, in2], tp_weights [E, W], edge_index [2, E]) -> [n_nodes, out]
    m_ji is never materialised: output rows are accumulated on the receiver inside the kernel."""

    def __init__(self, segmented_polynomial, weight_numel, irreps_out=None):
        super().__init__()
        if not isinstance(segmented_polynomial, ChannelwiseTP):
            raise TypeError("segmented_polynomial must be a mace_onegpu.fused_conv.ChannelwiseTP descriptor")
        self.m = segmented_polynomial
        self.weight_numel = int(weight_numel)
        if self.weight_numel != self.m.weight_numel:
            raise ValueError(f"weight_numel {self.weight_numel} != {self.m.weight_numel} of the descriptor")
        self.irreps_out = irreps_out

    def forward(self, node_feats, edge_attrs, tp_weights, edge_index):
        return _FusedConvFn.apply(node_feats, edge_attrs, tp_weights, edge_index, self.m)

"""fp32 torch-CPU restatement of the production three-pass algorithm -- TEST INFRASTRUCTURE ONLY (see __init__.py).

bench.py's cpu_baseline leg times it; tests/test_cpu_baseline.py checks it against the fp64 oracle.  It evaluates
oracle.mace_ref's layer functions in fp32 with the 512-knot cubic-Hermite tables of the radial weights (the
reference's production lookup: spline_w._w_fwd, spline_w.py:18-50; tables from spline_radial._sample,
spline_radial.py:116-151, and conv_spline.build_tables, conv_spline.py:230-249), over receiver chunks, with the
passes of ReceiverChunkMACE.compute (receiver_chunk_mace.py:278-386):
    A  h1 of the chunk's receivers (no gradient)
    B  layer-2 energy with gradients: pair forces and G1 = d(scale E2)/dh1 of every node of the chunk
    C  layer 1 again with gradient of scale R1 + G1 . h1: pair forces
The per-edge work of a chunk is done in receiver blocks of `sub` receivers: the dense CPU tensor product
materialises [edges, 40, 128] per block, so the block bounds the memory; the three-pass algorithm is exact for any
block size (the blocks are chunks of the reference's algorithm).
"""
import time

import torch

from . import mace_ref

F32 = torch.float32


def _graphs(pos, box, spec, recv, send, blocks, N, tables, dtype):
    """Local graph, edge vectors (fp64 minimum image, then `dtype`) and table pair index of each receiver block."""
    loc = torch.full((N,), -1, dtype=torch.long)
    out = []
    for a0, b0 in blocks:
        nodes, ls, lr, rg, sg = mace_ref.local_graph(a0, b0, recv, send, loc)
        vec = mace_ref.min_image(pos[rg] - pos[sg], box).to(dtype)
        c2s = tables.col2s
        pair = c2s[spec[sg]] * tables.S + c2s[spec[rg]]
        out.append((a0, b0, nodes, ls, lr, rg, sg, vec, pair))
    return out


def _pass_a(m, t, spec, graphs, H1):
    with torch.no_grad():
        for (a0, b0, nodes, ls, lr, rg, sg, vec, pair) in graphs:
            H1[a0:b0] = mace_ref.layer1(m, spec[nodes], b0 - a0, ls, lr, vec, t, pair)


def _pass_b(m, t, spec, graphs, H1, G1, F, eat):
    for (a0, b0, nodes, ls, lr, rg, sg, vec, pair) in graphs:
        v = vec.clone().requires_grad_(True)
        h1l = H1[nodes].clone().requires_grad_(True)
        e = mace_ref.layer2_energy(m, spec[nodes], b0 - a0, ls, lr, v, h1l, t, pair)
        gv, gh = torch.autograd.grad(m.scale * e.sum(), [v, h1l])
        G1.index_add_(0, nodes, gh)
        F.index_add_(0, rg, -gv.double())
        F.index_add_(0, sg, gv.double())
        eat[a0:b0] += m.scale * e.detach().double()


def _pass_c(m, t, spec, graphs, G1, F, eat):
    for (a0, b0, nodes, ls, lr, rg, sg, vec, pair) in graphs:
        v = vec.clone().requires_grad_(True)
        h1 = mace_ref.layer1(m, spec[nodes], b0 - a0, ls, lr, v, t, pair)
        r1 = mace_ref.readout1(m, h1)
        (gv,) = torch.autograd.grad(m.scale * r1.sum() + (G1[a0:b0] * h1).sum(), [v])
        F.index_add_(0, rg, -gv.double())
        F.index_add_(0, sg, gv.double())
        eat[a0:b0] += m.scale * r1.detach().double()


def _inputs(pos, box, spec, recv, send):
    return (torch.as_tensor(pos, dtype=torch.float64), torch.as_tensor(box, dtype=torch.float64),
            torch.as_tensor(spec, dtype=torch.long), torch.as_tensor(recv, dtype=torch.long),
            torch.as_tensor(send, dtype=torch.long))


def three_pass(m32, t32, pos, box, spec, recv, send, chunk):
    """Whole-system evaluation in fp32 (energies and forces accumulated in fp64): (E, eat [N], F [N, 3])."""
    pos, box, spec, recv, send = _inputs(pos, box, spec, recv, send)
    N = pos.shape[0]
    blocks = [(a, min(a + chunk, N)) for a in range(0, N, chunk)]
    graphs = _graphs(pos, box, spec, recv, send, blocks, N, t32, F32)
    H1 = torch.zeros(N, 4, m32.C, dtype=F32)
    G1 = torch.zeros_like(H1)
    F = torch.zeros(N, 3, dtype=torch.float64)
    eat = (m32.e0[spec] + m32.shift).double()
    _pass_a(m32, t32, spec, graphs, H1)
    _pass_b(m32, t32, spec, graphs, H1, G1, F, eat)
    _pass_c(m32, t32, spec, graphs, G1, F, eat)
    return float(eat.sum()), eat, F


def chunk_timing(m32, t32, pos, box, spec, rowptr, send, a, b, sub=512, seed=0):
    """Wall times of one receiver chunk [a, b) of a larger system: topology (local graphs, edge vectors), pass A,
    pass B and pass C, in seconds, and the chunk's edge count.  rowptr / send: the receiver CSR of the whole
    system.  H1 rows of the chunk's outside senders (pass A of other chunks) are N(0, 1) stand-ins and pass C reads
    this chunk's share of G1: the values do not change the work."""
    e0, e1 = int(rowptr[a]), int(rowptr[b])
    counts = torch.as_tensor(rowptr[a + 1:b + 1], dtype=torch.long) - torch.as_tensor(rowptr[a:b], dtype=torch.long)
    recv = torch.repeat_interleave(torch.arange(a, b), counts)
    pos, box, spec, recv, send_c = _inputs(pos, box, spec, recv, send[e0:e1])
    N = pos.shape[0]
    t0 = time.perf_counter()
    graphs = _graphs(pos, box, spec, recv, send_c, [(x, min(x + sub, b)) for x in range(a, b, sub)], N, t32, F32)
    t_topo = time.perf_counter() - t0
    H1 = torch.zeros(N, 4, m32.C, dtype=F32)
    halo = torch.unique(send_c)
    halo = halo[(halo < a) | (halo >= b)]
    H1[halo] = torch.randn(halo.numel(), 4, m32.C, generator=torch.Generator().manual_seed(seed), dtype=F32)
    G1 = torch.zeros_like(H1)
    F = torch.zeros(N, 3, dtype=torch.float64)
    eat = torch.zeros(N, dtype=torch.float64)
    t0 = time.perf_counter()
    _pass_a(m32, t32, spec, graphs, H1)
    t1 = time.perf_counter()
    _pass_b(m32, t32, spec, graphs, H1, G1, F, eat)
    t2 = time.perf_counter()
    _pass_c(m32, t32, spec, graphs, G1, F, eat)
    t3 = time.perf_counter()
    return dict(topology=t_topo, A=t1 - t0, B=t2 - t1, C=t3 - t2, edges=e1 - e0, receivers=b - a)

#!/usr/bin/env python
"""Benchmark of the MI355X three-pass MACE path on one GPU (benchmark configurations 2-5).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 5|4|3|2|1] [--no-cpu] [--graphs]

Prints ONE JSON line.  Default: configuration 5, the metric's "1M-atom water" -- 343,000 rigid H2O molecules
(1,029,000 atoms) at 1.0 g/cm^3, random-init MPA-0-medium architecture, fp32 kernels, velocity-Verlet MD (dt 0.5 fs,
300 K Maxwell-Boltzmann start, neighbour skin 2 A, rebuild when an atom moved > 1 A).  One step = one MD step
(per-step pair filter, energy + forces by the three passes with every full receiver chunk replayed from its HIP
graphs, integration, rebuilds when due; --no-graphs runs every chunk eagerly).  W untimed steps after the initial
force call, then K timed steps between synchronisations.
  --config 3 : 98,304-atom water, one energy + force evaluation per step (ReceiverChunkMACE, chunk 16384, full chunks
               replayed from HIP graphs), topology of the chunks rebuilt every call
  --config 4 : 500,000-atom FCC Fe/Ni/Cr/Co alloy (a = 3.6 A, sigma 0.05 A), one energy + force evaluation per step
  --config 2 : edge-convolution microbenchmark on one 16,384-receiver chunk of the config-3 box with synthetic edge
               vectors (unit directions x U[0.8, 6.0] A), features and cotangents; value = achieved algorithmic GB/s of
               the layer-2 forward kernel, every kernel listed
  --config 1 : the 192-atom water box through ThreePassMLIAP.compute_forces (periodic-image ghosts), one E+F per
               step, with the fp64 CPU restatement's E+F (median of 3) and the GPU-vs-CPU energy and force deviations
Objects beside the contract fields:
  roofline     : the dominant kernel, algorithmic bytes (or FLOPs) per launch / mean launch time measured with HIP
                 events on the launch stream (during the timed steps; with graphs, in one eager step after them).  bound: "valu" for the edge convolutions (fp32
                 v_fma_f32 on the vector ALUs, roof 157.3 TFLOP/s: gfx950 dual-issues VALU instructions of two waves),
                 "mfma" for the matrix-core kernels, "hbm" below the ridge; traffic = measured HBM bytes per launch
                 from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes of this workload (or null)
  node_kernels : the linears (bf16 MFMA: mfma_frac = 6 F / t / 2.5 PFLOP/s; fp32_equiv_frac = F / t / 157.3) and the
                 symmetric contractions (HBM roof; FLOPs = the operations the generated kernels execute) timed with
                 HIP events in one extra step after the timed ones
  step_roofline: atom-steps/s against the fp32 ceiling of the exact model's work per atom-step (edge terms, node
                 linears, and the symmetric contractions at the operations the kernels execute)
  cpu_baseline : configs 3-5: the fp32 torch-CPU restatement of the production three-pass algorithm
                 (oracle/cpu_fp32.py: spline tables, passes A / B / C) timed on one 16,384-receiver chunk of that
                 configuration's own system and extrapolated to all its chunks, in the metric's unit; config 2: the
                 restatement's layer-2 convolution forward and backward on 2,048 receivers of the chunk with the GPU
                 run's inputs, scaled to the chunk (and the GPU kernels' outputs checked against it); config 1: the
                 fp64 restatement on the whole box, median of 3
  configs      : (default run) configurations 3, 4, 2 and 1 measured in the same process after configuration 5, each
                 with its value, dominant-kernel roofline, per-kernel table and CPU baseline
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mace-million_amd"))

HBM_PEAK_GBS = 8000.0
# fp32 vector ALU roof.  The build disables packed-FP32 instructions, but gfx950 issues two VALU instructions from
# two waves of a SIMD in one quad-cycle (SQ_ACTIVE_INST_VALU2) when neither reads an SGPR or uses DPP: plain
# v_fma_f32 with VGPR operands measured 151.6 TFLOP/s (2.07 cycles per wave64 instruction, 32 waves per SIMD), so the
# chip figure of 157.3 TFLOP/s is the reachable roof; instructions that cannot pair run at half that rate
VALU_F32_PEAK_TFLOPS = 157.3
FP32_CHIP_PEAK_TFLOPS = 157.3    # MI355X fp32 figure (vector or MFMA)
MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA (the linears: fp32 products as six bf16 products)
C = 128


def conv_algorithmic(name, E, nC, N, tab, Kp=128):
    """Algorithmic HBM bytes and FLOPs of one convolution launch (per-edge, per-receiver and per-node terms;
    tables read once).  P = distinct tables (1: this model's radial weights do not depend on the species).
    ace1_*: layer 1 in the density-projection form -- per edge the 16 B record and the 16 B edge vector (the
    harmonics are evaluated in the kernel; bwd also writes 17 floats), the 64-feature table once, B / gB
    [nC, 16, Kp] once; FLOPs = the 64 x 16 outer product (fwd) or its two transposed products (bwd) plus the
    spline evaluation.
    tpw_*: explicit per-edge weights (FusedConvTP) -- W [E, nW, 128] and Y read once (backward: gW and dL/dY
    written once)."""
    P, M = 1, 512
    if name.startswith("ace1"):
        tab_bytes = 16 * (M - 1) * 64
        if name == "ace1_fwd":
            return 32 * E + 4 * (nC + 1) + tab_bytes + 4 * nC * 16 * Kp + 4 * nC, 2 * E * 64 * 16 + 6 * E * 64
        return 100 * E + 4 * (nC + 1) + tab_bytes + 4 * nC * 16 * Kp, 4 * E * 64 * 16 + 10 * E * 64
    nX, nW, nO, nT = tab["nX"], tab["nW"], tab["nO"], len(tab["terms"])
    if name.startswith("tpw"):
        if name.endswith("fwd"):
            return (E * (8 + 64 + 4 * nW * C) + 4 * (nC + 1) + 4 * N * nX * C + 4 * nC * nO * C,
                    2 * E * C * nT)
        return (E * (8 + 64 + 8 * nW * C + 64) + 4 * (nC + 1) + 8 * N * nX * C + 4 * nC * nO * C,
                2 * E * C * 3 * nT)
    gx = 1 if name in ("conv2_bwd", "conv0123_bwd") else 0
    if name.endswith("fwd"):
        B = 16 * E + 4 * (nC + 1) + N * (4 * nX * C + 4) + 8 * P * M * nW * C + 4 * nC * nO * C
        F = 2 * E * C * (nT + 4 * nW)
    else:
        B = 28 * E + 4 * (nC + 1) + N * (4 * nX * C * (1 + gx) + 4) + 8 * P * M * nW * C + 4 * nC * nO * C
        F = 2 * E * C * ((2 + gx) * nT + 8 * nW)
    return B, F


# the HIP sources that define each profiled kernel (a measurement stays valid while these are unchanged)
KERNEL_SOURCES = {
    "mm_conv2_bwd_kernel": ("gen/conv_l2.hip", "gen/sh.h", "common.h"),
    "mm_conv2_fwd_kernel": ("gen/conv_l2.hip", "gen/sh.h", "common.h"),
    "mm_ace1_fwd_kernel": ("ace.hip", "gen/sh.h", "common.h"),
    "mm_ace1_bwd_kernel": ("ace.hip", "gen/sh.h", "common.h"),
    "mm_conv1_fwd_kernel": ("gen/conv_l1.hip", "gen/sh.h", "common.h"),
    "mm_conv1_bwd_kernel": ("gen/conv_l1.hip", "gen/sh.h", "common.h"),
    "mm_conv0123_fwd_kernel": ("gen/conv_l0123.hip", "gen/sh.h", "common.h"),
    "mm_conv0123_bwd_kernel": ("gen/conv_l0123.hip", "gen/sh.h", "common.h"),
    **{f"mm_tpw_{t}_{d}_kernel": (f"gen/tpw_{t}.hip", "common.h") for t in ("l1", "l2", "l0123") for d in ("fwd", "bwd")},
    "mm_linear_kernel": ("linear.hip", "common.h"),
    "mm_fill_f32_kernel": ("node.hip", "common.h"),
    "mm_fill_i32_kernel_nl": ("nlist.hip", "common.h"),
}


def kernel_digest(kernel, read=None):
    """sha256 over the HIP sources that define `kernel` (paths relative to mace-million_amd/csrc), to tie a
    measurement to the code it measured.  `read(relpath) -> bytes` defaults to the working tree."""
    import hashlib
    base = os.path.join(ROOT, "mace-million_amd", "csrc")
    if read is None:
        def read(rel):
            with open(os.path.join(base, rel), "rb") as fh:
                return fh.read()
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES[kernel]:
        h.update(rel.encode() + read(rel))
    return h.hexdigest()


TRAFFIC_FILES = ("traffic_config5_water1M.json", "traffic_config3_water98k.json", "traffic_config4_fcc500k.json",
                 "traffic_config2_chunk16k.json")


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes of this
    workload (profiles/traffic_*.json: counters scaled by a copy kernel of known size), or None when no pass was
    recorded for this workload and the kernel's current sources."""
    if kernel not in KERNEL_SOURCES:
        return None
    for name in TRAFFIC_FILES:
        path = os.path.join(ROOT, "profiles", name)
        if not os.path.exists(path):
            continue
        with open(path) as fh:
            t = json.load(fh)
        if t["workload"] != workload:
            continue
        rec = t["kernels"].get(kernel)
        if rec is None or rec.get("sources_sha256") != kernel_digest(kernel):
            return None
        return rec["traffic_bytes_per_launch"]
    return None


def node_algorithmic(name, units, symc_flops):
    """Algorithmic HBM bytes and FLOPs of one node-level launch.
    linear (mm_linear, MFMA): units (rows, sum of K-chunks, distinct input blocks, output components, accumulate,
      distinct 128 x 128 weight blocks): 2 * 128 * 128 flops per row and K-chunk; each input block and output
      component read / written once per row (accumulating outputs read too), each weight block once.
    symc<L>_<dir>: units (rows,): symc_flops[(L, dir)] flops per row (the operations the generated kernel executes);
      bytes: the 16-component input, the output (layer 1: 4 components, layer 2: 1), the backward's cotangent in
      and gradient out, the species index and density terms."""
    if name == "linear":
        rows, k_sum, n_in, n_comp, acc, n_w = units
        return 4 * C * rows * (n_in + n_comp * (1 + acc)) + 4 * C * C * n_w, 2 * C * C * rows * k_sum
    layer, direction = int(name[4]), name[6:]
    (rows,) = units
    n_out = 4 if layer == 1 else 1
    F = rows * symc_flops[(layer, direction)]
    if direction == "fwd":
        return 4 * C * rows * (16 + n_out) + 4 * rows, F
    return 4 * C * rows * (16 + n_out + 16) + 12 * rows, F


def symc_flops_per_row(tables=None):
    """{(layer, 'fwd' | 'bwd'): floating-point operations per node} that the generated symmetric-contraction kernels
    execute, counted from their gfx950 assembly by the build (lib/kernel_ops.json)."""
    from mace_onegpu import codegen
    gen = os.path.join(ROOT, "mace-million_amd", "csrc", "gen")
    ops = os.path.join(ROOT, "mace-million_amd", "lib", "kernel_ops.json")
    out = {}
    for layer in (1, 2):
        for d, f in codegen.symc_executed_flops(gen, layer, ops_json=ops).items():
            out[(layer, d)] = f
    return out


def symc_dense_flops(tables):
    """S1, S2 by the reference's dense-coefficient convention (scripts/flop_budget.py:53-56): 2 (nu + 1) flops per
    non-zero of each path's coupling tensor and channel."""
    from mace_onegpu import codegen
    return codegen.symc_model_flops(tables.sc1, [0, 1]), codegen.symc_model_flops(tables.sc2, [0])


def node_kernel_table(fl, ktimes, steps):
    """Per-kernel statistics of the linears and symmetric contractions (HIP-event times of one timed step)."""
    sf = symc_flops_per_row(fl.tables)
    out = {}
    for name, d in ktimes.items():
        if not (name == "linear" or name.startswith("symc")):
            continue
        B = sum(node_algorithmic(name, u, sf)[0] for u in d["units"])
        F = sum(node_algorithmic(name, u, sf)[1] for u in d["units"])
        out[name] = summarize(name, d["launches"], d["ms_total"], B, F, steps)
    return out


def summarize(name, launches, ms_total, B, F, steps):
    sec = ms_total * 1e-3
    k = dict(launches=launches, ms_per_launch=ms_total / launches, ms_per_step=ms_total / steps,
             GBps=B / sec / 1e9, TFLOPs=F / sec / 1e12, hbm_frac=B / sec / 1e9 / HBM_PEAK_GBS,
             bytes_per_launch=B / launches, flops_per_launch=F / launches)
    eng = engine(name)
    k["engine"] = eng
    if name.startswith("ace1"):          # fp32 MFMA
        k["mfma_frac"] = F / sec / 1e12 / MFMA_F32_PEAK_TFLOPS
    elif name == "linear":               # six bf16 MFMA products per fp32 product
        k["mfma_frac"] = 6 * F / sec / 1e12 / MFMA_BF16_PEAK_TFLOPS
        k["fp32_equiv_frac"] = F / sec / 1e12 / MFMA_F32_PEAK_TFLOPS
    else:                                # vector ALUs (executed operations)
        k["valu_frac"] = F / sec / 1e12 / VALU_F32_PEAK_TFLOPS
    return k


def engine(name):
    """The unit a kernel's arithmetic runs on: the edge convolutions and the symmetric contractions are fp32 VALU
    code (v_fma_f32), the layer-1 ACE kernels fp32 MFMA, the linears bf16 MFMA."""
    if name.startswith("ace1"):
        return "mfma_f32"
    if name == "linear":
        return "mfma_bf16"
    return "valu"


def kernel_table(fl, ktimes, steps):
    """Per-kernel launch statistics with algorithmic bytes / FLOPs (HIP-event times)."""
    out = {}
    for name, d in ktimes.items():
        tab = fl.tables.tp1 if name.startswith("conv1") else fl.tables.tp2
        Kp = getattr(fl, "ace_Kp", 128)
        B = sum(conv_algorithmic(name, *u, tab, Kp)[0] for u in d["units"])
        F = sum(conv_algorithmic(name, *u, tab, Kp)[1] for u in d["units"])
        out[name] = summarize(name, d["launches"], d["ms_total"], B, F, steps)
    return out


def roofline_of(kernels, workload=None):
    """Roofline of the dominant kernel (most time per step): the compute roof of the unit it runs on (fp32 VALU
    157.3 TFLOP/s with gfx950's dual issue, fp32 MFMA 157.3 TFLOP/s) when its intensity is above that unit's ridge
    with 8 TB/s, the HBM roof below it.  Both the HBM and the compute figures are reported."""
    if not kernels:
        return None
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    k = kernels[dom]
    intensity = k["flops_per_launch"] / k["bytes_per_launch"]
    eng = k.get("engine", engine(dom))
    peak = {"valu": VALU_F32_PEAK_TFLOPS, "mfma_f32": MFMA_F32_PEAK_TFLOPS,
            "mfma_bf16": MFMA_F32_PEAK_TFLOPS}[eng]
    compute = intensity > peak * 1e12 / (HBM_PEAK_GBS * 1e9)
    out = {"kernel": f"mm_{dom}_kernel"}
    if compute:
        out.update({"bound": "valu" if eng == "valu" else "mfma", "achieved": round(k["TFLOPs"], 3), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(k["TFLOPs"] / peak, 4),
                    "frac_of_fp32_chip_peak": round(k["TFLOPs"] / FP32_CHIP_PEAK_TFLOPS, 4)})
    else:
        out.update({"bound": "hbm", "achieved": round(k["GBps"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(k["hbm_frac"], 5)})
    out.update({"traffic": measured_traffic(f"mm_{dom}_kernel", workload) if workload else None,
                "intensity_flop_per_byte": round(intensity, 1),
                "hbm_achieved_GBps": round(k["GBps"], 2), "hbm_frac": round(k["hbm_frac"], 5),
                "flop_rate_TFLOPs": round(k["TFLOPs"], 3),
                **{f: round(k[f], 4) for f in ("valu_frac", "mfma_frac") if f in k},
                "bytes_per_launch": int(k["bytes_per_launch"]), "flops_per_launch": int(k["flops_per_launch"]),
                "ms_per_launch": round(k["ms_per_launch"], 4), "launches": k["launches"]})
    if compute and eng == "valu":
        out["note"] = ("the kernel runs on the vector ALUs (v_fma_f32, no packed FP32): 157.3 TFLOP/s needs two VALU "
                       "instructions from two waves per SIMD issued per quad-cycle (gfx950 dual issue; 151.6 TFLOP/s "
                       "measured for VGPR-operand FMAs); DPP, v_cndmask and SGPR-operand instructions cannot pair")
    return out


def step_roofline(value, pairs_per_atom, tables):
    """Work of the exact model per atom-step (the reference's three-pass algorithm: layer-1 conv forward in pass A
    and forward + backward in pass C, layer-2 conv forward + backward in pass B, at 2 flops per FMA; node-level
    linears 4 L1node + 3 L2node; the symmetric contractions at the operations the generated kernels execute,
    forward + backward of layer 1 twice and of layer 2 once) and the fp32 ceiling it implies."""
    t1, t2 = tables.tp1, tables.tp2
    n1, w1, n2, w2 = len(t1["terms"]), t1["nW"], len(t2["terms"]), t2["nW"]
    edge = pairs_per_atom * 2 * C * ((n1 + 4 * w1) * 2 + (2 * n1 + 8 * w1) + (n2 + 4 * w2) + (3 * n2 + 8 * w2))
    l1node = 2 * C * C * (16 + 16 + 4)
    l2node = 2 * C * C * (40 + 4 * 1.83 + 1 + 1)
    sf = symc_flops_per_row()
    symc = 2 * sf[(1, "fwd")] + sf[(1, "bwd")] + sf[(2, "fwd")] + sf[(2, "bwd")]
    f_atom = edge + 4 * l1node + 3 * l2node + symc
    ceiling = FP32_CHIP_PEAK_TFLOPS * 1e12 / f_atom
    S1d, S2d = symc_dense_flops(tables)
    return {"flop_per_atom_step": round(f_atom), "ceiling_atom_steps_per_s": round(ceiling),
            "peak_TFLOPs": FP32_CHIP_PEAK_TFLOPS, "frac": round(value / ceiling, 4),
            "symc_flop_per_node_step": symc, "S1_dense_flop_per_node": S1d, "S2_dense_flop_per_node": S2d,
            "note": "edge and linear terms count the reference algorithm's work (this build executes less: layer 1 "
                    "in the density-projection form, pass C reuses pass A's layer-1 state); the symmetric "
                    "contractions count the operations the generated kernels execute, not the dense-coefficient "
                    "convention (S1/S2_dense, shown for comparison)"}


def ncores():
    """Host threads this run may use: the affinity mask, capped by OMP_NUM_THREADS when it is set (the box's
    CPU share for one GPU)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else n


def cpu_baseline_chunk(pos, box, spec, NN, send, chunk=16384, label=""):
    """fp32 torch-CPU restatement of the production three-pass algorithm (oracle/cpu_fp32.py: the oracle's layer
    functions in fp32 with the 512-knot Hermite tables) timed on the first `chunk` receivers of this system -- one
    receiver chunk of each pass -- and extrapolated to every chunk of the system, in atom-steps/s.  Inputs are
    the system's own positions, species and pair list (host copies)."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from mace_onegpu import model as mm, o3
    from oracle import cpu_fp32, mace_ref

    torch.set_num_threads(ncores())
    m = mace_ref.RefModel(mm.MaceModel(seed=0), o3.coupling)
    N = len(pos)
    t32 = mace_ref.Tables64(m, sorted(set(np.asarray(spec).tolist())), n_grid=512).astype(torch.float32)
    rowptr = np.concatenate([[0], np.cumsum(NN)])
    b = min(chunk, N)
    r = cpu_fp32.chunk_timing(m.astype(torch.float32), t32, pos, box, spec, rowptr, send, 0, b, sub=512)
    t_chunk = r["topology"] + r["A"] + r["B"] + r["C"]
    n_chunks = N / b
    value = N / (t_chunk * n_chunks)
    return dict(value=round(value, 2), unit="atom-steps/s", cores=ncores(), kind="port",
                sample=f"fp32 torch-CPU restatement of the three-pass algorithm with 512-knot spline tables "
                       f"(oracle/cpu_fp32.py) on receivers [0, {b}) of {label} ({r['edges']} edges): topology "
                       f"{r['topology']:.1f} s, pass A {r['A']:.1f} s, B {r['B']:.1f} s, C {r['C']:.1f} s = "
                       f"{t_chunk:.1f} s per chunk on {ncores()} threads, extrapolated to {n_chunks:.2f} chunks "
                       f"of {b} receivers ({N} atoms)",
                extrapolated=True, seconds_per_chunk=round(t_chunk, 2))


def cpu_baseline_conv(rij, recv_local, ls, rowptr, E_full, nC_full, nN_full, X_gpu, gA_gpu, n_recv=2048):
    """fp32 torch-CPU layer-2 edge convolution of the restatement (512-knot table lookup of W, channelwise TP over
    the sparse path table, receiver sum), forward and backward (autograd: dL/dvec and dL/dX for L = gA . out, as
    the reference's conv_spline._bench times both, conv_spline.py:304-455), on the first n_recv receivers of the
    config-2 chunk with the GPU run's own sender features X and cotangent gA.  The times are scaled to the chunk's
    edges; the value is the forward's algorithmic GB/s of mm_conv2_fwd over the whole chunk (the metric's unit).
    Returns (baseline dict, (out [n_recv, 40, C], dL/dvec [ne, 3], dL/dX [n, 4, C])) for the in-bench check."""
    import torch

    sys.path.insert(0, ROOT)
    from mace_onegpu import model as mm, o3
    from mace_onegpu.fused_conv import ChannelwiseTP
    from oracle import mace_ref

    torch.set_num_threads(ncores())
    m = mace_ref.RefModel(mm.MaceModel(seed=0), o3.coupling)
    t32 = mace_ref.Tables64(m, [0, 7], n_grid=512).astype(torch.float32)
    d = ChannelwiseTP([0, 1])
    ne = int(rowptr[n_recv])
    vec = torch.as_tensor(rij[:ne]).float().requires_grad_(True)
    lr = torch.as_tensor(recv_local[:ne]).long()
    send = torch.as_tensor(ls[:ne]).long()
    n = int(send.max()) + 1
    X = torch.as_tensor(X_gpu[:n]).float().reshape(n, d.nX, C).clone().requires_grad_(True)
    G = torch.as_tensor(gA_gpu[:n_recv]).float().reshape(n_recv, d.nO, C)
    pair = torch.zeros(ne, dtype=torch.long)
    t0 = time.perf_counter()
    r = torch.linalg.vector_norm(vec, dim=1)
    W = t32.lookup(1, r, pair).reshape(ne, d.nW, C)
    Y = mace_ref.sh(vec)
    mid = mace_ref.channelwise_tp(W, X, Y, send, d.table["paths"], d.table["in_ls"], o3.coupling)
    out = mace_ref.scatter_sum(mid, lr, n_recv)
    t_fwd = time.perf_counter() - t0
    t0 = time.perf_counter()
    gv, gx = torch.autograd.grad((out * G).sum(), [vec, X])
    t_bwd = time.perf_counter() - t0
    B, _ = conv_algorithmic("conv2_fwd", E_full, nC_full, nN_full, d.table)
    scale = E_full / ne
    cpu = dict(value=round(B / (t_fwd * scale) / 1e9, 3), unit="GB/s", cores=ncores(), kind="port",
               fwd_s_scaled=round(t_fwd * scale, 2), bwd_s_scaled=round(t_bwd * scale, 2),
               sample=f"fp32 torch-CPU layer-2 convolution of the restatement (table lookup of W, channelwise TP, "
                      f"receiver sum; oracle/mace_ref.py) on the chunk's first {n_recv} receivers ({ne} edges) with "
                      f"the GPU run's features and cotangent: forward {t_fwd:.2f} s, backward (dL/dvec, dL/dX by "
                      f"autograd) {t_bwd:.2f} s on {ncores()} threads, scaled to the chunk's {E_full} edges "
                      f"({t_fwd * scale:.1f} s + {t_bwd * scale:.1f} s); bytes counted as for mm_conv2_fwd",
               extrapolated=True)
    return cpu, (out.detach(), gv, gx, n_recv, ne, n)


def cpu_baseline_config1(pos, box, spec, recv, send, reps=3):
    """Configuration 1 on the CPU as the reference evaluates it: fp64, exact radial MLP (no tables), the three-pass
    algorithm of ReceiverChunkMACE.compute (oracle/mace_ref.py three_pass, one chunk of all 192 atoms), median wall
    time of `reps` evaluations.  Returns (baseline dict, (E, F [N, 3])) for the GPU parity figures."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from mace_onegpu import model as mm, o3
    from oracle import mace_ref

    torch.set_num_threads(ncores())
    m = mace_ref.RefModel(mm.MaceModel(seed=0), o3.coupling)
    N = len(pos)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        E0, _, F0, _, _ = mace_ref.three_pass(m, pos, box, spec, recv, send, chunk=N)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    return (dict(value=round(N / t, 2), unit="atom-steps/s", cores=ncores(), kind="port",
                 sample=f"fp64 torch-CPU three-pass restatement (oracle/mace_ref.py, exact radial MLP) of the whole "
                        f"{N}-atom box, median of {reps} E+F evaluations: {t:.2f} s on {ncores()} threads",
                 extrapolated=False, seconds_per_step=round(t, 3)), (E0, F0))


def run_config1(a):
    """Configuration 1: the 64-molecule water box (192 atoms, L = 12.416 A) through the ML-IAP boundary on the GPU
    (ThreePassMLIAP.compute_forces with periodic-image ghosts, fp32 kernels), one E+F per step, against the fp64 CPU
    restatement timed beside it (median of 3); the GPU energies and forces are compared with it."""
    import numpy as np
    import torch

    from mace_onegpu import model as mm, systems
    from mace_onegpu.lammps_data import PeriodicMLIAPData
    from mace_onegpu.mliap_threepass import ThreePassMLIAP
    from mace_onegpu.receiver_chunk_mace import System

    pos, box, Z = systems.water_box(64, seed=0)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    tp = ThreePassMLIAP(mm.MaceModel(seed=0))
    data = PeriodicMLIAPData(s, s.spidx.long(), ghosts=True)
    for _ in range(max(a.warmup, 1)):
        tp.compute_forces(data)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        tp.compute_forces(data)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    F = data.atom_forces().cpu()
    E = float(data.energy)
    cpu, parity = None, None
    if not a.no_cpu:
        recv = np.repeat(np.arange(s.N), s.NN.cpu().numpy())
        cpu, (E0, F0) = cpu_baseline_config1(s.pos.cpu().numpy(), box, s.spidx.cpu().numpy(), recv,
                                             s.send.cpu().numpy())
        parity = {"E_gpu_eV": round(E, 9), "E_cpu_fp64_eV": round(E0, 9), "dE_per_atom_eV": abs(E - E0) / s.N,
                  "max_abs_dF_eV_per_A": float((F - F0).abs().max()), "max_abs_F_eV_per_A": float(F0.abs().max()),
                  "tolerance": {"dE_per_atom_eV": 1e-5, "max_abs_dF_eV_per_A": 1e-3}}
        parity["pass"] = parity["dE_per_atom_eV"] < 1e-5 and parity["max_abs_dF_eV_per_A"] < 1e-3
    value = s.N * a.steps / dt
    line = base_line(a, "atom-steps/s (E+F, 192-atom water, fp32 GPU vs fp64 CPU, 1 GPU)", value,
                     dt / a.steps * 1e3, "atom-steps/s", "synthetic (seeded water generator, random-init weights)",
                     {"workload": "config1: 64-molecule water (192 atoms, L = 12.416 A), random-init MPA-0-medium "
                                  "architecture, one E+F per step through ThreePassMLIAP.compute_forces with "
                                  "periodic-image ghosts (fp32 kernels); the CPU leg is the fp64 restatement",
                      "atoms": s.N, "ghosts": data.nghost, "pairs": data.npairs, "E_per_atom_eV": round(E / s.N, 9),
                      "parity_vs_fp64_cpu": parity}, None, {}, cpu)
    return line


def exit_multi_gpu():
    print(json.dumps({"error": "this build runs on exactly one GPU: the multi-GPU path (spatial domain "
                               "decomposition with RCCL halo exchange) is designed, not built; use --gpus 1"}))
    sys.exit(2)


def copy_calibration(mib):
    import torch

    from mace_onegpu._lib import K, stream
    n = mib << 18
    src = torch.empty(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    K.mm_fill_f32(src, n, 1.0, stream())      # writes n * 4 bytes
    torch.mul(src, 2.0, out=dst)              # reads n * 4 bytes, writes n * 4 bytes
    torch.cuda.synchronize()


def rounded(kernels):
    return {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
            for k, v in kernels.items()}


def base_line(a, metric, value, ms, unit, data, config, roof, kernels, cpu, higher=True):
    return {"metric": metric, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": round(ms, 3), "higher_is_better": higher, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": data, "config": config, "roofline": roof,
            "kernels": rounded(kernels), "cpu_baseline": cpu}


# ----------------------------------------------------------------------------- config 5: MD
def run_md(a):
    import torch

    from mace_onegpu import model as mm, systems
    from mace_onegpu.md import MDRunner

    t0 = time.perf_counter()
    pos, box, Z = systems.water_box(a.n_mol, seed=0)
    t_gen = time.perf_counter() - t0
    model = mm.MaceModel(seed=0)
    md = MDRunner(model, pos, box, Z, chunk=a.chunk, skin=2.0, dt_fs=0.5, T=300.0, seed_v=4, device="cuda",
                  use_graphs=a.graphs)
    N = md.skin_sys.N
    print(f"# generated {N} atoms (L = {box[0]:.3f} A) in {t_gen:.1f} s; chunk {a.chunk}", file=sys.stderr, flush=True)
    md.forces()                      # initial forces (set-up: builds the tables and chunk workspaces)
    for i in range(a.warmup):
        md.step()
        print(f"# warmup step {i}: E/N {md.E / N:.6f} eV", file=sys.stderr, flush=True)
    rebuilds0 = md.n_rebuild
    e_tot0 = md.E + md.kinetic()          # total energy before and after the timed steps (outside the timing)
    fl = md.ev.fl
    fl.start_kernel_timing()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        md.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ktimes = fl.stop_kernel_timing()
    e_kin = md.kinetic()
    e_drift = md.E + e_kin - e_tot0
    n_pairs = int(md.pairs.E)
    if a.graphs:
        # HIP events cannot time launches inside graph replays: one more step with every chunk run eagerly, each
        # launch timed, gives the per-kernel table (the same kernels the graphs replay)
        md.ev.use_graphs = False
        fl.start_kernel_timing()
        md.step()
        ktimes = fl.stop_kernel_timing()
        ksteps = 1
    else:
        ksteps = a.steps
    # one more step, after the timed ones, with the linears' and contractions' launches timed as well
    fl.start_kernel_timing(node_kernels=True)
    md.step()
    nodes = node_kernel_table(fl, fl.stop_kernel_timing(), 1)
    md.ev.use_graphs = a.graphs
    if a.copy_calib_mib > 0:
        copy_calibration(a.copy_calib_mib)
    value = N * a.steps / dt
    kernels = kernel_table(fl, ktimes, ksteps)
    roof = roofline_of(kernels, {"n_mol": a.n_mol, "chunk": a.chunk})
    cpu = None
    if not a.no_cpu:
        print("# cpu baseline: one 16,384-receiver chunk of this system", file=sys.stderr, flush=True)
        cpu = cpu_baseline_chunk(md.pos.cpu().numpy(), box, (md.Z - 1).cpu().numpy(), md.pairs.NN.cpu().numpy(),
                                 md.pairs.send_view.cpu().numpy(), 16384, "the configuration-5 water box")
    line = base_line(a, "atom-steps/s (E+F, 1M-atom water, fp32, 1 GPU)", value, dt / a.steps * 1e3, "atom-steps/s",
                     "synthetic (seeded water generator, random-init weights)",
                     {"workload": "config5: 343,000-molecule water (1,029,000 atoms), random-init MPA-0-medium "
                                  "architecture, velocity-Verlet MD dt 0.5 fs, skin 2 A",
                      "atoms": N, "pairs": n_pairs, "chunk": a.chunk, "graphs": a.graphs,
                      "rebuilds_timed": md.n_rebuild - rebuilds0,
                      "energy_drift_eV": round(e_drift, 6), "kinetic_energy_eV": round(e_kin, 3),
                      "peak_hbm_GB": round(torch.cuda.max_memory_allocated() / 1e9, 2),
                      "box_A": round(float(box[0]), 4)}, roof, kernels, cpu)
    if a.graphs:
        line["roofline_note"] = ("kernels timed with HIP events in one eager MD step after the graph-replayed timed "
                                 "steps (events cannot time launches inside a replay)")
    line["node_kernels"] = rounded(nodes)
    line["step_roofline"] = step_roofline(value, n_pairs / N, fl.tables)
    return line


# ----------------------------------------------------------------------------- configs 3 and 4: E+F evaluations
def run_ef(a):
    import torch

    from mace_onegpu import model as mm, systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System

    if a.config == 3:
        pos, box, Z = systems.water_box(32768, seed=0)
        chunk = a.chunk or 16384
        graphs = True if a.graphs is None else a.graphs
        workload = ("config3: 32,768-molecule water (98,304 atoms), random-init MPA-0-medium architecture, one "
                    f"three-pass E+F evaluation per step, chunk {chunk}" + (", HIP-graph chunks" if graphs else ""))
        metric = "atom-steps/s (E+F, 98,304-atom water, fp32, 1 GPU)"
    else:
        pos, box, Z = systems.fcc_alloy(n_cells=50)
        chunk = a.chunk or 131072
        graphs = bool(a.graphs)
        workload = ("config4: 500,000-atom FCC Fe/Ni/Cr/Co (a = 3.6 A, 50^3 cells, sigma 0.05 A), random-init "
                    f"MPA-0-medium architecture, one three-pass E+F evaluation per step, chunk {chunk}"
                    + (", HIP-graph chunks" if graphs else ""))
        metric = "atom-steps/s (E+F, 500,000-atom FCC alloy, fp32, 1 GPU)"
    model = mm.MaceModel(seed=0)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    ev = ReceiverChunkMACE(model, chunk=chunk, device="cuda", use_graphs=graphs)
    ev.compute(s)
    for _ in range(a.warmup):
        ev.compute(s)
    fl = ev.fl
    fl.start_kernel_timing()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        E, eat, F, PF = ev.compute(s)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ktimes = fl.stop_kernel_timing()
    value = s.N * a.steps / dt
    if a.copy_calib_mib > 0:
        copy_calibration(a.copy_calib_mib)
    if graphs:
        # HIP events cannot time launches inside graph replays: one eager evaluation of the same system, with every
        # launch timed, gives the per-kernel table (the same kernels the graphs replay)
        eager = ReceiverChunkMACE(model, chunk=chunk, device="cuda", use_graphs=False)
        eager.compute(s)
        fl = eager.fl
        fl.start_kernel_timing()
        eager.compute(s)
        kernels = kernel_table(fl, fl.stop_kernel_timing(), 1)
        ev_nodes = eager
    else:
        kernels = kernel_table(fl, ktimes, a.steps)
        ev_nodes = ev
    fl.start_kernel_timing(node_kernels=True)   # one more evaluation with the node-level launches timed as well
    ev_nodes.compute(s)
    nodes = node_kernel_table(fl, fl.stop_kernel_timing(), 1)
    cpu = None
    if a.cpu_from is not None:
        cpu = dict(a.cpu_from)
    elif not a.no_cpu:
        print(f"# cpu baseline: one 16,384-receiver chunk of configuration {a.config}", file=sys.stderr, flush=True)
        # configuration 3 has exactly 6 such chunks, configuration 4 30.5: the extrapolation counts the chunks
        cpu = cpu_baseline_chunk(s.pos.cpu().numpy(), s.box, s.spidx.cpu().numpy(), s.NN.cpu().numpy(),
                                 s.send.cpu().numpy(), 16384, f"the configuration-{a.config} system")
    n_pairs = int(s.rowptr[-1])
    line = base_line(a, metric, value, dt / a.steps * 1e3, "atom-steps/s",
                     "synthetic (seeded generator, random-init weights)",
                     {"workload": workload, "atoms": s.N, "pairs": n_pairs, "chunk": chunk, "graphs": graphs,
                      "E_per_atom_eV": round(E / s.N, 8),
                      "peak_hbm_GB": round(torch.cuda.max_memory_allocated() / 1e9, 2)},
                     roofline_of(kernels, {"config": a.config, "chunk": chunk}), kernels, cpu)
    if graphs:
        line["roofline_note"] = ("kernels timed with HIP events in one eager evaluation of the same system after the "
                                 "graph-replayed steps (events cannot time launches inside a replay)")
    line["node_kernels"] = rounded(nodes)
    line["step_roofline"] = step_roofline(value, n_pairs / s.N, fl.tables)
    return line


# ----------------------------------------------------------------------------- config 2: edge-convolution kernels
def run_conv(a):
    import torch

    from mace_onegpu import codegen, model as mm, o3, systems
    from mace_onegpu._lib import K, stream
    from mace_onegpu.fused_conv import ChannelwiseTP, FusedConvTP
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System

    pos, box, Z = systems.water_box(32768, seed=0)
    s = System(pos, box, Z - 1, 6.0, "cuda")
    s.build_neighbors()
    ev = ReceiverChunkMACE(mm.MaceModel(seed=0), chunk=16384, device="cuda")
    g = ev.graphs(s)[0]
    fl = ev._layers(s)
    ws = fl.prepare(g)
    E, nC, nN = g.nE, g.nC, g.n_nodes
    gen = torch.Generator().manual_seed(1)
    u = torch.randn(E, 3, generator=gen, dtype=torch.float64)
    u /= u.norm(dim=1, keepdim=True)
    r = 0.8 + 5.2 * torch.rand(E, 1, generator=gen, dtype=torch.float64)
    g.rij = (u * r).float().double().cuda()
    g.pair_i = (g.recv_local + g.a).to(torch.int32)
    gen2 = torch.Generator(device="cuda").manual_seed(2)
    X2 = torch.randn(nN, 4 * C, device="cuda", generator=gen2)
    gA2 = torch.randn(nC, 40 * C, device="cuda", generator=gen2)
    Kp = getattr(fl, "ace_Kp", C)
    gM1 = torch.randn(nC, 16 * Kp, device="cuda", generator=gen2)
    gA1 = torch.randn(nC, 16 * C, device="cuda", generator=gen2)
    fl._geometry(0, g)
    pk1, eu1 = ws["e_pk"][:E].clone(), ws["e_u"][:E].clone()
    fl._geometry(1, g)
    pk2, eu2 = ws["e_pk"][:E].clone(), ws["e_u"][:E].clone()
    out1 = torch.empty(nC, 16 * C, device="cuda")
    out2 = torch.empty(nC, 40 * C, device="cuda")
    Bace = torch.empty(nC, 16 * Kp, device="cuda")
    rho = torch.empty(nC, device="cuda")
    part = torch.empty(8 * E * 17, device="cuda")
    gX = torch.zeros(nN, 4 * C, device="cuda")
    st = stream()
    calls = {
        "conv1_fwd": (lambda: K.mm_conv1_fwd(g.rowptr, nC, pk1, eu1, fl.Xs1, C, fl.tab[0], fl.n_tab, fl.M, out1, rho,
                                             st), fl.tables.tp1),
        "conv1_bwd": (lambda: K.mm_conv1_bwd(g.rowptr, nC, pk1, eu1, fl.Xs1, C, fl.tab[0], fl.n_tab, fl.M, fl.inv_h,
                                             gA1, part, E * 17, None, st), fl.tables.tp1),
        "conv2_fwd": (lambda: K.mm_conv2_fwd(g.rowptr, nC, pk2, eu2, X2, 4 * C, fl.tab[1], fl.n_tab, fl.M, out2, rho,
                                             st), fl.tables.tp2),
        "conv2_bwd": (lambda: K.mm_conv2_bwd(g.rowptr, nC, pk2, eu2, X2, 4 * C, fl.tab[1], fl.n_tab, fl.M, fl.inv_h,
                                             gA2, part, E * 17, gX, st), fl.tables.tp2),
    }
    if fl.ace:
        calls["ace1_fwd"] = (lambda: K.mm_ace1_fwd(g.rowptr, nC, pk1, eu1, fl.tab_h, fl.S, fl.S_pad, Bace, rho, st),
                             fl.tables.tp1)
        calls["ace1_bwd"] = (lambda: K.mm_ace1_bwd(g.rowptr, nC, pk1, eu1, fl.tab_h, fl.S, fl.S_pad, gM1, fl.inv_h,
                                                   part, st), fl.tables.tp1)
    # the fused spline-table convolution for the literal V3 node features 0e+1o+2e+3o (23 paths, 353 terms) on the
    # same edge records: a 23-path table sampled from a radial network of the model's layer sizes with random
    # weights (seed 6)
    d3 = ChannelwiseTP([0, 1, 2, 3])
    g6 = torch.Generator().manual_seed(6)
    dims = [fl.spec.num_bessel] + list(fl.spec.radial_mlp) + [d3.nW * C]
    Ws3 = [torch.randn(dims[j], dims[j + 1], generator=g6, dtype=torch.float64).cuda() for j in range(4)]
    M = fl.M
    r_k = torch.linspace(fl.r_lo, fl.r_hi, M, dtype=torch.float64, device="cuda")
    eps = 1e-5 * (fl.r_hi - fl.r_lo)
    pts = torch.cat([r_k, r_k + eps, r_k - eps]).contiguous()
    smp = torch.empty(3 * M, d3.nW * C, dtype=torch.float64, device="cuda")
    K.mm_radial_mlp_f64(3 * M, pts, *Ws3, fl.spec.num_bessel, dims[1], d3.nW * C, fl.spec.r_max, fl.spec.p_cutoff,
                        mm.SILU_NORM, smp, st)
    tab3 = torch.empty(8 * (M - 1) * d3.nW * 16 * 4, device="cuda")
    K.mm_spline_coeffs(smp, M, d3.nW, eps, fl.h, 0, 1, tab3, st)
    del smp
    X3 = torch.randn(nN, d3.nX * C, device="cuda", generator=gen2)
    gA3 = torch.randn(nC, d3.nO * C, device="cuda", generator=gen2)
    out3 = torch.empty(nC, d3.nO * C, device="cuda")
    n3 = codegen.tpw_layout(d3.table)["parts"]
    part3 = torch.empty(n3 * E * 17, device="cuda")
    gX3 = torch.zeros(nN, d3.nX * C, device="cuda")
    calls["conv0123_fwd"] = (lambda: K.mm_conv0123_fwd(g.rowptr, nC, pk2, eu2, X3, d3.nX * C, tab3, 1, M, out3, rho,
                                                       st), d3.table)
    calls["conv0123_bwd"] = (lambda: K.mm_conv0123_bwd(g.rowptr, nC, pk2, eu2, X3, d3.nX * C, tab3, 1, M, fl.inv_h,
                                                       gA3, part3, E * 17, gX3, st), d3.table)
    # explicit-weight FusedConvTP kernels (V1, V2 and the literal V3 table 0e+1o+2e+3o) on the same edges
    Y16 = torch.from_numpy(o3.spherical_harmonics(g.rij.cpu().numpy())).float().cuda()
    send = g.ls
    rp = torch.zeros(nN + 1, dtype=torch.int32, device="cuda")
    rp[: nC + 1] = g.rowptr
    rp[nC + 1:] = g.rowptr[-1]
    for key, ls in (("tpw_l1", [0]), ("tpw_l2", [0, 1]), ("tpw_l0123", [0, 1, 2, 3])):
        d = ChannelwiseTP(ls)
        Xd = torch.randn(nN, d.nX * C, device="cuda", generator=gen2)
        Wd = torch.randn(E, d.nW * C, device="cuda", generator=gen2)
        Od = torch.empty(nN, d.nO * C, device="cuda")
        Gd = torch.randn(nN, d.nO * C, device="cuda", generator=gen2)
        gWd = torch.empty_like(Wd)
        gYp = torch.empty(d.gy_parts, E, 16, device="cuda")
        gXd = torch.zeros_like(Xd)
        f = getattr(K, f"mm_{key}_fwd")
        b = getattr(K, f"mm_{key}_bwd")
        calls[key + "_fwd"] = ((lambda f=f, Xd=Xd, Wd=Wd, Od=Od:
                                f(rp, nC, None, send, Y16, 16, Wd, Wd.stride(0), Xd, Xd.stride(0), Od, Od.stride(0),
                                  st)), d.table)
        calls[key + "_bwd"] = ((lambda b=b, Xd=Xd, Wd=Wd, Gd=Gd, gWd=gWd, gYp=gYp, gXd=gXd:
                                b(rp, nC, None, send, Y16, 16, Wd, Wd.stride(0), Xd, Xd.stride(0), Gd, Gd.stride(0),
                                  gWd, gWd.stride(0), gYp, E * 16, gXd, gXd.stride(0), st)), d.table)
    kernels = {}
    for name, (fn, tab) in calls.items():
        for _ in range(max(a.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        B, F = conv_algorithmic(name, E, nC, nN, tab, Kp)
        kernels[name] = summarize(name, a.steps, ms, B * a.steps, F * a.steps, a.steps)
    # check the layer-2 forward against FusedConvTP fed with the spline weights of the same edges (first 256
    # receivers): W[e, w, c] evaluated in fp64 from the kernel's interval coefficients
    calls["conv2_fwd"][0]()
    torch.cuda.synchronize()
    nr = 256
    ne = int(g.rowptr[nr])
    coef = fl.tab[1].view(8, fl.n_tab, fl.M - 1, 10, 16, 4).double()
    pk = pk2[:ne]
    row = pk[:, 1].contiguous().view(torch.int32).long()
    t = pk[:, 0].double()[None, :, None, None]
    cw = coef[:, 0, row]                                            # [8, ne, 10, 16, 4]
    Wsp = ((cw[..., 3] * t + cw[..., 2]) * t + cw[..., 1]) * t + cw[..., 0]
    Wsp = Wsp.permute(1, 2, 0, 3).reshape(ne, 10 * C).float().contiguous()
    Yc = torch.from_numpy(o3.spherical_harmonics(eu2[:ne, :3].double().cpu().numpy())).float().cuda()
    tp = FusedConvTP(ChannelwiseTP([0, 1]), 10 * C)
    ei = torch.stack([pk[:, 2].contiguous().view(torch.int32).long(), g.recv_local[:ne].long()])
    ref = tp(X2, Yc, Wsp, ei)[:nr]
    err = float((ref - out2[:nr]).abs().max() / ref.abs().max())
    v = kernels["conv2_fwd"]
    cpu, oracle_check = None, None
    if not a.no_cpu:
        rp_h = g.rowptr.cpu().numpy()
        cpu, (o_out, o_gv, o_gx, nr_c, ne_c, nn_c) = cpu_baseline_conv(
            g.rij.cpu().numpy(), g.recv_local.cpu().numpy(), g.ls.cpu().numpy(), rp_h, E, nC, nN, X2.cpu(),
            gA2.cpu())
        # the same receivers through the GPU kernels: forward output, and the backward of L = gA . out restricted
        # to them (gA zero elsewhere) -> dL/dX (G1 path) and per-edge dL/dvec (mm_edge_grad, no density term)
        gAm = gA2.clone()
        gAm[nr_c:] = 0
        gXm = torch.zeros_like(X2)
        partm = torch.empty_like(part)
        PFm = torch.empty(E, 3, device="cuda")
        K.mm_conv2_bwd(g.rowptr, nC, pk2, eu2, X2, 4 * C, fl.tab[1], fl.n_tab, fl.M, fl.inv_h, gAm, partm, E * 17,
                       gXm, st)
        K.mm_edge_grad(E, None, partm, E * 17, 8, torch.zeros(nC, device="cuda"), ws["e_recv"], ws["e_dd"], eu2,
                       PFm, 0, st)
        calls["conv2_fwd"][0]()
        torch.cuda.synchronize()

        def rel(gpu, ref):
            return float((gpu.double().cpu() - ref.double()).abs().max() / ref.double().abs().max())
        oracle_check = {"receivers": nr_c, "edges": ne_c, "tolerance": 1e-4,
                        "out_max_rel": rel(out2[:nr_c].view(nr_c, 40, C), o_out),
                        "dL_dvec_max_rel": rel(PFm[:ne_c], o_gv),
                        # mm_conv2_bwd's dL/dX rows are 16-channel-block-major: gX[s][cb][k][16]
                        "dL_dX_max_rel": rel(gXm[:nn_c].view(nn_c, 8, 4, 16).permute(0, 2, 1, 3).reshape(nn_c, 4, C),
                                             o_gx)}
        oracle_check["pass"] = all(oracle_check[k] < 1e-4 for k in ("out_max_rel", "dL_dvec_max_rel",
                                                                      "dL_dX_max_rel"))
    line = base_line(a, "edge-conv achieved algorithmic GB/s (layer-2 forward, one 16,384-receiver chunk)", v["GBps"],
                     v["ms_per_launch"], "GB/s",
                     "synthetic (config-3 topology; random unit directions x U[0.8, 6] A, N(0,1) features and "
                     "cotangents, spline tables of the random-init model)",
                     {"workload": "config2: edge-convolution kernels on chunk 0 (16,384 receivers) of the 98,304-atom "
                                  "water box", "edges": E, "receivers": nC, "nodes": nN,
                      "check_vs_FusedConvTP_max_rel": err, "check_vs_oracle": oracle_check},
                     roofline_of(kernels, {"config": 2, "chunk": 16384}), kernels, cpu)
    line["steps_note"] = "steps = launches of each kernel"
    if a.copy_calib_mib > 0:
        copy_calibration(a.copy_calib_mib)
    return line


def sub_line(line):
    """The summary of a configuration measured inside the default run."""
    keep = ("metric", "value", "unit", "steps", "warmup", "ms_per_step", "higher_is_better", "config", "roofline",
            "kernels", "node_kernels", "step_roofline", "cpu_baseline", "roofline_note", "steps_note")
    return {k: line[k] for k in keep if k in line}


def free_gpu():
    import gc

    import torch
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()


def symc_gemm_probe():
    """The layer-1 symmetric contraction as the kernel runs it against the dense-monomial form a matrix-core version
    would need, on 131,072 nodes of one species.  The contraction is channelwise: out[n, M, c] = sum over the 968
    monomials (degree 1..3) of x[n, :, c] times a coefficient that depends on (monomial, M, species, c), so it is a
    batched GEMM over the 128 channels, [nodes, 968] x [968, 4 outputs] (4 padded to the 16 columns of an MFMA tile).
    Timed: mm_symc1_fwd as built; forming the monomials (torch elementwise ops on a slice of 8,192 nodes, scaled);
    the batched fp32 GEMM of that slice in hipBLASLt (torch.bmm), scaled, with 4 and 16 output columns."""
    import torch

    from mace_onegpu import model as mm
    from mace_onegpu._lib import K, stream
    from mace_onegpu.fast_layers import FastLayers
    C, n, nb = 128, 131072, 8192
    fl = FastLayers(mm.MaceModel(seed=0), [0, 7], device="cuda")
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(n, 16 * C, device="cuda", generator=g)
    spec = torch.zeros(n, dtype=torch.int32, device="cuda")
    out = torch.empty(n, 4 * C, device="cuda")

    def timed(fn, k=10):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(k):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / k

    t_kernel = timed(lambda: K.mm_symc1_fwd(n, x, 16 * C, spec, fl.Wsc1, out, 4 * C, stream()))
    xs = x[:nb].view(nb, 16, C).permute(2, 0, 1).contiguous()            # [C, nb, 16]
    i2 = torch.tensor([(i, j) for i in range(16) for j in range(i, 16)], device="cuda")
    i3 = torch.tensor([(i, j, k) for i in range(16) for j in range(i, 16) for k in range(j, 16)], device="cuda")
    form = lambda: torch.cat([xs, xs[..., i2[:, 0]] * xs[..., i2[:, 1]],
                              xs[..., i3[:, 0]] * xs[..., i3[:, 1]] * xs[..., i3[:, 2]]], -1)
    A = form()                                                             # [C, nb, 968]
    t_form = timed(form)
    res = {}
    for nout in (4, 16):
        B = torch.randn(C, A.shape[-1], nout, device="cuda", generator=g)
        t = timed(lambda: torch.bmm(A, B))
        res[nout] = (t, 2.0 * C * nb * A.shape[-1] * nout / (t * 1e-3) / 1e12)
    scale = n / nb
    print(json.dumps({"probe": "symmetric contraction, layer 1, 131072 nodes x 128 channels, one species",
                      "monomials": int(A.shape[-1]), "mm_symc1_fwd_ms": round(t_kernel, 4),
                      "form_monomials_ms_scaled": round(t_form * scale, 3),
                      "bmm_fp32_4col_ms_scaled": round(res[4][0] * scale, 3), "bmm_fp32_4col_TFLOPs": round(res[4][1], 2),
                      "bmm_fp32_16col_ms_scaled": round(res[16][0] * scale, 3),
                      "bmm_fp32_16col_TFLOPs": round(res[16][1], 2)}), flush=True)


def run_capacity(a):
    """Memory and exactness at scale: the configuration-5 water box and its periodic replicas evaluated by
    ReceiverChunkMACE (chunk 131072, eager chunks) in three memory layouts: the default one with the pass-A
    layer-1 cache, without it, and low_memory (chunk topologies per pass, per-chunk force sums: the reference's
    layout).  Per run: peak device GB (torch allocator), seconds per E+F, E/N and, for replicas, the largest
    deviations of per-atom energies and forces from the base box's (atom j of a replica is atom j % N of the base).
    resident bytes per atom = the slope of peak GB against N between the base and the largest replica that fits;
    the largest N on this GPU follows from that line and the device's memory.  A layout is not tried on replicas
    larger than one it ran out of memory on."""
    import torch

    from mace_onegpu import model as mm, systems
    from mace_onegpu.receiver_chunk_mace import ReceiverChunkMACE, System
    pos, box, Z = systems.water_box(a.n_mol, seed=0)
    model = mm.MaceModel(seed=0)
    reps = [tuple(int(x) for x in r.split("x")) for r in a.capacity.split(",")]
    modes = {"cache_on": dict(cache_layer1=True), "cache_off": dict(cache_layer1=False),
             "low_memory": dict(low_memory=True)}
    runs, base = [], {}

    def one(rp, mode, rec):
        n_rep = rp[0] * rp[1] * rp[2]
        p_r, b_r, z_r = systems.replicate(pos, box, Z, rp) if n_rep > 1 else (pos, box, Z)
        rec["atoms"] = len(p_r)
        s = System(p_r, b_r, z_r - 1, 6.0, "cuda")
        s.build_neighbors()
        ev = ReceiverChunkMACE(model, chunk=a.chunk or 131072, device="cuda", **modes[mode])
        ev.compute(s)                  # set-up call (tables, workspaces)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        E, eat, F, PF = ev.compute(s)
        torch.cuda.synchronize()
        rec.update(pairs=int(s.rowptr[-1]), s_per_EF=round(time.perf_counter() - t0, 4), E_per_atom_eV=E / s.N,
                   peak_GB=round(torch.cuda.max_memory_allocated() / 1e9, 3))
        perm = s.perm.long()
        Fo = torch.empty_like(F)
        Fo[perm] = F
        eo = torch.empty_like(eat)
        eo[perm] = eat
        if n_rep == 1:
            base[mode] = (E / s.N, Fo.cpu(), eo.cpu())
        elif mode in base:
            E0, F0, e0 = base[mode]
            rec.update(dE_per_atom_vs_base=abs(E / s.N - E0),
                       max_abs_de_i_vs_base=float((eo.cpu() - e0.repeat(n_rep)).abs().max()),
                       max_abs_dF_vs_base=float((Fo.cpu() - F0.repeat(n_rep, 1)).abs().max()),
                       max_abs_F=float(F0.abs().max()))

    for mode in modes:
        for rp in reps:
            free_gpu()
            print(f"# capacity: replica {rp}, {mode}", file=sys.stderr, flush=True)
            rec = {"replica": "x".join(map(str, rp)), "layout": mode}
            try:
                one(rp, mode, rec)
            except torch.cuda.OutOfMemoryError as exc:
                rec["out_of_memory"] = str(exc).splitlines()[0][:200]
            print(json.dumps(rec), file=sys.stderr, flush=True)
            runs.append(rec)
            if "out_of_memory" in rec:
                break
    free_gpu()
    total = torch.cuda.get_device_properties(0).total_memory / 1e9
    out = {"capacity": "configuration-5 water box and periodic replicas, ReceiverChunkMACE E+F, chunk "
                       f"{a.chunk or 131072}", "device_GB": round(total, 1), "runs": runs}
    for mode in modes:
        ok = sorted((r for r in runs if r["layout"] == mode and "peak_GB" in r), key=lambda r: r["atoms"])
        if len(ok) >= 2:
            slope = (ok[-1]["peak_GB"] - ok[0]["peak_GB"]) * 1e9 / (ok[-1]["atoms"] - ok[0]["atoms"])
            icpt = ok[0]["peak_GB"] - slope * ok[0]["atoms"] / 1e9
            out[mode] = {"resident_bytes_per_atom": round(slope), "fixed_GB": round(icpt, 2),
                         "largest_atoms_estimate": int((total - icpt) * 1e9 / slope),
                         "largest_measured": ok[-1]["atoms"]}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=None, choices=[1, 2, 3, 4, 5],
                    help="run one configuration only (default: configuration 5, then 3, 4, 2 and 1 in the same run)")
    ap.add_argument("--n-mol", type=int, default=343000, help="config 5: water molecules")
    ap.add_argument("--chunk", type=int, default=None, help="receiver chunk (default: 131072; config 3: 16384)")
    ap.add_argument("--graphs", action="store_true", default=None,
                    help="replay full chunks from HIP graphs (default on for configs 5 and 3)")
    ap.add_argument("--no-graphs", dest="graphs", action="store_false", help="run every chunk eagerly")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="after the timed steps, run a plain elementwise kernel over this many MiB (reads and "
                         "writes a buffer of known size: calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--capacity", default=None, metavar="REPLICAS",
                    help="memory and replica exactness at scale, e.g. 1x1x1,2x2x2: the configuration-5 box and its "
                         "periodic replicas, layer-1 cache on and off; prints one JSON object and exits")
    ap.add_argument("--symc-gemm-probe", action="store_true",
                    help="time the layer-1 symmetric contraction against its dense-monomial GEMM form and exit")
    a = ap.parse_args()
    a.cpu_from = None
    if a.symc_gemm_probe:
        symc_gemm_probe()
        return
    if a.capacity:
        run_capacity(a)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        exit_multi_gpu()
    only = a.config is not None
    cfg = a.config or 5
    if cfg == 5:
        a.config = 5
        a.chunk = a.chunk or 131072
        a.graphs = True if a.graphs is None else a.graphs
        line = run_md(a)
    elif cfg in (3, 4):
        line = run_ef(a)
    elif cfg == 2:
        line = run_conv(a)
    else:
        line = run_config1(a)
    if not only:
        # the other configurations in the same process, each with its own roofline and per-kernel table
        extras = {}
        for c, steps, warm in ((3, 20, 2), (4, 8, 1), (2, 20, 2), (1, 20, 2)):
            free_gpu()
            print(f"# configuration {c}", file=sys.stderr, flush=True)
            b = argparse.Namespace(**vars(a))
            b.config, b.steps, b.warmup, b.chunk, b.graphs, b.copy_calib_mib = c, steps, warm, None, None, 0
            b.cpu_from = None
            run = {1: run_config1, 2: run_conv, 3: run_ef, 4: run_ef}[c]
            extras[f"config{c}"] = sub_line(run(b))
        line["configs"] = extras
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python
"""Benchmark of the MI355X three-pass MACE path: BASELINE configuration 5 on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--n-mol 343000] [--chunk 131072] [--no-cpu]

Workload (the metric's "1M-atom water"): 343,000 rigid H2O molecules (1,029,000
atoms) at 1.0 g/cm^3, random-init MPA-0-medium architecture, fp32 kernels, velocity-Verlet MD (dt 0.5 fs, 300 K
Maxwell-Boltzmann start, neighbour skin 2 A, rebuild when an atom moved > 1 A).  One step = one MD step
(per-step pair filter, energy + forces by the three passes, integration, rebuilds when due).  W untimed steps,
then K timed steps between synchronisations.  Prints ONE JSON line.
  roofline     : the dominant edge-convolution kernel, algorithmic bytes per launch / mean launch time measured
                 with HIP events on the launch stream during the timed steps, against 8 TB/s HBM
  cpu_baseline : the fp64 CPU oracle (oracle/mace_ref.py, a restatement of the reference's three-pass algorithm)
                 on a bounded sample of the same workload (one 512-molecule box of the same generator, one full
                 energy + force evaluation), in atom-steps/s
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mace-million_amd"))

HBM_PEAK_GBS = 8000.0
VALU_F32_PEAK_TFLOPS = 78.6      # fp32 vector FMA without packed-FP32 instructions (the build disables them)
MFMA_F32_PEAK_TFLOPS = 157.3


def conv_algorithmic(name, E, nC, N, tab, Kp=128):
    """Algorithmic HBM bytes and FLOPs of one convolution launch (per-edge, per-receiver and per-node terms;
    tables read once).  P = distinct tables (1: this model's radial weights do not depend on the species).
    ace1_*: layer 1 in the density-projection form -- per edge the 16 B record and 16 harmonics (fwd; bwd also
    writes 17 floats), the 64-feature table once, B / gB [nC, 16, Kp] once; FLOPs = the 64 x 16 outer product
    (fwd) or its two transposed products (bwd) plus the spline evaluation."""
    C, P, M = 128, 1, 512
    if name.startswith("ace1"):
        tab_bytes = 16 * (M - 1) * 64
        if name == "ace1_fwd":
            return 80 * E + 4 * (nC + 1) + tab_bytes + 4 * nC * 16 * Kp + 4 * nC, 2 * E * 64 * 16 + 6 * E * 64
        return 148 * E + 4 * (nC + 1) + tab_bytes + 4 * nC * 16 * Kp, 4 * E * 64 * 16 + 10 * E * 64
    nX, nW, nO, nT = tab["nX"], tab["nW"], tab["nO"], len(tab["terms"])
    gx = 1 if name == "conv2_bwd" else 0
    if name.endswith("fwd"):
        B = 16 * E + 4 * (nC + 1) + N * (4 * nX * C + 4) + 8 * P * M * nW * C + 4 * nC * nO * C
        F = 2 * E * C * (nT + 4 * nW)
    else:
        B = 28 * E + 4 * (nC + 1) + N * (4 * nX * C * (1 + gx) + 4) + 8 * P * M * nW * C + 4 * nC * nO * C
        F = 2 * E * C * ((2 + gx) * nT + 8 * nW)
    return B, F


def kernel_sources_digest():
    """sha256 over the HIP sources of the library (csrc/ and csrc/gen/), to tie measurements to the kernels."""
    import hashlib
    h = hashlib.sha256()
    base = os.path.join(ROOT, "mace-million_amd", "csrc")
    for d in (base, os.path.join(base, "gen")):
        for f in sorted(os.listdir(d)):
            if f.endswith((".hip", ".h", ".cpp")):
                with open(os.path.join(d, f), "rb") as fh:
                    h.update(f.encode() + fh.read())
    return h.hexdigest()


def measured_traffic(kernel, n_mol, chunk):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes of this
    workload (profiles/traffic_config5_water1M.json: counters scaled by a copy kernel of known size), or None
    when no pass was recorded for this workload and these kernel sources."""
    path = os.path.join(ROOT, "profiles", "traffic_config5_water1M.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        t = json.load(fh)
    if (t["workload"] != {"n_mol": n_mol, "chunk": chunk} or kernel not in t["kernels"]
            or t.get("kernel_sources_sha256") != kernel_sources_digest()):
        return None
    return t["kernels"][kernel]["traffic_bytes_per_launch"]


def cpu_baseline(seed=0):
    """fp64 CPU oracle, one full E+F of a 512-molecule box from the same generator."""
    import torch

    sys.path.insert(0, ROOT)
    import numpy as np
    from mace_onegpu import model as mm, o3, systems
    from oracle import mace_ref, neighbors

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    model = mm.MaceModel(seed=0)
    m = mace_ref.RefModel(model, o3.coupling)
    pos, box, Z = systems.water_box(512, seed=seed)
    s = neighbors.SystemRef(pos, box, Z - 1, 6.0)
    NN, rp, send = s.build_neighbors()
    recv = np.repeat(np.arange(s.N), NN)
    mace_ref.silu_norm()
    t0 = time.perf_counter()
    mace_ref.three_pass(m, s.pos, box, s.spidx, recv, send, chunk=512)
    dt = time.perf_counter() - t0
    return dict(value=s.N / dt, unit="atom-steps/s", cores=ncores, kind="port",
                sample=f"fp64 CPU oracle (oracle/mace_ref.three_pass), one E+F of a 512-molecule water box "
                       f"({s.N} atoms, {len(send)} pairs, chunk 512), {dt:.1f} s on {ncores} threads")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n-mol", type=int, default=343000)
    ap.add_argument("--chunk", type=int, default=131072)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="after the timed steps, copy a buffer of this many MiB once (a plain copy kernel of known "
                         "size that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU: the multi-GPU path (spatial domain "
                                   "decomposition with RCCL halo exchange) is designed, not built; use --gpus 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    from mace_onegpu import model as mm, systems
    from mace_onegpu.md import MDRunner

    dev = "cuda"
    t0 = time.perf_counter()
    pos, box, Z = systems.water_box(a.n_mol, seed=0)
    t_gen = time.perf_counter() - t0
    model = mm.MaceModel(seed=0)
    md = MDRunner(model, pos, box, Z, chunk=a.chunk, skin=2.0, dt_fs=0.5, T=300.0, seed_v=4, device=dev)
    N = md.skin_sys.N
    print(f"# generated {N} atoms (L = {box[0]:.3f} A) in {t_gen:.1f} s; chunk {a.chunk}", file=sys.stderr, flush=True)
    md.forces()                      # initial forces (set-up: builds the tables and chunk workspaces)
    for i in range(a.warmup):
        md.step()
        print(f"# warmup step {i}: E/N {md.E / N:.6f} eV", file=sys.stderr, flush=True)
    rebuilds0 = md.n_rebuild
    fl = md.ev.fl
    fl.start_kernel_timing()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        md.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ktimes = fl.stop_kernel_timing()
    if a.copy_calib_mib > 0:
        from mace_onegpu._lib import K, stream
        n = a.copy_calib_mib << 18
        src = torch.empty(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        K.mm_fill_f32(src, n, 1.0, stream())      # writes n * 4 bytes
        torch.mul(src, 2.0, out=dst)              # reads n * 4 bytes, writes n * 4 bytes
        torch.cuda.synchronize()
        del src, dst
    n_pairs = int(md.pairs.E)
    value = N * a.steps / dt
    # roofline of the dominant convolution kernel
    kernels = {}
    for name, d in ktimes.items():
        tab = fl.tables.tp1 if name.startswith("conv1") else fl.tables.tp2
        Kp = getattr(fl, "ace_Kp", 128)
        B = sum(conv_algorithmic(name, *u, tab, Kp)[0] for u in d["units"])
        F = sum(conv_algorithmic(name, *u, tab, Kp)[1] for u in d["units"])
        sec = d["ms_total"] * 1e-3
        kernels[name] = dict(launches=d["launches"], ms_per_launch=d["ms_total"] / d["launches"],
                             ms_per_step=d["ms_total"] / a.steps, GBps=B / sec / 1e9, TFLOPs=F / sec / 1e12,
                             hbm_frac=B / sec / 1e9 / HBM_PEAK_GBS,
                             bytes_per_launch=B / d["launches"], flops_per_launch=F / d["launches"])
        if name.startswith("ace1"):      # the edge products run on MFMA
            kernels[name]["mfma_frac"] = F / sec / 1e12 / MFMA_F32_PEAK_TFLOPS
        else:
            kernels[name]["valu_frac"] = F / sec / 1e12 / VALU_F32_PEAK_TFLOPS
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"]) if kernels else None
    roof = None
    if dom:
        k = kernels[dom]
        roof = {"kernel": f"mm_{dom}_kernel", "bound": "hbm", "achieved": round(k["GBps"], 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(k["hbm_frac"], 5),
                "traffic": measured_traffic(f"mm_{dom}_kernel", a.n_mol, a.chunk),
                "flop_rate_TFLOPs": round(k["TFLOPs"], 3),
                **{f: round(k[f], 4) for f in ("valu_frac", "mfma_frac") if f in k},
                "bytes_per_launch": int(k["bytes_per_launch"]), "ms_per_launch": round(k["ms_per_launch"], 4),
                "launches": k["launches"]}
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline()
    line = {
        "metric": "atom-steps/s (E+F, 1M-atom water, fp32, 1 GPU)",
        "value": round(value, 1), "unit": "atom-steps/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(dt / a.steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic (seeded water generator, random-init weights)",
        "config": {"workload": "config5: 343,000-molecule water (1,029,000 atoms), random-init MPA-0-medium "
                               "architecture, velocity-Verlet MD dt 0.5 fs, skin 2 A",
                   "atoms": N, "pairs": n_pairs, "chunk": a.chunk, "rebuilds_timed": md.n_rebuild - rebuilds0,
                   "peak_hbm_GB": round(torch.cuda.max_memory_allocated() / 1e9, 2),
                   "box_A": round(float(box[0]), 4)},
        "roofline": roof,
        "kernels": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kernels.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

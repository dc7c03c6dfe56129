"""Velocity-Verlet molecular dynamics driven by the three-pass evaluator (benchmark configuration 5).

The reference runs MD through LAMMPS (inputs/in.water_scan.lmp: nve, neighbour skin, ML-IAP pair list within the
cutoff every step) and benchmarks the evaluator standalone (graphed_three_pass.py).  This driver keeps the whole
step on the GPU:
  * a skin neighbour list (cell list with r_cut = r_max + skin, System: Morton-sorted atoms, bit-exact build);
  * every step the pairs within r_max are filtered from the skin list (mm_nl_filter_*, candidate order kept);
  * energy + forces by ReceiverChunkMACE (three passes over receiver chunks);
  * kick-drift-kick velocity Verlet in metal units (eV, A, ps, amu; 1 eV/(A amu) = 9648.533 A/ps^2);
  * the skin list is rebuilt (atoms re-sorted, velocities and masses permuted with them) as soon as an atom has
    moved more than skin / 2 since the last build.
"""
import numpy as np
import torch

from ._lib import K, stream
from .receiver_chunk_mace import ReceiverChunkMACE, System, host_f64
from .systems import maxwell_boltzmann

ACC = 9648.533212331          # eV / (A amu) -> A / ps^2


class PairList:
    """Pairs within r_max filtered from a skin list (same fields as System for ReceiverChunkMACE)."""

    def __init__(self, skin_sys, r_max):
        self.N, self.device, self.box = skin_sys.N, skin_sys.device, skin_sys.box
        self.pos, self.spidx = skin_sys.pos, skin_sys.spidx
        self.r_max = r_max
        self._skin = skin_sys
        self._box_h = host_f64(skin_sys.box)
        self.NN = torch.empty(self.N, dtype=torch.int32, device=self.device)
        self.rowptr = torch.empty(self.N + 1, dtype=torch.int64, device=self.device)
        self.send = None
        # per skin pair: its index in the filtered list (-1 if dropped) and the skin index of its reverse pair; the
        # per-atom forces of every step are summed through them (mm_pair_forces_skin, no per-step sort)
        E_s = int(skin_sys.rowptr[-1])
        self.fidx = torch.empty(max(E_s, 1), dtype=torch.int32, device=self.device)
        self.rev = reverse_pairs(skin_sys)

    def refresh(self):
        s = self._skin
        r2 = self.r_max ** 2
        # the count pass leaves its keep flags in fidx, so the fill pass does not test the distances again
        K.mm_nl_filter_count(self.pos, self.N, self._box_h, s.rowptr, s.send, r2, self.NN, self.fidx, stream())
        K.mm_nl_scan(self.NN, self.rowptr, self.N, s._ws, s._ws.numel(), stream())
        self.rp_cpu = self.rowptr.cpu().numpy()          # the one device-to-host read of a step
        E = int(self.rp_cpu[-1])
        if self.send is None or self.send.numel() < E:
            self.send = torch.empty(int(E * 1.1) + 1, dtype=torch.int32, device=self.device)
        K.mm_nl_filter_fill(self.pos, self.N, self._box_h, s.rowptr, s.send, r2, self.rowptr, self.send, self.fidx, 1,
                            stream())
        self.E = E
        self.send_view = self.send[:E]
        return E

    def chunk_graphs(self, chunk, col2s):
        """Chunks of the current filtered pairs for ReceiverChunkMACE, without per-chunk device-to-host reads.

        The node list of a chunk (its receivers, then the senders outside it in ascending order, as
        chunk_topology builds it) is taken from the SKIN list once per neighbour-list rebuild: a superset of the
        senders of every filtered list until the next rebuild.  Rows of senders that no filtered edge uses are
        computed and never read.  Per step, the local sender index of every filtered edge is one gather,
        loc[chunk(recv), send]; the chunk objects (and the species lists FastLayers keeps on them) persist."""
        from .receiver_chunk_mace import chunk_topology, ChunkGraph
        dev, N = self.device, self.N
        key = (int(chunk), col2s.data_ptr())      # col2s: model column -> compact species of the layers
        if getattr(self, "_tmpl_key", None) != key:
            s = self._skin
            node_spec_all = col2s[self.spidx.long()]
            rp_s = s.rowptr.cpu().numpy()
            loc = torch.full((N,), -1, dtype=torch.int32, device=dev)
            flag = torch.zeros(N, dtype=torch.bool, device=dev)
            n_chunks = (N + chunk - 1) // chunk
            self._loc2d = torch.full((n_chunks, N), -1, dtype=torch.int32, device=dev)
            self._tmpl = []
            for c, a in enumerate(range(0, N, chunk)):
                b = min(a + chunk, N)
                nodes, _ = chunk_topology(a, b, int(rp_s[a]), int(rp_s[b]), s.send, loc, flag)
                self._loc2d[c, nodes.long()] = torch.arange(nodes.numel(), device=dev, dtype=torch.int32)
                g = ChunkGraph()
                g.a, g.b, g.nC = a, b, b - a
                g.nodes = nodes.contiguous()
                g.n_nodes = nodes.numel()
                g.node_spec = node_spec_all[g.nodes.long()].contiguous()
                self._tmpl.append(g)
            self._tmpl_key = key
        E = self.E
        if getattr(self, "_ls_all", None) is None or self._ls_all.numel() < E:
            self._ls_all = torch.empty(int(E * 1.1) + 1, dtype=torch.int32, device=dev)
            self._recv_local = torch.empty_like(self._ls_all)
        # every chunk's local sender rows and local receivers in one pass over the filtered pairs
        K.mm_chunk_edge_index(N, self.rowptr, self.send_view, self._loc2d, chunk, self._ls_all, self._recv_local,
                              stream())
        rp = self.rp_cpu
        for g in self._tmpl:
            e0, e1 = int(rp[g.a]), int(rp[g.b])
            g.e0, g.e1, g.nE = e0, e1, e1 - e0
            g.ls = self._ls_all[e0:e1]
            g.rowptr = (self.rowptr[g.a:g.b + 1] - e0).to(torch.int32)
            g.recv_local = self._recv_local[e0:e1]
            g.pos, g.box_host = self.pos, self._box_h
        return self._tmpl

    def atom_forces(self, PF):
        """F_i = -sum_{pairs (i, j)} PF + sum_{pairs (j, i)} PF of the current filtered list (fp64)."""
        F = torch.empty(self.N, 3, dtype=torch.float64, device=self.device)
        K.mm_pair_forces_skin(self.N, self._skin.rowptr, self.fidx, self.rev, PF, F, stream())
        return F


def reverse_pairs(sysm):
    """rev[e] = index of the pair (j, i) for every pair e = (i, j) of a symmetric CSR neighbour list (the cell-list
    test is symmetric bit for bit: d(j, i) = -d(i, j) exactly in fp64), by mm_nl_reverse: each pair's reverse is
    found by scanning the sender's row, so the map needs no memory beyond its own int32 per pair."""
    E = int(sysm.send.numel())
    rev = torch.full((max(E, 1),), -1, dtype=torch.int32, device=sysm.send.device)
    K.mm_nl_reverse(sysm.rowptr, sysm.send, sysm.N, E, rev, stream())
    if E and int(rev[:E].min()) < 0:
        raise RuntimeError("neighbour list is not symmetric")
    return rev


class MDRunner:
    def __init__(self, model, pos, box, Z, chunk=65536, skin=2.0, dt_fs=0.5, T=300.0, seed_v=4, device="cuda",
                 spline_grid=512, use_graphs=False, deterministic=None):
        self.model = model
        self.dev = torch.device(device)
        self.r_max = float(model.spec.r_max)
        self.skin = float(skin)
        self.dt = dt_fs * 1e-3                          # ps
        self.box = np.asarray(box, dtype=np.float64)
        Z = np.asarray(Z)
        v, m = maxwell_boltzmann(Z, T, seed_v)
        self.Z = torch.as_tensor(Z, device=self.dev)
        self.vel = torch.as_tensor(v, dtype=torch.float64, device=self.dev)
        self.mass = torch.as_tensor(m, dtype=torch.float64, device=self.dev)
        self.gid = torch.arange(len(Z), device=self.dev)       # original atom index of each current slot
        self.ev = ReceiverChunkMACE(model, chunk=chunk, spline_grid=spline_grid, device=self.dev,
                                    use_graphs=use_graphs, deterministic=deterministic)
        self.n_rebuild = 0
        self._build(torch.as_tensor(pos, dtype=torch.float64, device=self.dev))
        self.F = None
        self.E = None
        self.eat = None

    def _build(self, pos):
        # the previous lists go first: the new skin list is then built in their memory
        self.pairs = self.skin_sys = None
        spidx = (self.Z - 1).to(torch.int32)
        s = System(pos, self.box, spidx, self.r_max + self.skin, device=self.dev)
        perm = s.perm
        self.vel, self.mass, self.Z, self.gid = self.vel[perm], self.mass[perm], self.Z[perm], self.gid[perm]
        s.build_neighbors()
        self.skin_sys = s
        self.pos = s.pos                                   # updated in place by the integrator
        self.x_build = s.pos.clone()
        self.pairs = PairList(s, self.r_max)
        self.n_rebuild += 1

    def forces(self):
        pl = self.pairs
        pl.refresh()
        view = _PairView(pl)
        E, eat, F, PF = self.ev.compute(view)
        self.E, self.eat, self.F = E, eat, F
        return E, F

    def _maybe_rebuild(self):
        disp = (self.pos - self.x_build).norm(dim=1).max()
        if float(disp) > 0.5 * self.skin:
            self._build(self.pos.clone())
            return True
        return False

    def step(self):
        if self.F is None:
            self.forces()
        a = self.F / self.mass[:, None] * ACC
        self.vel.add_(0.5 * self.dt * a)
        self.pos.add_(self.dt * self.vel)
        rebuilt = self._maybe_rebuild()
        self.forces()
        a = self.F / self.mass[:, None] * ACC
        self.vel.add_(0.5 * self.dt * a)
        return rebuilt

    def kinetic(self):
        return float(0.5 * (self.mass[:, None] * self.vel ** 2).sum() / ACC)


class _PairView:
    """System-like view of a PairList for ReceiverChunkMACE (send trimmed to the current pair count)."""

    def __init__(self, pl):
        self.N, self.device, self.box, self.pos, self.spidx = pl.N, pl.device, pl.box, pl.pos, pl.spidx
        self.NN, self.rowptr, self.send = pl.NN, pl.rowptr, pl.send_view
        self.atom_forces_fn = pl.atom_forces
        self.chunk_graphs = pl.chunk_graphs


def main(argv=None):
    """Command line of the MD driver: velocity-Verlet NVE from Maxwell-Boltzmann velocities, forces by the
    three-pass evaluator over a skin neighbour list (the standalone MD loop of the reference's
    graphed_three_pass.py:83-334 and its benchmark decks).  Prints the energies every --every steps, then the
    throughput (atom-steps/s over the whole run, rebuilds included), the total-energy drift and the peak memory.

        python -m mace_onegpu.md --water 343000 --steps 100 --graphs --json md.json
    """
    import argparse
    import json
    import time

    from . import systems
    from .model import from_arg

    ap = argparse.ArgumentParser(prog="python -m mace_onegpu.md", description=main.__doc__.split("\n\n")[0])
    ap.add_argument("--model", default="seed:0", help='"seed:N" (random-init weights) or a weights file')
    systems.add_structure_args(ap)
    ap.add_argument("--chunk", type=int, default=131072, help="receivers per chunk")
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--dt-fs", type=float, default=0.5)
    ap.add_argument("--T", type=float, default=300.0, help="initial temperature (K)")
    ap.add_argument("--seed-v", type=int, default=4, help="seed of the initial velocities")
    ap.add_argument("--skin", type=float, default=2.0, help="neighbour-list skin (A); rebuilt at skin / 2 moved")
    ap.add_argument("--graphs", action="store_true", help="replay full chunks from HIP graphs")
    ap.add_argument("--deterministic", action="store_true", help="bitwise-repeatable trajectories")
    ap.add_argument("--every", type=int, default=10, help="print the energies every this many steps")
    ap.add_argument("--json", default=None, help="write the results here")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("the MD driver runs on the GPU; no GPU is visible")
    pos, box, Z, _ = systems.structure_from_args(a)
    N = len(pos)
    md = MDRunner(from_arg(a.model), pos, box, Z, chunk=a.chunk, skin=a.skin, dt_fs=a.dt_fs, T=a.T,
                  seed_v=a.seed_v, device="cuda", use_graphs=a.graphs, deterministic=True if a.deterministic else None)
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    md.forces()
    e_tot = [md.E + md.kinetic()]
    print(f"N={N:,} steps={a.steps} dt={a.dt_fs} fs T0={a.T} K chunk={a.chunk} graphs={a.graphs}: "
          f"E_pot {md.E:.6f} E_kin {md.kinetic():.6f} eV", flush=True)
    for k in range(a.steps):
        md.step()
        e_tot.append(md.E + md.kinetic())
        if a.every and (k + 1) % a.every == 0:
            print(f"step {k + 1}: E_pot {md.E:.6f} E_kin {md.kinetic():.6f} E_tot {e_tot[-1]:.6f} eV "
                  f"builds {md.n_rebuild}", flush=True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res = dict(N=N, steps=a.steps, dt_fs=a.dt_fs, chunk=a.chunk, graphs=a.graphs, wall_s=wall,
               atom_step_per_s=N * a.steps / wall, E_tot_range=float(np.ptp(e_tot)), E_pot=md.E,
               E_kin=md.kinetic(), builds=md.n_rebuild, peak_gb=torch.cuda.max_memory_allocated() / 1e9)
    print(f"{res['atom_step_per_s']:.3e} atom-steps/s ({wall:.2f} s for {a.steps} steps and the first force call), "
          f"E_tot range {res['E_tot_range']:.3e} eV, {md.n_rebuild} neighbour-list builds, "
          f"peak {res['peak_gb']:.1f} GB", flush=True)
    if a.json:
        with open(a.json, "w") as fh:
            json.dump(res, fh, indent=1)
    return res


if __name__ == "__main__":
    main()

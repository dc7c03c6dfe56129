"""ML-IAP unified data object of one GPU that owns a whole periodic box: periodic images stand in for ghosts.

LAMMPS hands ThreePassMLIAP.compute_forces (mliap_threepass.py:444-605) an object with nlocal, ntotal, npairs,
elems, pair_i (local receiver), pair_j (local or ghost sender), rij (pair vector used as MACE's edge vector,
x_i - x_j), eatoms, energy, forward_exchange(src, dst, D), reverse_exchange(src, dst, D) and
update_pair_forces_gpu(PF).  This class builds the same object without LAMMPS:
  * local atoms = the System's atoms (Morton order), pairs = its neighbour list within r_max;
  * every pair whose minimum image crosses the box gets a ghost sender: the periodic image (j, shift) of its
    owner, one ghost per distinct (owner, shift); rij = x_i - x_j - shift * L (the fp64 minimum image);
  * forward_exchange copies owner rows to ghost rows, reverse_exchange sums ghost rows into owners
    (csrc/node.hip mm_ghost_forward / mm_ghost_reverse);
  * update_pair_forces_gpu keeps PF and assembles per-atom forces the way LAMMPS does
    (f_i -= PF, f_j += PF, then ghost forces summed onto owners).
"""
import torch

from ._lib import K, stream


class PeriodicMLIAPData:
    def __init__(self, sysm, elems, ghosts=True, shuffle_pairs_seed=None):
        """sysm: System with neighbour list built; elems: model element index per sorted atom (int)."""
        dev = sysm.device
        N = sysm.N
        self.device = dev
        self.nlocal = N
        recv = torch.repeat_interleave(torch.arange(N, device=dev, dtype=torch.int64), sysm.NN.long())
        send = sysm.send.long()
        box = torch.as_tensor(sysm.box, dtype=torch.float64, device=dev)
        raw = sysm.pos[recv] - sysm.pos[send]
        shift = torch.round(raw / box)                         # image shift of the sender, in box lengths
        rij = raw - box * shift                                # == the minimum image of System.min_image
        pj = send.clone()
        owner = torch.zeros(0, dtype=torch.int64, device=dev)
        if ghosts:
            crossing = (shift != 0).any(1)
            if bool(crossing.any()):
                code = send[crossing] * 27 + ((shift[crossing] + 1).long() * torch.tensor([9, 3, 1], device=dev)).sum(1)
                uniq, inv = torch.unique(code, return_inverse=True)
                owner = torch.div(uniq, 27, rounding_mode="floor")
                pj[crossing] = N + inv
        self.owner = owner.to(torch.int32).contiguous()
        self.nghost = int(owner.numel())
        self.ntotal = N + self.nghost
        # owner-sorted CSR of the ghosts for the reverse sum
        og = torch.argsort(owner, stable=True) if self.nghost else owner
        cnt = torch.bincount(owner, minlength=N) if self.nghost else torch.zeros(N, dtype=torch.int64, device=dev)
        self.g_rowptr = torch.zeros(N + 1, dtype=torch.int32, device=dev)
        self.g_rowptr[1:] = torch.cumsum(cnt, 0).to(torch.int32)
        self.g_list = og.to(torch.int32).contiguous() if self.nghost else torch.zeros(1, dtype=torch.int32, device=dev)
        pi = recv.to(torch.int32)
        pj = pj.to(torch.int32)
        if shuffle_pairs_seed is not None:        # LAMMPS may hand over unsorted pairs
            g = torch.Generator(device="cpu").manual_seed(int(shuffle_pairs_seed))
            p = torch.randperm(pi.numel(), generator=g).to(dev)
            pi, pj, rij = pi[p], pj[p], rij[p]
        self.pair_i, self.pair_j, self.rij = pi.contiguous(), pj.contiguous(), rij.contiguous()
        self.npairs = int(pi.numel())
        ghost_elems = torch.as_tensor(elems, device=dev)[owner] if self.nghost else torch.zeros(0, dtype=torch.int64,
                                                                                               device=dev)
        self.elems = torch.cat([torch.as_tensor(elems, device=dev).long(), ghost_elems.long()])
        self.eatoms = torch.zeros(N, dtype=torch.float64, device=dev)
        self.energy = 0.0
        self.pair_forces = None

    # ---- ghost communication (one GPU: periodic images)
    def forward_exchange(self, src, dst, D):
        K.mm_ghost_forward(src, dst, int(D), self.nlocal, self.nghost, self.owner, stream())

    def reverse_exchange(self, src, dst, D):
        K.mm_ghost_reverse(src, dst, int(D), self.nlocal, self.g_rowptr, self.g_list, stream())

    def update_pair_forces_gpu(self, PF):
        self.pair_forces = PF

    def atom_forces(self):
        """Per-atom forces of the local atoms (fp64): f_i -= PF, f_j += PF, ghost forces onto owners."""
        PF = self.pair_forces
        F = torch.zeros(self.ntotal, 3, dtype=torch.float64, device=self.device)
        F.index_add_(0, self.pair_i.long(), -PF)
        F.index_add_(0, self.pair_j.long(), PF)
        out = F[: self.nlocal].clone()
        if self.nghost:
            out.index_add_(0, self.owner.long(), F[self.nlocal:])
        return out

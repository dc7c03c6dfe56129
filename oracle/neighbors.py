"""numpy restatement of the reference's neighbour build (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Follows receiver_chunk_mace.py:82-165 operation by operation so that the result is bit-identical:
  * wrap: torch.remainder(pos, box) == fmod(pos, box), plus box where the signs differ   (:98)
  * ncell = max(1, floor(box / r_max)); cell = min(floor(pos / (box / ncell)), ncell - 1)  (:99-100)
  * 10-bit Morton code, x -> bit 3b+2, y -> 3b+1, z -> 3b; stable argsort -> perm           (:82-88, :101-106)
  * candidates of receiver i: 27 offset cells in meshgrid-"ij" order of (-1, 0, 1)^3, atoms of a cell in sorted
    order; brute force over all j ascending if any ncell < 3                                  (:117-146)
  * d = v - box * round(v / box) (round half to even), dd = (d0^2 + d1^2) + d2^2, keep dd < r_max^2 and j != i,
    candidate order preserved                                                                 (:110-111, :143-163)
Pinned by: golden vectors written by importing the reference's own System (tests/golden/), and O(N^2)
brute-force minimum-image set equality on small boxes.
"""
import numpy as np


def wrap(pos, box):
    box = np.asarray(box, dtype=np.float64)
    m = np.fmod(pos, box)
    fix = (m != 0) & ((m < 0) != (box < 0))
    return np.where(fix, m + box, m)


def morton3(cx, cy, cz, bits=10):
    code = np.zeros(cx.shape, dtype=np.int64)
    for b in range(bits):
        code |= ((cx >> b) & 1) << (3 * b + 2)
        code |= ((cy >> b) & 1) << (3 * b + 1)
        code |= ((cz >> b) & 1) << (3 * b)
    return code


class SystemRef:
    """Positions wrapped and sorted in Morton order of cells; perm maps sorted -> original index."""

    def __init__(self, pos, box, spidx, r_max):
        pos = np.asarray(pos, dtype=np.float64)
        self.box = np.asarray(box, dtype=np.float64)
        assert (self.box > 2 * r_max).all(), "minimum image needs box > 2 r_max in every direction"
        pos = wrap(pos, self.box)
        self.ncell = np.maximum(np.floor(self.box / r_max).astype(np.int64), 1)
        cs = self.box / self.ncell.astype(np.float64)
        c = np.minimum(np.floor(pos / cs).astype(np.int64), self.ncell - 1)
        code = morton3(c[:, 0], c[:, 1], c[:, 2])
        order = np.argsort(code, kind="stable")
        self.perm = order
        self.pos = pos[order]
        self.spidx = np.asarray(spidx)[order]
        self.cell = c[order]
        self.N = len(pos)
        self.r_max = float(r_max)

    def min_image(self, v):
        return v - self.box * np.round(v / self.box)

    def candidates(self, i):
        """Candidate senders of receiver i in the reference's order (with duplicates impossible for ncell >= 3)."""
        nc = self.ncell
        if (nc < 3).any():
            return np.arange(self.N)
        if not hasattr(self, "_start"):
            lin = (self.cell[:, 0] * nc[1] + self.cell[:, 1]) * nc[2] + self.cell[:, 2]
            ncells = int(np.prod(nc))
            self._counts = np.bincount(lin, minlength=ncells)
            start = np.full(ncells, self.N, dtype=np.int64)
            np.minimum.at(start, lin, np.arange(self.N))
            self._start = start
        out = []
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    cc = (self.cell[i] + np.array([dx, dy, dz])) % nc
                    cl = (cc[0] * nc[1] + cc[1]) * nc[2] + cc[2]
                    st, ct = self._start[cl], self._counts[cl]
                    out.append(np.arange(st, st + ct))
        return np.concatenate(out)

    def build_neighbors(self):
        """Returns (NN int32 [N], CSR rowptr int64 [N+1], senders int32 [E]) in the reference's edge order."""
        r2 = self.r_max ** 2
        rows = []
        for i in range(self.N):
            cand = self.candidates(i)
            d = self.min_image(self.pos[i][None, :] - self.pos[cand])
            dd = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
            ok = (dd < r2) & (cand != i)
            rows.append(cand[ok].astype(np.int32))
        NN = np.array([len(r) for r in rows], dtype=np.int32)
        rowptr = np.zeros(self.N + 1, dtype=np.int64)
        rowptr[1:] = np.cumsum(NN)
        send = np.concatenate(rows) if rows else np.zeros(0, np.int32)
        return NN, rowptr, send


def brute_force_pairs(pos, box, r_max):
    """Set of (i, j) with 0 < |mic(x_i - x_j)| < r_max, by O(N^2) enumeration (order-free check)."""
    pos = np.asarray(pos, dtype=np.float64)
    box = np.asarray(box, dtype=np.float64)
    out = set()
    for i in range(len(pos)):
        d = pos[i][None, :] - pos
        d = d - box * np.round(d / box)
        dd = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
        for j in np.nonzero((dd < r_max * r_max) & (np.arange(len(pos)) != i))[0]:
            out.add((i, int(j)))
    return out

/* Plain-C restatement of the reference's cell-list neighbour build -- TEST INFRASTRUCTURE ONLY (only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline may load it).
 *
 * Follows receiver_chunk_mace.py:82-165 (System.__init__, morton3, build_neighbors) operation by operation, with
 * every fp64 operation rounded separately (built with -ffp-contract=off), so that its output is bit-identical to
 * the reference's:
 *   wrap        m = fmod(p, L); m += L where m != 0 and sign(m) != sign(L)              (torch.remainder, :98)
 *   cells       ncell = max(1, floor(L / r_max)); c = min(floor(p / (L / ncell)), ncell - 1)        (:99-100)
 *   order       10-bit Morton code (x -> bit 3b+2, y -> 3b+1, z -> 3b), stable sort        (:82-88, :101-106)
 *   candidates  27 offset cells in meshgrid-"ij" order of (-1, 0, 1)^3, atoms of a cell in sorted order;
 *               all j ascending when some ncell < 3                                              (:117-146)
 *   keep        d = v - L * rint(v / L) (half to even), dd = (dx^2 + dy^2) + dz^2 < r_max^2, j != i   (:143-163)
 * Pinned by the golden vectors of the reference's own System (tests/golden/neighbors.npz) and by equality with the
 * numpy restatement (oracle/neighbors.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

static double wrap1(double p, double L) {
  double m = fmod(p, L);
  if (m != 0.0 && ((m < 0.0) != (L < 0.0))) m = m + L;
  return m;
}

static int64_t morton3(int64_t cx, int64_t cy, int64_t cz) {
  int64_t code = 0;
  for (int b = 0; b < 10; ++b) {
    code |= ((cx >> b) & 1) << (3 * b + 2);
    code |= ((cy >> b) & 1) << (3 * b + 1);
    code |= ((cz >> b) & 1) << (3 * b);
  }
  return code;
}

typedef struct { int64_t code; int64_t idx; } key_t_;

static int cmp_key(const void* a, const void* b) {
  const key_t_* x = (const key_t_*)a;
  const key_t_* y = (const key_t_*)b;
  if (x->code != y->code) return x->code < y->code ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);   /* index tie-break: a stable order */
}

/* Wrap, cell, Morton sort.  Outputs: perm [N] (sorted -> original), pos_sorted [N,3], cell_sorted [N,3],
 * ncell [3].  Returns 0, or -1 on allocation failure. */
int onl_sort(long N, const double* pos, const double* box, double r_max, long* ncell, long long* perm,
             double* pos_sorted, long* cell_sorted) {
  double cs[3];
  for (int k = 0; k < 3; ++k) {
    double q = floor(box[k] / r_max);
    ncell[k] = q < 1.0 ? 1 : (long)q;
    cs[k] = box[k] / (double)ncell[k];
  }
  key_t_* keys = (key_t_*)malloc(sizeof(key_t_) * (size_t)(N > 0 ? N : 1));
  double* pw = (double*)malloc(sizeof(double) * 3 * (size_t)(N > 0 ? N : 1));
  long* cl = (long*)malloc(sizeof(long) * 3 * (size_t)(N > 0 ? N : 1));
  if (!keys || !pw || !cl) { free(keys); free(pw); free(cl); return -1; }
  for (long i = 0; i < N; ++i) {
    for (int k = 0; k < 3; ++k) {
      const double p = wrap1(pos[3 * i + k], box[k]);
      long c = (long)floor(p / cs[k]);
      if (c > ncell[k] - 1) c = ncell[k] - 1;
      pw[3 * i + k] = p;
      cl[3 * i + k] = c;
    }
    keys[i].code = morton3(cl[3 * i], cl[3 * i + 1], cl[3 * i + 2]);
    keys[i].idx = i;
  }
  qsort(keys, (size_t)N, sizeof(key_t_), cmp_key);
  for (long s = 0; s < N; ++s) {
    const long i = (long)keys[s].idx;
    perm[s] = i;
    for (int k = 0; k < 3; ++k) {
      pos_sorted[3 * s + k] = pw[3 * i + k];
      cell_sorted[3 * s + k] = cl[3 * i + k];
    }
  }
  free(keys); free(pw); free(cl);
  return 0;
}

static int keep(const double* pos, const double* box, long i, long j, double r2) {
  if (j == i) return 0;
  double dd = 0.0;
  double d[3];
  for (int k = 0; k < 3; ++k) {
    const double v = pos[3 * i + k] - pos[3 * j + k];
    const double n = nearbyint(v / box[k]);
    const double t = box[k] * n;
    d[k] = v - t;
  }
  const double d0 = d[0] * d[0];
  const double d1 = d[1] * d[1];
  const double d2 = d[2] * d[2];
  dd = d0 + d1;
  dd = dd + d2;
  return dd < r2;
}

/* Neighbours of every sorted atom in the reference's candidate order.  Pass send == NULL to count only (NN);
 * with send, rowptr [N+1] must hold the exclusive prefix sum of NN.  cell_start / cell_count: scratch of
 * ncell[0] * ncell[1] * ncell[2] entries. */
int onl_neighbors(long N, const double* pos, const long* cell, const double* box, const long* ncell, double r_max,
                  long* cell_start, long* cell_count, int* NN, const long* rowptr, int* send) {
  const double r2 = r_max * r_max;
  const long nc0 = ncell[0], nc1 = ncell[1], nc2 = ncell[2];
  const int brute = nc0 < 3 || nc1 < 3 || nc2 < 3;
  const long ncells = nc0 * nc1 * nc2;
  if (!brute) {
    for (long c = 0; c < ncells; ++c) { cell_start[c] = N; cell_count[c] = 0; }
    for (long i = 0; i < N; ++i) {
      const long c = (cell[3 * i] * nc1 + cell[3 * i + 1]) * nc2 + cell[3 * i + 2];
      if (i < cell_start[c]) cell_start[c] = i;
      cell_count[c] += 1;
    }
  }
#pragma omp parallel for schedule(dynamic, 256)
  for (long i = 0; i < N; ++i) {
    int n = 0;
    long w = send ? rowptr[i] : 0;
    if (brute) {
      for (long j = 0; j < N; ++j)
        if (keep(pos, box, i, j, r2)) { if (send) send[w++] = (int)j; ++n; }
    } else {
      for (int dx = -1; dx <= 1; ++dx)
        for (int dy = -1; dy <= 1; ++dy)
          for (int dz = -1; dz <= 1; ++dz) {
            const long cx = ((cell[3 * i] + dx) % nc0 + nc0) % nc0;
            const long cy = ((cell[3 * i + 1] + dy) % nc1 + nc1) % nc1;
            const long cz = ((cell[3 * i + 2] + dz) % nc2 + nc2) % nc2;
            const long c = (cx * nc1 + cy) * nc2 + cz;
            for (long j = cell_start[c]; j < cell_start[c] + cell_count[c]; ++j)
              if (keep(pos, box, i, j, r2)) { if (send) send[w++] = (int)j; ++n; }
          }
    }
    NN[i] = n;
  }
  return 0;
}

// Node-level small kernels of the three-pass path: buffer fills (graph-capture-safe zeroing), per-species row
// lists, the two readouts with their gradients and energy accumulation, the periodic-image ghost exchange, and
// the assembly of per-atom forces from per-pair forces.
#include "common.h"

#include <math.h>

// ------------------------------------------------------------------------------------------------ fills
__global__ void mm_fill_f32_kernel(float* p, long n, float v) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = v;
}
__global__ void mm_fill_f64_kernel(double* p, long n, double v) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = v;
}
__global__ void mm_fill_i32_kernel(int* p, long n, int v) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = v;
}

static dim3 fill_grid(long n) {
  long b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return dim3((unsigned)b);
}

extern "C" int mm_fill_f32(float* p, long n, float v, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0, "negative size");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_fill_f32_kernel, fill_grid(n), dim3(256), 0, stream, p, n, v);
  return mm::launch_status("mm_fill_f32");
}
extern "C" int mm_fill_f64(double* p, long n, double v, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0, "negative size");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_fill_f64_kernel, fill_grid(n), dim3(256), 0, stream, p, n, v);
  return mm::launch_status("mm_fill_f64");
}
extern "C" int mm_fill_i32(int* p, long n, int v, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0, "negative size");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_fill_i32_kernel, fill_grid(n), dim3(256), 0, stream, p, n, v);
  return mm::launch_status("mm_fill_i32");
}

// ------------------------------------------------------------------------------------------------ species lists
// Stable partition of rows 0..n-1 by species: lists[s * stride + j] = j-th row of species s, counts[s].
// One workgroup of 1024 threads; thread t owns a contiguous segment of rows.
#define MM_MAX_SPECIES 16
__global__ void __launch_bounds__(1024) mm_species_lists_kernel(const int* __restrict__ spec, int n, int S,
                                                                int* __restrict__ lists, long stride,
                                                                int* __restrict__ counts) {
  __shared__ int cnt[MM_MAX_SPECIES][1024];
  const int t = threadIdx.x;
  const int per = (n + 1023) / 1024;
  const int b = t * per, e = min(n, b + per);
  int local[MM_MAX_SPECIES];
  for (int s = 0; s < S; ++s) local[s] = 0;
  for (int j = b; j < e; ++j) local[spec[j]]++;
  for (int s = 0; s < S; ++s) cnt[s][t] = local[s];
  __syncthreads();
  // exclusive scan per species over the 1024 thread counts (Hillis-Steele in place on a copy)
  for (int s = 0; s < S; ++s) {
    for (int off = 1; off < 1024; off <<= 1) {
      const int v = t >= off ? cnt[s][t - off] : 0;
      __syncthreads();
      cnt[s][t] += v;
      __syncthreads();
    }
  }
  int pos[MM_MAX_SPECIES];
  for (int s = 0; s < S; ++s) pos[s] = cnt[s][t] - local[s];
  for (int j = b; j < e; ++j) {
    const int s = spec[j];
    lists[(size_t)s * stride + pos[s]++] = j;
  }
  if (t == 1023)
    for (int s = 0; s < S; ++s) counts[s] = cnt[s][1023];
}

extern "C" int mm_species_lists(const int* spec, int n, int S, int* lists, long stride, int* counts,
                                hipStream_t stream) {
  MM_CHECK_ARG(S >= 1 && S <= MM_MAX_SPECIES && n >= 0 && stride >= n, "bad sizes");
  hipLaunchKernelGGL(mm_species_lists_kernel, dim3(1), dim3(1024), 0, stream, spec, n, S, lists, stride, counts);
  return mm::launch_status("mm_species_lists");
}

// ------------------------------------------------------------------------------------------------ readouts
// R1(h1) = h1[0e] . w0 (w0 = r0 / sqrt(C)); in pass C: eat[i] += scale R1_i and
// g_h1[i] = G1r[i] + scale dR1/dh1 (the loss of pass C is scale sum R1 + sum G1r . h1, mliap_threepass.py:579).
// One wave per node.
__global__ void mm_readout1_kernel(int n, const float* __restrict__ h1, long h_stride, const float* __restrict__ w0,
                                   float scale, double* __restrict__ eat, const float* __restrict__ g1r,
                                   long g1_stride, float* __restrict__ gh, long gh_stride, int D) {
  const int node = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (node >= n) return;
  const int lane = threadIdx.x & 63;
  const float* __restrict__ hp = h1 + (size_t)node * h_stride;
  float s = hp[lane] * w0[lane] + hp[lane + 64] * w0[lane + 64];
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) eat[node] += (double)(scale * s);
  if (gh) {
    const float* __restrict__ gp = g1r + (size_t)node * g1_stride;
    float* __restrict__ op = gh + (size_t)node * gh_stride;
    for (int j = lane; j < D; j += 64) op[j] = gp[j] + (j < MM_C ? scale * w0[j] : 0.f);
  }
}

extern "C" int mm_readout1(int n, const float* h1, long h_stride, const float* w0, float scale, double* eat,
                           const float* g1r, long g1_stride, float* gh, long gh_stride, int D, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0 && D >= MM_C, "bad sizes");
  MM_CHECK_ARG((gh == nullptr) == (g1r == nullptr), "g1r and gh must both be given (gradient mode) or both be null");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_readout1_kernel, dim3((n + 3) / 4), dim3(256), 0, stream, n, h1, h_stride, w0, scale, eat,
                     g1r, g1_stride, gh, gh_stride, D);
  return mm::launch_status("mm_readout1");
}

// R2(h2) = sum_j w2_j silu_n(h2 . W1[:, j]) with W1 = r1_w1 / sqrt(C), w2 = r1_w2 / sqrt(16), silu_n = cst silu;
// eat[i] += scale R2_i;  g_h2[i] = scale dR2/dh2.
// Four lanes per node (hidden width H <= MM_RO2_HMAX): lane q of a node's group takes the features 4 (q + 4 j) .. + 3,
// j = 0..7, so the group reads and writes 64 contiguous bytes per access and a lane issues its 8 loads together.
// W1 is staged in LDS with row stride H + 1 (the 4 lanes of a group read 4 different banks).  The partial
// pre-activations are summed over the group with two xor-shuffles, which leaves the same sum in all four lanes.
#define MM_RO2_HMAX 32
#define MM_RO2_NODES 64   // nodes per 256-thread workgroup
__global__ void __launch_bounds__(256) mm_readout2_kernel(int n, const float* __restrict__ h2, long h_stride,
                                                          const float* __restrict__ W1, const float* __restrict__ w2,
                                                          int H, float cst, float scale, double* __restrict__ eat,
                                                          float* __restrict__ gh, long gh_stride) {
  __shared__ float w1s[MM_C * (MM_RO2_HMAX + 1)];
  const int ws = H + 1;
  for (int t = threadIdx.x; t < MM_C * H; t += 256) w1s[(t / H) * ws + t % H] = W1[t];
  __syncthreads();
  const int node = blockIdx.x * MM_RO2_NODES + (threadIdx.x >> 2);
  if (node >= n) return;   // the four lanes of a group share the node, so no shuffle partner is missing
  const int q = threadIdx.x & 3;
  const floatx4* __restrict__ hp = (const floatx4*)(h2 + (size_t)node * h_stride);
  floatx4 a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = hp[q + 4 * j];
  float z[MM_RO2_HMAX];
#pragma unroll
  for (int j = 0; j < MM_RO2_HMAX; ++j) z[j] = 0.f;
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const float* __restrict__ wr = w1s + 4 * (q + 4 * jj) * ws;
#pragma unroll
    for (int j = 0; j < MM_RO2_HMAX; ++j) {
      if (j < H) {
        z[j] = fmaf(a[jj].x, wr[j], z[j]);
        z[j] = fmaf(a[jj].y, wr[ws + j], z[j]);
        z[j] = fmaf(a[jj].z, wr[2 * ws + j], z[j]);
        z[j] = fmaf(a[jj].w, wr[3 * ws + j], z[j]);
      }
    }
  }
  float e = 0.f;
#pragma unroll
  for (int j = 0; j < MM_RO2_HMAX; ++j) {
    if (j < H) {
      z[j] += __shfl_xor(z[j], 1);
      z[j] += __shfl_xor(z[j], 2);
      const float sg = 1.f / (1.f + expf(-z[j]));
      e += w2[j] * cst * z[j] * sg;
      z[j] = scale * w2[j] * cst * sg * (1.f + z[j] * (1.f - sg));   // scale * d/dz (w2_j cst silu(z))
    }
  }
  if (q == 0) eat[node] += (double)(scale * e);
  floatx4* __restrict__ op = (floatx4*)(gh + (size_t)node * gh_stride);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const float* __restrict__ wr = w1s + 4 * (q + 4 * jj) * ws;
    floatx4 g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MM_RO2_HMAX; ++j) {
      if (j < H) {
        g.x = fmaf(z[j], wr[j], g.x);
        g.y = fmaf(z[j], wr[ws + j], g.y);
        g.z = fmaf(z[j], wr[2 * ws + j], g.z);
        g.w = fmaf(z[j], wr[3 * ws + j], g.w);
      }
    }
    op[q + 4 * jj] = g;
  }
}

extern "C" int mm_readout2(int n, const float* h2, long h_stride, const float* W1, const float* w2, int H,
                           float cst, float scale, double* eat, float* gh, long gh_stride, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0 && H >= 1 && H <= MM_RO2_HMAX, "bad sizes (1 <= H <= 32)");
  MM_CHECK_ARG(h_stride % 4 == 0 && gh_stride % 4 == 0, "row strides must be multiples of 4 floats");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_readout2_kernel, dim3((n + MM_RO2_NODES - 1) / MM_RO2_NODES), dim3(256), 0, stream, n, h2,
                     h_stride, W1, w2, H, cst, scale, eat, gh, gh_stride);
  return mm::launch_status("mm_readout2");
}

// ------------------------------------------------------------------------------------------------ ghost exchange
// Periodic images stand in for LAMMPS' ghost atoms on one GPU: ghost g (row nlocal + g) is a copy of owner[g].
// forward: dst[0:nlocal] = src[0:nlocal]; dst[nlocal + g] = src[owner[g]]     (data.forward_exchange)
// reverse: dst[o] = src[o] + sum_{ghosts g of o} src[nlocal + g]               (data.reverse_exchange)
// The reverse sum walks an owner-sorted CSR of the ghosts (deterministic, no atomics).
__global__ void mm_ghost_forward_kernel(const float* __restrict__ src, float* __restrict__ dst, int D, int nlocal,
                                        int nghost, const int* __restrict__ owner) {
  const long row = blockIdx.y * (long)gridDim.x + blockIdx.x;
  if (row >= (long)nlocal + nghost) return;
  const long from = row < nlocal ? row : (long)owner[row - nlocal];
  for (int j = threadIdx.x; j < D; j += blockDim.x) dst[row * D + j] = src[from * D + j];
}

__global__ void mm_ghost_reverse_kernel(const float* __restrict__ src, float* __restrict__ dst, int D, int nlocal,
                                        const int* __restrict__ g_rowptr, const int* __restrict__ g_list) {
  const long row = blockIdx.y * (long)gridDim.x + blockIdx.x;
  if (row >= nlocal) return;
  const int b = g_rowptr[row], e = g_rowptr[row + 1];
  for (int j = threadIdx.x; j < D; j += blockDim.x) {
    float s = src[row * D + j];
    for (int k = b; k < e; ++k) s += src[((long)nlocal + g_list[k]) * D + j];
    dst[row * D + j] = s;
  }
}

static dim3 rows_grid(long rows) {
  const long gx = rows < 65535 ? (rows > 0 ? rows : 1) : 65535;
  return dim3((unsigned)gx, (unsigned)((rows + gx - 1) / gx));
}

extern "C" int mm_ghost_forward(const float* src, float* dst, int D, int nlocal, int nghost, const int* owner,
                                hipStream_t stream) {
  MM_CHECK_ARG(D >= 1 && nlocal >= 0 && nghost >= 0, "bad sizes");
  if (nlocal + nghost == 0) return MM_OK;
  hipLaunchKernelGGL(mm_ghost_forward_kernel, rows_grid((long)nlocal + nghost), dim3(128), 0, stream, src, dst, D,
                     nlocal, nghost, owner);
  return mm::launch_status("mm_ghost_forward");
}

extern "C" int mm_ghost_reverse(const float* src, float* dst, int D, int nlocal, const int* g_rowptr,
                                const int* g_list, hipStream_t stream) {
  MM_CHECK_ARG(D >= 1 && nlocal >= 0, "bad sizes");
  if (nlocal == 0) return MM_OK;
  hipLaunchKernelGGL(mm_ghost_reverse_kernel, rows_grid(nlocal), dim3(128), 0, stream, src, dst, D, nlocal, g_rowptr,
                     g_list);
  return mm::launch_status("mm_ghost_reverse");
}

// ------------------------------------------------------------------------------------------------ row gather
// dst[r][0:D] = sum over j in [rowptr[r], rowptr[r + 1]) of src[idx[j]][0:D], summed in ascending j by one thread
// per column (a fixed order: the deterministic reduction of the per-edge dL/dX rows of mm_conv2_bwd_det per
// sender).  Rows with an empty range are set to 0.  One 64-lane wave per row, float4 columns (D % 4 == 0).
__global__ void mm_gather_rows_csr_kernel(const int* __restrict__ rowptr, const int* __restrict__ idx,
                                          const float* __restrict__ src, long src_stride, int D,
                                          float* __restrict__ dst, long dst_stride, int n_rows) {
  const long r = (blockIdx.y * (long)gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const int b = rowptr[r], e = rowptr[r + 1];
  for (int c = 4 * lane; c < D; c += 256) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int j = b; j < e; ++j) acc += *(const floatx4*)(src + (long)idx[j] * src_stride + c);
    *(floatx4*)(dst + r * dst_stride + c) = acc;
  }
}

extern "C" int mm_gather_rows_csr(const int* rowptr, const int* idx, const float* src, long src_stride, int D,
                                  float* dst, long dst_stride, int n_rows, hipStream_t stream) {
  MM_CHECK_ARG(n_rows >= 0 && D >= 4 && D % 4 == 0 && src_stride % 4 == 0 && dst_stride % 4 == 0 &&
                   src_stride >= D && dst_stride >= D, "bad sizes (D, strides: multiples of 4, strides >= D)");
  if (n_rows == 0) return MM_OK;
  hipLaunchKernelGGL(mm_gather_rows_csr_kernel, rows_grid(((long)n_rows + 3) / 4), dim3(256), 0, stream, rowptr, idx,
                     src, src_stride, D, dst, dst_stride, n_rows);
  return mm::launch_status("mm_gather_rows_csr");
}

// ------------------------------------------------------------------------------------------------ forces
// F[i] = - sum_{e in row(i)} PF_e + sum_{e : send(e) = i} PF_e with v_e = x_recv - x_send (the reference's
// _accum_forces, receiver_chunk_mace.py:272-276).  Receiver part: CSR over the receiver-sorted pairs; sender
// part: CSR over the pairs sorted by sender (s_perm lists pair ids per sender).  fp64 accumulation.
// One wave per atom: the lanes stride over the atom's pairs as receiver (-PF) and as sender (+PF, through the
// sender CSR), fp64 sums per lane, then a fixed xor butterfly over the wave (repeated runs give identical sums).
__global__ void __launch_bounds__(256) mm_pair_forces_to_atoms_kernel(int n, const long* __restrict__ rowptr,
                                                                      const long* __restrict__ s_rowptr,
                                                                      const long* __restrict__ s_perm,
                                                                      const float* __restrict__ pf,
                                                                      double* __restrict__ F) {
  const long i = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (i >= n) return;
  const int lane = threadIdx.x & 63;
  double fx = 0, fy = 0, fz = 0;
  const long r1 = rowptr[i + 1];
  for (long e = rowptr[i] + lane; e < r1; e += 64) {
    fx -= pf[3 * e];
    fy -= pf[3 * e + 1];
    fz -= pf[3 * e + 2];
  }
  const long s1 = s_rowptr[i + 1];
  for (long k = s_rowptr[i] + lane; k < s1; k += 64) {
    const long e = s_perm[k];
    fx += pf[3 * e];
    fy += pf[3 * e + 1];
    fz += pf[3 * e + 2];
  }
  for (int o = 32; o >= 1; o >>= 1) {
    fx += __shfl_xor(fx, o);
    fy += __shfl_xor(fy, o);
    fz += __shfl_xor(fz, o);
  }
  if (lane == 0) {
    F[3 * i] = fx;
    F[3 * i + 1] = fy;
    F[3 * i + 2] = fz;
  }
}

extern "C" int mm_pair_forces_to_atoms(int n, const long* rowptr, const long* s_rowptr, const long* s_perm,
                                       const float* pf, double* F, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0, "bad sizes");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_pair_forces_to_atoms_kernel, dim3((unsigned)((n + 3L) / 4)), dim3(256), 0, stream, n,
                     rowptr, s_rowptr, s_perm, pf, F);
  return mm::launch_status("mm_pair_forces_to_atoms");
}

// Per-chunk force accumulation of the low-memory evaluator (the reference's ReceiverChunkMACE._accum_forces,
// receiver_chunk_mace.py:272-276, which index_adds each chunk's edge gradients into F): for every node n of the
// chunk, F[nodes[n]] += -(sum of PF over the edges received by n, when n < nC is a receiver) + (sum of PF over the
// edges sent by n, through the chunk's sender CSR).  Only this chunk's pair forces (pf [nE, 3], chunk-local edge
// order) are read, so no pair-force array of the whole system is kept.  One wave per node, the lanes striding
// over its edges, fp64 sums and a fixed xor butterfly: the result does not depend on scheduling, and chunks are
// added in the order the host launches them.
__global__ void __launch_bounds__(256) mm_chunk_forces_kernel(int n_nodes, int nC, const int* __restrict__ rowptr,
                                                              const int* __restrict__ s_rowptr,
                                                              const int* __restrict__ s_perm,
                                                              const int* __restrict__ nodes,
                                                              const float* __restrict__ pf, double* __restrict__ F) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  double fx = 0, fy = 0, fz = 0;
  if (n < nC) {
    const int r1 = rowptr[n + 1];
    for (int e = rowptr[n] + lane; e < r1; e += 64) {
      fx -= pf[3L * e];
      fy -= pf[3L * e + 1];
      fz -= pf[3L * e + 2];
    }
  }
  const int s1 = s_rowptr[n + 1];
  for (int k = s_rowptr[n] + lane; k < s1; k += 64) {
    const long e = s_perm[k];
    fx += pf[3 * e];
    fy += pf[3 * e + 1];
    fz += pf[3 * e + 2];
  }
  for (int o = 32; o >= 1; o >>= 1) {
    fx += __shfl_xor(fx, o);
    fy += __shfl_xor(fy, o);
    fz += __shfl_xor(fz, o);
  }
  if (lane == 0) {
    const long i = nodes[n];
    F[3 * i] += fx;
    F[3 * i + 1] += fy;
    F[3 * i + 2] += fz;
  }
}

extern "C" int mm_chunk_forces(int n_nodes, int nC, const int* rowptr, const int* s_rowptr, const int* s_perm,
                               const int* nodes, const float* pf, double* F, hipStream_t stream) {
  MM_CHECK_ARG(n_nodes >= 0 && nC >= 0 && nC <= n_nodes, "bad sizes (0 <= nC <= n_nodes)");
  if (n_nodes == 0) return MM_OK;
  hipLaunchKernelGGL(mm_chunk_forces_kernel, dim3((unsigned)((n_nodes + 3L) / 4)), dim3(256), 0, stream, n_nodes, nC,
                     rowptr, s_rowptr, s_perm, nodes, pf, F);
  return mm::launch_status("mm_chunk_forces");
}

// Per-atom forces of an MD step from the pair forces of the filtered list, through the skin list (no sort): for
// every skin pair e of atom i that survived the filter (fidx[e] = its index in the filtered list, -1 otherwise),
// F[i] += -PF[fidx[e]] + PF[fidx[rev[e]]], rev[e] = the skin index of the reverse pair (j, i); the neighbour test
// is symmetric, so the reverse pair survives with it.  One wave per atom, fp64 accumulation.
__global__ void __launch_bounds__(256) mm_pair_forces_skin_kernel(long n, const long* __restrict__ skin_rowptr,
                                                                  const int* __restrict__ fidx,
                                                                  const int* __restrict__ rev,
                                                                  const float* __restrict__ pf,
                                                                  double* __restrict__ F) {
  const long i = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (i >= n) return;
  const int lane = threadIdx.x & 63;
  double fx = 0, fy = 0, fz = 0;
  const long e1 = skin_rowptr[i + 1];
  // 4 x 64 skin pairs per step, each level of the chain fidx[e] -> rev[e] -> fidx[rev[e]] -> the two pair forces
  // loaded together.  A lane past the row or on a dropped pair reads the row's first entries and pf row 0 (one
  // shared address, not a random one; pf holds at least one row) and adds 0.0 through a select, so an unwritten
  // pf row 0 (no pair survived the filter) cannot reach the sums, which run in the same order as one pair at a
  // time.
  for (long eb = skin_rowptr[i]; eb < e1; eb += 256) {
    int f[4], r[4];
    bool use[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) f[k] = fidx[min(eb + lane + 64 * k, e1 - 1)];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      use[k] = (eb + lane + 64 * k < e1) & (f[k] >= 0);
      r[k] = rev[use[k] ? eb + lane + 64 * k : eb];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = fidx[r[k]];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const long a = use[k] ? f[k] : 0, b = use[k] ? max(r[k], 0) : 0;   // r >= 0 when f >= 0 (symmetric test)
      const double dx = (double)pf[3 * b] - (double)pf[3 * a];
      const double dy = (double)pf[3 * b + 1] - (double)pf[3 * a + 1];
      const double dz = (double)pf[3 * b + 2] - (double)pf[3 * a + 2];
      fx += use[k] ? dx : 0.0;
      fy += use[k] ? dy : 0.0;
      fz += use[k] ? dz : 0.0;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    fx += __shfl_xor(fx, o);
    fy += __shfl_xor(fy, o);
    fz += __shfl_xor(fz, o);
  }
  if (lane == 0) {
    F[3 * i] = fx;
    F[3 * i + 1] = fy;
    F[3 * i + 2] = fz;
  }
}

extern "C" int mm_pair_forces_skin(long n, const long* skin_rowptr, const int* fidx, const int* rev, const float* pf,
                                   double* F, hipStream_t stream) {
  MM_CHECK_ARG(n >= 0, "bad sizes");
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(mm_pair_forces_skin_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream, n, skin_rowptr,
                     fidx, rev, pf, F);
  return mm::launch_status("mm_pair_forces_skin");
}

// Chunk-local indices of every edge of a receiver-CSR pair list split into receiver chunks [c * chunk, (c + 1) *
// chunk): ls[e] = loc[c * N + send[e]] (the sender's row in chunk c's node list) and recv_local[e] = i - c * chunk
// for the edges e of receiver i.  One wave per receiver.
__global__ void __launch_bounds__(256) mm_chunk_edge_index_kernel(long N, const long* __restrict__ rowptr,
                                                                  const int* __restrict__ send,
                                                                  const int* __restrict__ loc, int chunk,
                                                                  int* __restrict__ ls, int* __restrict__ recv_local) {
  const long i = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (i >= N) return;
  const int lane = threadIdx.x & 63;
  const long c = i / chunk;
  const int* __restrict__ lc = loc + c * N;
  const int rl = (int)(i - c * chunk);
  for (long e = rowptr[i] + lane; e < rowptr[i + 1]; e += 64) {
    ls[e] = lc[send[e]];
    recv_local[e] = rl;
  }
}

extern "C" int mm_chunk_edge_index(long N, const long* rowptr, const int* send, const int* loc, int chunk, int* ls,
                                   int* recv_local, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && chunk >= 1, "bad sizes");
  if (N == 0) return MM_OK;
  hipLaunchKernelGGL(mm_chunk_edge_index_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, N, rowptr, send,
                     loc, chunk, ls, recv_local);
  return mm::launch_status("mm_chunk_edge_index");
}

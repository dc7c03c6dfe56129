// Cell-list neighbour build, bit-exact with the reference's System / build_neighbors
// (receiver_chunk_mace.py:82-165):
//   wrap      : m = fmod(x, L); m + L where the signs of m and L differ (torch.remainder)
//   cell      : min(floor(m / (L / ncell)), ncell - 1), ncell = max(1, floor(L / r_max)) (host)
//   order     : 10-bit Morton code (x -> bit 3b+2, y -> 3b+1, z -> 3b), stable radix sort -> perm
//   candidates: the 27 cells (c + o) mod ncell for o in (-1, 0, 1)^3, x-offset slowest (meshgrid "ij"), each
//               cell's atoms in sorted order; all atoms 0..N-1 in order if any ncell < 3
//   test      : d = v - L * rint(v / L) (half to even, as torch.round), dd = (dx^2 + dy^2) + dz^2, keep
//               dd < r_max^2 and j != i; candidate order preserved.
// Every fp64 operation is a separately rounded IEEE operation: the file is compiled with -ffp-contract=off and
// the arithmetic scopes carry "#pragma clang fp contract(off)" (HIP's __dmul_rn / __dadd_rn are plain * and +,
// which clang would otherwise fuse into FMAs and so change dd at the last bit).  Output: CSR (rowptr int64 [N+1], senders int32 [E]) in the sorted index space.
#include "common.h"

#include <hipcub/hipcub.hpp>

#include <mutex>
#include <string>

__global__ void mm_nl_prepare_kernel(const double* __restrict__ pos_in, long N, double bx, double by, double bz,
                                     double cx, double cy, double cz, int nx, int ny, int nz,
                                     double* __restrict__ pos_w, int* __restrict__ cell,
                                     long long* __restrict__ key, long long* __restrict__ idx) {
#pragma clang fp contract(off)
  const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (i >= N) return;
  const double L[3] = {bx, by, bz};
  const double cs[3] = {cx, cy, cz};
  const int nc[3] = {nx, ny, nz};
  int c[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    double m = fmod(pos_in[3 * i + k], L[k]);
    if (m != 0.0 && ((m < 0.0) != (L[k] < 0.0))) m = __dadd_rn(m, L[k]);
    pos_w[3 * i + k] = m;
    long q = (long)floor(__ddiv_rn(m, cs[k]));
    if (q > nc[k] - 1) q = nc[k] - 1;
    c[k] = (int)q;
    cell[3 * i + k] = c[k];
  }
  long long code = 0;
#pragma unroll
  for (int b = 0; b < 10; ++b) {
    code |= ((long long)((c[0] >> b) & 1)) << (3 * b + 2);
    code |= ((long long)((c[1] >> b) & 1)) << (3 * b + 1);
    code |= ((long long)((c[2] >> b) & 1)) << (3 * b);
  }
  key[i] = code;
  idx[i] = i;
}

__global__ void mm_nl_gather_kernel(const long long* __restrict__ perm, long N, const double* __restrict__ pos_w,
                                    const int* __restrict__ cell, const int* __restrict__ spec_in,
                                    double* __restrict__ pos_s, int* __restrict__ cell_s, int* __restrict__ spec_s) {
  const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (i >= N) return;
  const long j = perm[i];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    pos_s[3 * i + k] = pos_w[3 * j + k];
    cell_s[3 * i + k] = cell[3 * j + k];
  }
  if (spec_in) spec_s[i] = spec_in[j];
}

// start[cl] = first sorted atom of cell cl (N if empty), count[cl]; atoms of a cell are contiguous after the sort
__global__ void mm_nl_ranges_kernel(const int* __restrict__ cell_s, long N, int ny, int nz, int* __restrict__ start,
                                    int* __restrict__ count) {
  const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int cl = (cell_s[3 * i] * ny + cell_s[3 * i + 1]) * nz + cell_s[3 * i + 2];
  const int prev = i > 0 ? (cell_s[3 * (i - 1)] * ny + cell_s[3 * (i - 1) + 1]) * nz + cell_s[3 * (i - 1) + 2] : -1;
  const int next = i + 1 < N ? (cell_s[3 * (i + 1)] * ny + cell_s[3 * (i + 1) + 1]) * nz + cell_s[3 * (i + 1) + 2]
                             : -1;
  if (cl != prev) start[cl] = (int)i;
  if (cl != next) count[cl] = (int)(i + 1);   // end, turned into a count below
}

__global__ void mm_nl_counts_kernel(int ncells, const int* __restrict__ start, int* __restrict__ count, long N) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncells) return;
  count[c] = start[c] < N ? count[c] - start[c] : 0;
}

__global__ void mm_fill_i32_kernel_nl(int* __restrict__ p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__device__ __forceinline__ double mm_mic(double v, double L) {
#pragma clang fp contract(off)
  return __dsub_rn(v, __dmul_rn(L, rint(__ddiv_rn(v, L))));
}

template <bool FILL>
__global__ void mm_nl_pairs_kernel(const double* __restrict__ pos, const int* __restrict__ cell, long N, double bx,
                                   double by, double bz, int nx, int ny, int nz, const int* __restrict__ start,
                                   const int* __restrict__ count, double r2, int brute, int* __restrict__ NN,
                                   const long* __restrict__ rowptr, int* __restrict__ send) {
  const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (i >= N) return;
  const double xi = pos[3 * i], yi = pos[3 * i + 1], zi = pos[3 * i + 2];
  long n = 0;
  const long base = FILL ? rowptr[i] : 0;
  auto test = [&](long j) {
#pragma clang fp contract(off)
    const double dx = mm_mic(__dsub_rn(xi, pos[3 * j]), bx);
    const double dy = mm_mic(__dsub_rn(yi, pos[3 * j + 1]), by);
    const double dz = mm_mic(__dsub_rn(zi, pos[3 * j + 2]), bz);
    const double dd = __dadd_rn(__dadd_rn(__dmul_rn(dx, dx), __dmul_rn(dy, dy)), __dmul_rn(dz, dz));
    if (dd < r2 && j != i) {
      if (FILL) send[base + n] = (int)j;
      ++n;
    }
  };
  if (brute) {
    for (long j = 0; j < N; ++j) test(j);
  } else {
    const int cx = cell[3 * i], cy = cell[3 * i + 1], cz = cell[3 * i + 2];
    for (int ox = -1; ox <= 1; ++ox) {
      const int ax = ((cx + ox) % nx + nx) % nx;
      for (int oy = -1; oy <= 1; ++oy) {
        const int ay = ((cy + oy) % ny + ny) % ny;
        for (int oz = -1; oz <= 1; ++oz) {
          const int az = ((cz + oz) % nz + nz) % nz;
          const int cl = (ax * ny + ay) * nz + az;
          const int st = start[cl], ct = count[cl];
          for (int k = 0; k < ct; ++k) test((long)st + k);
        }
      }
    }
  }
  if (!FILL) NN[i] = (int)n;
}

extern "C" int mm_nl_workspace_bytes(long N, size_t* bytes) {
  MM_CHECK_ARG(N >= 0 && N < (1L << 31) && bytes, "bad sizes");
  size_t a = 0, b = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, a, (const long long*)nullptr, (long long*)nullptr,
                                     (const long long*)nullptr, (long long*)nullptr, (int)N, 0, 30);
  hipcub::DeviceScan::ExclusiveSum(nullptr, b, (const long*)nullptr, (long*)nullptr, (int)N + 1);
  *bytes = (a > b ? a : b) + 256;
  return MM_OK;
}

extern "C" int mm_nl_prepare(const double* pos_in, long N, const double* box, const int* ncell, const double* cs,
                             double* pos_w, int* cell, long long* key, long long* idx, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && box && ncell && cs, "bad arguments");
  for (int k = 0; k < 3; ++k) MM_CHECK_ARG(ncell[k] >= 1 && ncell[k] <= 1024, "ncell out of range (10-bit Morton)");
  if (N == 0) return MM_OK;
  hipLaunchKernelGGL(mm_nl_prepare_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, stream, pos_in, N, box[0],
                     box[1], box[2], cs[0], cs[1], cs[2], ncell[0], ncell[1], ncell[2], pos_w, cell, key, idx);
  return mm::launch_status("mm_nl_prepare");
}

extern "C" int mm_nl_sort(const long long* key_in, long long* key_out, const long long* idx_in, long long* perm,
                          long N, void* ws, size_t ws_bytes, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && N < (1L << 31), "bad sizes");
  if (N == 0) return MM_OK;
  size_t need = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, need, key_in, key_out, idx_in, perm, (int)N, 0, 30, stream);
  MM_CHECK_ARG(ws_bytes >= need, "workspace too small");
  if (hipcub::DeviceRadixSort::SortPairs(ws, need, key_in, key_out, idx_in, perm, (int)N, 0, 30, stream) !=
      hipSuccess)
    return mm::launch_status("mm_nl_sort");
  return mm::launch_status("mm_nl_sort");
}

extern "C" int mm_nl_gather(const long long* perm, long N, const double* pos_w, const int* cell, const int* spec_in,
                            double* pos_s, int* cell_s, int* spec_s, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0, "bad sizes");
  if (N == 0) return MM_OK;
  hipLaunchKernelGGL(mm_nl_gather_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, stream, perm, N, pos_w, cell,
                     spec_in, pos_s, cell_s, spec_s);
  return mm::launch_status("mm_nl_gather");
}

extern "C" int mm_nl_cell_ranges(const int* cell_s, long N, const int* ncell, int* start, int* count,
                                 hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && ncell, "bad arguments");
  const int ncells = ncell[0] * ncell[1] * ncell[2];
  hipLaunchKernelGGL(mm_fill_i32_kernel_nl, dim3((ncells + 255) / 256), dim3(256), 0, stream, start, ncells, (int)N);
  hipLaunchKernelGGL(mm_fill_i32_kernel_nl, dim3((ncells + 255) / 256), dim3(256), 0, stream, count, ncells, 0);
  if (N > 0)
    hipLaunchKernelGGL(mm_nl_ranges_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, stream, cell_s, N,
                       ncell[1], ncell[2], start, count);
  hipLaunchKernelGGL(mm_nl_counts_kernel, dim3((ncells + 255) / 256), dim3(256), 0, stream, ncells, start, count, N);
  return mm::launch_status("mm_nl_cell_ranges");
}

extern "C" int mm_nl_count(const double* pos_s, const int* cell_s, long N, const double* box, const int* ncell,
                           const int* start, const int* count, double r2, int brute, int* NN, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && box && ncell, "bad arguments");
  if (N == 0) return MM_OK;
  hipLaunchKernelGGL(mm_nl_pairs_kernel<false>, dim3((unsigned)((N + 127) / 128)), dim3(128), 0, stream, pos_s,
                     cell_s, N, box[0], box[1], box[2], ncell[0], ncell[1], ncell[2], start, count, r2, brute, NN,
                     (const long*)nullptr, (int*)nullptr);
  return mm::launch_status("mm_nl_count");
}

extern "C" int mm_nl_scan(const int* NN, long* rowptr, long N, void* ws, size_t ws_bytes, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && N < (1L << 31), "bad sizes");
  // rowptr[0] = 0, rowptr[i + 1] = sum_{j <= i} NN[j]: exclusive scan of NN widened to int64, over N + 1 items
  // (the last input item is a zero appended by the widening iterator)
  struct Widen {
    const int* p;
    long n;
    __host__ __device__ long operator()(const long& i) const { return i < n ? (long)p[i] : 0L; }
  };
  hipcub::CountingInputIterator<long> cnt(0);
  hipcub::TransformInputIterator<long, Widen, hipcub::CountingInputIterator<long>> it(cnt, Widen{NN, N});
  size_t need = 0;
  hipcub::DeviceScan::ExclusiveSum(nullptr, need, it, rowptr, (int)N + 1, stream);
  MM_CHECK_ARG(ws_bytes >= need, "workspace too small");
  hipcub::DeviceScan::ExclusiveSum(ws, need, it, rowptr, (int)N + 1, stream);
  return mm::launch_status("mm_nl_scan");
}

// ------------------------------------------------------------------------------------------------------------
// Allocation-free receiver-CSR scan (no counterpart in the reference).  mm_nl_scan_noalloc gives the result of
// mm_nl_scan (rowptr[0] = 0, rowptr[i + 1] = sum_{j <= i} NN[j], int64) without a workspace argument, for callers
// that cannot allocate one (code under HIP-graph capture, serving loops).  Its tile partials live in `scratch`, a
// file-scope device array that every GPU the library runs on holds until the process ends:
//   * N + 1 <= MM_SCAN_MAX_TILES * MM_SCAN_TILE = 134,217,728 counts (larger N is rejected with MM_ERANGE);
//   * the array's device address is looked up once per device (hipGetSymbolAddress, first call on that device);
//   * every partial is written before it is read within one call, so nothing needs clearing between calls;
//   * calls that overlap on one GPU (different streams) share the array and race.
// Three kernels: per-tile sums -> one block scans the tile sums in place -> per-tile scan plus its offset.
#define MM_SCAN_THREADS 256
#define MM_SCAN_ITEMS 16
#define MM_SCAN_TILE (MM_SCAN_THREADS * MM_SCAN_ITEMS)
#define MM_SCAN_MAX_TILES 32768
#define MM_SCAN_OFFSET_THREADS 1024

static __device__ __align__(256) long long scratch[MM_SCAN_MAX_TILES];

// item i of the scan: NN[i] for i < N, 0 for i = N (the appended zero that makes rowptr[N] the total)
__device__ __forceinline__ long long mm_scan_item(const int* __restrict__ NN, long N, long i) {
  return i < N ? (long long)NN[i] : 0LL;
}

// In-place inclusive scan of v[0..n) (n = blockDim.x threads, one value each) in LDS; returns the inclusive value
// of this thread.
__device__ __forceinline__ long long mm_block_inclusive_scan(long long x, long long* lds) {
  const int t = threadIdx.x;
  lds[t] = x;
  __syncthreads();
  for (int d = 1; d < (int)blockDim.x; d <<= 1) {
    const long long y = t >= d ? lds[t - d] : 0LL;
    __syncthreads();
    lds[t] += y;
    __syncthreads();
  }
  return lds[t];
}

__global__ void __launch_bounds__(MM_SCAN_THREADS) mm_scan_tile_sums_kernel(const int* __restrict__ NN, long N,
                                                                             long long* __restrict__ part) {
  __shared__ long long lds[MM_SCAN_THREADS];
  const long base = (long)blockIdx.x * MM_SCAN_TILE + (long)threadIdx.x * MM_SCAN_ITEMS;
  long long s = 0;
#pragma unroll
  for (int k = 0; k < MM_SCAN_ITEMS; ++k) s += mm_scan_item(NN, N, base + k);
  const long long tot = mm_block_inclusive_scan(s, lds);
  if (threadIdx.x == MM_SCAN_THREADS - 1) part[blockIdx.x] = tot;
}

// One block: part[0..tiles) <- exclusive prefix sums of the tile sums.
__global__ void __launch_bounds__(MM_SCAN_OFFSET_THREADS) mm_scan_tile_offsets_kernel(long long* __restrict__ part,
                                                                                        int tiles) {
  __shared__ long long lds[MM_SCAN_OFFSET_THREADS];
  const int per = (tiles + MM_SCAN_OFFSET_THREADS - 1) / MM_SCAN_OFFSET_THREADS;
  const int lo = threadIdx.x * per;
  const int hi = min(lo + per, tiles);
  long long s = 0;
  for (int i = lo; i < hi; ++i) s += part[i];
  long long run = mm_block_inclusive_scan(s, lds) - s;     // exclusive prefix of this thread's run
  for (int i = lo; i < hi; ++i) {
    const long long v = part[i];
    part[i] = run;
    run += v;
  }
}

__global__ void __launch_bounds__(MM_SCAN_THREADS) mm_scan_tile_apply_kernel(const int* __restrict__ NN, long N,
                                                                              const long long* __restrict__ part,
                                                                              long* __restrict__ rowptr) {
  __shared__ long long lds[MM_SCAN_THREADS];
  const long base = (long)blockIdx.x * MM_SCAN_TILE + (long)threadIdx.x * MM_SCAN_ITEMS;
  long long v[MM_SCAN_ITEMS];
  long long s = 0;
#pragma unroll
  for (int k = 0; k < MM_SCAN_ITEMS; ++k) {
    v[k] = mm_scan_item(NN, N, base + k);
    s += v[k];
  }
  long long run = mm_block_inclusive_scan(s, lds) - s + part[blockIdx.x];
#pragma unroll
  for (int k = 0; k < MM_SCAN_ITEMS; ++k) {
    if (base + k <= N) rowptr[base + k] = (long)run;
    run += v[k];
  }
}

namespace {
std::mutex g_scratch_mu;
long long* g_scratch_ptr[64] = {};     // device address of `scratch` per device ordinal

int scan_scratch(long long** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    mm::set_error("mm_nl_scan_noalloc: no current HIP device");
    return MM_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      mm::set_error(std::string("mm_nl_scan_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return MM_ELAUNCH;
    }
    g_scratch_ptr[dev] = (long long*)p;
  }
  *out = g_scratch_ptr[dev];
  return MM_OK;
}
}  // namespace

extern "C" int mm_nl_scan_noalloc(const int* NN, long* rowptr, long N, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && rowptr && (N == 0 || NN), "bad arguments");
  const long tiles = (N + 1 + MM_SCAN_TILE - 1) / MM_SCAN_TILE;
  if (tiles > MM_SCAN_MAX_TILES) {
    mm::set_error("mm_nl_scan_noalloc: N = " + std::to_string(N) + " exceeds the scratch limit N + 1 <= " +
                  std::to_string((long)MM_SCAN_MAX_TILES * MM_SCAN_TILE) + " (use mm_nl_scan with a workspace)");
    return MM_ERANGE;
  }
  long long* part = nullptr;
  const int rc = scan_scratch(&part);
  if (rc != MM_OK) return rc;
  hipLaunchKernelGGL(mm_scan_tile_sums_kernel, dim3((unsigned)tiles), dim3(MM_SCAN_THREADS), 0, stream, NN, N,
                     part);
  hipLaunchKernelGGL(mm_scan_tile_offsets_kernel, dim3(1), dim3(MM_SCAN_OFFSET_THREADS), 0, stream, part,
                     (int)tiles);
  hipLaunchKernelGGL(mm_scan_tile_apply_kernel, dim3((unsigned)tiles), dim3(MM_SCAN_THREADS), 0, stream, NN, N,
                     (const long long*)part, rowptr);
  return mm::launch_status("mm_nl_scan_noalloc");
}

extern "C" int mm_nl_fill(const double* pos_s, const int* cell_s, long N, const double* box, const int* ncell,
                          const int* start, const int* count, double r2, int brute, const long* rowptr, int* send,
                          hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && box && ncell, "bad arguments");
  if (N == 0) return MM_OK;
  hipLaunchKernelGGL(mm_nl_pairs_kernel<true>, dim3((unsigned)((N + 127) / 128)), dim3(128), 0, stream, pos_s,
                     cell_s, N, box[0], box[1], box[2], ncell[0], ncell[1], ncell[2], start, count, r2, brute,
                     (int*)nullptr, rowptr, send);
  return mm::launch_status("mm_nl_fill");
}

// Per-step pair list of an MD run: the pairs of a skin list (built with r_cut = r_max + skin) whose current
// minimum-image distance is below r_max, in the skin list's order (the same test as mm_nl_pairs_kernel).
// One wave per receiver: 256 candidates per step, kept ones compacted in order with ballots and prefix popcounts.
// FILL = false: NN[i] = number of skin pairs of atom i within r_max; with flags != nullptr also flags[e] = 0 (kept)
// or -1 per skin pair.  FILL = true: the kept pairs in candidate order, send[rowptr[i] + k], and fidx[e] = the
// filtered index of skin pair e or -1; with FROM_FLAGS the keep decisions are read from fidx (the count pass's
// flags, written in place) instead of recomputed from the positions.
template <bool FILL, bool FROM_FLAGS>
__global__ void __launch_bounds__(256) mm_nl_filter_kernel(const double* __restrict__ pos, long N, double bx,
                                                           double by, double bz, const long* __restrict__ rp_s,
                                                           const int* __restrict__ send_s, double r2,
                                                           int* __restrict__ NN, const long* __restrict__ rowptr,
                                                           int* __restrict__ send, int* __restrict__ fidx) {
  const long i = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (i >= N) return;
  const int lane = threadIdx.x & 63;
  double xi = 0, yi = 0, zi = 0;
  if (!FROM_FLAGS) {
    xi = pos[3 * i];
    yi = pos[3 * i + 1];
    zi = pos[3 * i + 2];
  }
  const long end = rp_s[i + 1];
  long n = 0;
  const long base = FILL ? rowptr[i] : 0;
  // 4 x 64 candidates per step: their loads are issued together (a lane past the row reads the row's last
  // candidate and keeps nothing), then the kept ones are compacted in candidate order, 64 at a time
  for (long e0 = rp_s[i]; e0 < end; e0 += 256) {
    int j[4];
    bool keep[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) j[k] = send_s[min(e0 + lane + 64 * k, end - 1)];
    if (FROM_FLAGS) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int flag = fidx[min(e0 + lane + 64 * k, end - 1)];
        keep[k] = (e0 + lane + 64 * k < end) & (flag >= 0);
      }
    } else {
      double px[4], py[4], pz[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        px[k] = pos[3 * (long)j[k]];
        py[k] = pos[3 * (long)j[k] + 1];
        pz[k] = pos[3 * (long)j[k] + 2];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma clang fp contract(off)
        const double dx = mm_mic(xi - px[k], bx);
        const double dy = mm_mic(yi - py[k], by);
        const double dz = mm_mic(zi - pz[k], bz);
        const double dd = (dx * dx + dy * dy) + dz * dz;
        keep[k] = (e0 + lane + 64 * k < end) & (dd < r2) & (j[k] != i);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const long e = e0 + lane + 64 * k;
      const unsigned long long m = __ballot(keep[k]);
      if (FILL) {
        const long slot = base + n + __popcll(m & ((1ull << lane) - 1ull));
        if (keep[k]) send[slot] = j[k];
        if (fidx && e < end) fidx[e] = keep[k] ? (int)slot : -1;
      } else if (fidx && e < end) {
        fidx[e] = keep[k] ? 0 : -1;
      }
      n += __popcll(m);
    }
  }
  if (!FILL && lane == 0) NN[i] = (int)n;
}

extern "C" int mm_nl_filter_count(const double* pos, long N, const double* box, const long* rp_s, const int* send_s,
                                  double r2, int* NN, int* flags, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && box, "bad arguments");
  if (N == 0) return MM_OK;
  hipLaunchKernelGGL((mm_nl_filter_kernel<false, false>), dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, pos,
                     N, box[0], box[1], box[2], rp_s, send_s, r2, NN, (const long*)nullptr, (int*)nullptr, flags);
  return mm::launch_status("mm_nl_filter_count");
}

extern "C" int mm_nl_filter_fill(const double* pos, long N, const double* box, const long* rp_s, const int* send_s,
                                 double r2, const long* rowptr, int* send, int* fidx, int from_flags,
                                 hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && box, "bad arguments");
  MM_CHECK_ARG(!from_flags || fidx, "from_flags needs the count pass's flags in filtered_index");
  if (N == 0) return MM_OK;
  if (from_flags)
    hipLaunchKernelGGL((mm_nl_filter_kernel<true, true>), dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, pos,
                       N, box[0], box[1], box[2], rp_s, send_s, r2, (int*)nullptr, rowptr, send, fidx);
  else
    hipLaunchKernelGGL((mm_nl_filter_kernel<true, false>), dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, pos,
                       N, box[0], box[1], box[2], rp_s, send_s, r2, (int*)nullptr, rowptr, send, fidx);
  return mm::launch_status("mm_nl_filter_fill");
}

// rev[e] = index of the pair (j, i) for every pair e = (i, j) of a symmetric CSR pair list (the MD driver's skin
// list), found by scanning row j; no sort and no memory beyond rev.  One wave per receiver i: the senders of 64 of
// its pairs and the bounds of their rows are loaded together, then each 16-lane quarter of the wave searches one
// pair's row, 256 candidates per round (16 loads per lane in flight).  Every sender occurs at most once in a row
// (one minimum image), so at most one lane writes each rev[e]; a pair without a reverse keeps the caller's fill.
__global__ void __launch_bounds__(256) mm_nl_reverse_kernel(long N, const long* __restrict__ rowptr,
                                                            const int* __restrict__ send, int* __restrict__ rev) {
  const long i = blockIdx.x * 4L + (threadIdx.x >> 6);
  if (i >= N) return;
  const int lane = threadIdx.x & 63, q = lane >> 4, lq = lane & 15;
  const long b0 = rowptr[i], b1 = rowptr[i + 1];
  for (long eb = b0; eb < b1; eb += 64) {
    // lanes past the row hold an empty range [0, 0)
    int s0 = 0, len = 0;
    if (eb + lane < b1) {
      const int j = send[eb + lane];
      s0 = (int)rowptr[j];
      len = (int)(rowptr[j + 1] - s0);
    }
    const int n = (int)min(64L, b1 - eb);
    for (int k = 0; k < n; k += 4) {
      const int src = k + q;                       // the pair this quarter searches: eb + src
      const int c0 = __shfl(s0, src), cl = __shfl(len, src);
      for (int c = 0; c < cl; c += 256) {
        int v[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const int x = c + 16 * t + lq;
          v[t] = x < cl ? send[c0 + x] : -1;
        }
#pragma unroll
        for (int t = 0; t < 16; ++t)
          if (v[t] == (int)i) rev[eb + src] = c0 + c + 16 * t + lq;
      }
    }
  }
}

extern "C" int mm_nl_reverse(const long* rowptr, const int* send, long N, long E, int* rev, hipStream_t stream) {
  MM_CHECK_ARG(N >= 0 && E >= 0 && (N == 0 || (rowptr && send && rev)), "bad arguments");
  if (E > 2147483647L) {
    mm::set_error("mm_nl_reverse: " + std::to_string(E) + " pairs exceed the int32 pair index");
    return MM_ERANGE;
  }
  if (N == 0 || E == 0) return MM_OK;
  hipLaunchKernelGGL(mm_nl_reverse_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, N, rowptr, send, rev);
  return mm::launch_status("mm_nl_reverse");
}

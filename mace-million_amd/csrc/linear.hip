// Equivariant linear maps of the node features on the fp32 matrix cores (v_mfma_f32_16x16x4f32).
//
// Every node-level linear of the two layers is a set of 128x128 channel-mixing blocks applied to 128-channel rows
// of ir_mul features (one row per (node, component)): linear_up, linear (with the density division), skip_tp per
// species (fast_layers.SpeciesSkip, fast_layers.py:41-105 -- here the species rows are gathered by per-species
// row lists instead of computing every species and selecting), the product-block linear, and their transposes in
// the backward passes.  For each output component j of one launch:
//     out[out_row(r), comp_j] (= or +=) scale(r) * sum_q in[in_row(r), src_{j,q}] @ W[w_{j,q}]
// Launch: grid (ceil(rows / (128 n_blk)), n_comp, n_groups); 512 threads = 8 waves, each wave 16 rows x 128
// columns (8 MFMA tiles) of each of its n_blk row blocks; the 128x128 weight block is staged in LDS (64 KiB) in the
// lane order of the B operand.
// Weight blocks are stored pre-permuted: element W[k][n], k = 16 t + 4 g + u, n = 16 nt + i, at float index
// (((t * 8 + nt) * 4 + g) * 16 + i) * 4 + u, so that lane (i, g) reads its 4 k-values of step t and tile nt as one
// 16-byte LDS read, the 16 lanes of a group reading 256 consecutive bytes (no bank conflicts), and the A operand of
// lane (row, g) is the float4 in[row][16 t + 4 g .. + 3].
#include "common.h"

#include <algorithm>

#define MM_LIN_MAX_COMP 48
#define MM_LIN_MAX_SRC 3
// 8 waves of one 16-row M-tile each: 128 rows per workgroup block.  With the 64 KiB weight block in LDS two
// workgroups share a CU, i.e. 4 waves per SIMD (measured faster than 4 waves of two M-tiles, 2 waves per SIMD).
#define MM_LIN_MT 1
#define MM_LIN_NW 8
#define MM_LIN_BLOCK_ROWS (16 * MM_LIN_MT * MM_LIN_NW)
// a launch keeps at least this many workgroups (8 per CU) when it groups row blocks per workgroup
#define MM_LIN_MIN_WG 2048

struct MMLinComp {
  int n_src;
  int in_off[MM_LIN_MAX_SRC];   // float offset of the source chunk inside an input row
  int w_idx[MM_LIN_MAX_SRC];    // weight block index
  int out_off;                  // float offset of the output chunk inside an output row
};

struct MMLinArgs {
  const float* in;
  long in_stride;
  const int* in_rows;     // nullable: in row of logical row id
  float* out;
  long out_stride;
  const int* out_rows;    // nullable
  const float* W;         // weight blocks, 16384 floats each
  const float* row_scale; // nullable: per logical row id
  int scale_mode;         // 0: scale = row_scale[id]; 1: scale = 1 / (row_scale[id] + 1)
  const int* list;        // nullable: per group g, list[g * list_stride + r] = logical row id
  const int* list_count;  // per group row count (device), with list
  long list_stride;
  int n_rows;             // without list
  int w_group_stride;     // weight block offset of group g (species)
  int accumulate;
  int n_comp;
  MMLinComp comp[MM_LIN_MAX_COMP];
};

template <int MT>
struct MMLinRows {
  bool valid[MT];
  long in_row[MT];
};

template <int MT>
__device__ __forceinline__ void mm_lin_rows(const MMLinArgs& args, const int* list, int nrows, int row0, int wave,
                                            int i, MMLinRows<MT>& rw) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = row0 + (wave * MT + mt) * 16 + i;
    rw.valid[mt] = r < nrows;
    const int rid = rw.valid[mt] ? (list ? list[r] : r) : 0;
    rw.in_row[mt] = args.in_rows ? (long)args.in_rows[rid] : (long)rid;
  }
}

template <int MT>
__device__ __forceinline__ void mm_lin_load_a(const MMLinArgs& args, const MMLinRows<MT>& rw, int in_off, int g,
                                              floatx4 (&a)[MT][8]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const float* __restrict__ ap = args.in + rw.in_row[mt] * args.in_stride + in_off + 4 * g;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      a[mt][t] = rw.valid[mt] ? *(const floatx4*)(ap + 16 * t) : floatx4{0.f, 0.f, 0.f, 0.f};
  }
}

// MT = 16-row M-tiles per wave, NW waves (rows per workgroup block = 16 NW MT): every B operand read from LDS
// feeds MT MFMAs.
// A workgroup handles n_blk consecutive row blocks of one output component; with a single source the weight block
// is staged in LDS once for all of them.  The A operands of the next (block, source) step are loaded while the
// MFMAs of the current one run.
template <int MT, int NW>
__global__ void __launch_bounds__(64 * NW) mm_linear_kernel(MMLinArgs args, int n_blk) {
  __shared__ floatx4 Wl[4096];
  const MMLinComp cp = args.comp[blockIdx.y];
  const int grp = blockIdx.z;
  const int nrows = args.list ? args.list_count[grp] : args.n_rows;
  const int blk_rows = 16 * NW * MT;
  const int blk0 = blockIdx.x * n_blk;
  if (blk0 * blk_rows >= nrows) return;
  const int blk1 = min(blk0 + n_blk, (nrows + blk_rows - 1) / blk_rows);
  const int* __restrict__ list = args.list ? args.list + (size_t)grp * args.list_stride : nullptr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const int n_src = cp.n_src;
  const bool restage = n_src > 1;
  MMLinRows<MT> rw, rw_next;
  mm_lin_rows<MT>(args, list, nrows, blk0 * blk_rows, wave, i, rw);
  floatx4 a[MT][8];
  mm_lin_load_a<MT>(args, rw, cp.in_off[0], g, a);
  for (int blk = blk0; blk < blk1; ++blk) {
    const int row0 = blk * blk_rows;
    floatx4 acc[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) acc[mt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < n_src; ++q) {
      // next step: source q + 1 of this block, else source 0 of the next block
      floatx4 an[MT][8];
      const bool next_here = q + 1 < n_src;
      const bool has_next = next_here || blk + 1 < blk1;
      if (has_next) {
        if (!next_here) mm_lin_rows<MT>(args, list, nrows, row0 + blk_rows, wave, i, rw_next);
        mm_lin_load_a<MT>(args, next_here ? rw : rw_next, cp.in_off[next_here ? q + 1 : 0], g, an);
      }
      if (restage || blk == blk0) {
        const floatx4* __restrict__ Wg =
            (const floatx4*)(args.W + (size_t)(cp.w_idx[q] + grp * args.w_group_stride) * 16384);
        __syncthreads();
        for (int j = threadIdx.x; j < 4096; j += 64 * NW) Wl[j] = Wg[j];
        __syncthreads();
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const floatx4 b = Wl[((t * 8 + nt) * 4 + g) * 16 + i];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][t].x, b.x, acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][t].y, b.y, acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][t].z, b.z, acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][t].w, b.w, acc[mt][nt], 0, 0, 0);
          }
        }
      }
      if (has_next) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < 8; ++t) a[mt][t] = an[mt][t];
      }
    }
    // D layout of the 16x16 tile: lane (i, g) holds rows 4 g + v (v = 0..3) of column i
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int rr = row0 + (wave * MT + mt) * 16 + 4 * g + v;
        if (rr >= nrows) continue;
        const int id = list ? list[rr] : rr;
        const long orow = args.out_rows ? (long)args.out_rows[id] : (long)id;
        float s = 1.f;
        if (args.row_scale) s = args.scale_mode == 1 ? 1.f / (args.row_scale[id] + 1.f) : args.row_scale[id];
        float* __restrict__ op = args.out + orow * args.out_stride + cp.out_off + i;
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const float val = s * acc[mt][nt][v];
          if (args.accumulate)
            op[16 * nt] += val;
          else
            op[16 * nt] = val;
        }
      }
    }
    rw = rw_next;
  }
}

// Flat argument form for the C ABI: comp table as int arrays [n_comp][MM_LIN_MAX_SRC] etc.
extern "C" int mm_linear(const float* in, long in_stride, const int* in_rows, float* out, long out_stride,
                         const int* out_rows, const float* W, const float* row_scale, int scale_mode,
                         const int* list, const int* list_count, long list_stride, int n_groups, int w_group_stride,
                         int n_rows_max, int accumulate, int n_comp, const int* comp_nsrc, const int* comp_in_off,
                         const int* comp_w_idx, const int* comp_out_off, hipStream_t stream) {
  MM_CHECK_ARG(n_comp >= 1 && n_comp <= MM_LIN_MAX_COMP, "n_comp out of range");
  MM_CHECK_ARG(n_groups >= 1 && n_rows_max >= 0, "bad sizes");
  MM_CHECK_ARG((list == nullptr) == (list_count == nullptr), "list and list_count go together");
  MM_CHECK_ARG(list != nullptr || n_groups == 1, "groups need row lists");
  MM_CHECK_ARG(in_stride % 4 == 0, "input row stride must be a multiple of 4 floats");
  MMLinArgs a;
  a.in = in;
  a.in_stride = in_stride;
  a.in_rows = in_rows;
  a.out = out;
  a.out_stride = out_stride;
  a.out_rows = out_rows;
  a.W = W;
  a.row_scale = row_scale;
  a.scale_mode = scale_mode;
  a.list = list;
  a.list_count = list_count;
  a.list_stride = list_stride;
  a.n_rows = n_rows_max;
  a.w_group_stride = w_group_stride;
  a.accumulate = accumulate;
  a.n_comp = n_comp;
  for (int j = 0; j < n_comp; ++j) {
    MM_CHECK_ARG(comp_nsrc[j] >= 1 && comp_nsrc[j] <= MM_LIN_MAX_SRC, "n_src out of range");
    a.comp[j].n_src = comp_nsrc[j];
    for (int q = 0; q < MM_LIN_MAX_SRC; ++q) {
      a.comp[j].in_off[q] = comp_in_off[j * MM_LIN_MAX_SRC + q];
      a.comp[j].w_idx[q] = comp_w_idx[j * MM_LIN_MAX_SRC + q];
      MM_CHECK_ARG(q >= comp_nsrc[j] || a.comp[j].in_off[q] % 4 == 0, "source offsets must be multiples of 4");
    }
    a.comp[j].out_off = comp_out_off[j];
  }
  if (n_rows_max == 0) return MM_OK;
  // row blocks per workgroup: as many as keep at least MM_LIN_MIN_WG workgroups in the launch (at most 8)
  const long n_blocks = (n_rows_max + MM_LIN_BLOCK_ROWS - 1) / MM_LIN_BLOCK_ROWS;
  const long per_blk = (long)n_comp * n_groups;
  const int n_blk = (int)std::max(1L, std::min(8L, n_blocks * per_blk / MM_LIN_MIN_WG));
  dim3 grid((unsigned)((n_blocks + n_blk - 1) / n_blk), n_comp, n_groups);
  hipLaunchKernelGGL((mm_linear_kernel<MM_LIN_MT, MM_LIN_NW>), grid, dim3(64 * MM_LIN_NW), 0, stream, a, n_blk);
  return mm::launch_status("mm_linear");
}

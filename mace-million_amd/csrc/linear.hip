// Equivariant linear maps of the node features on the matrix cores, at fp32 accuracy from bf16 products
// (v_mfma_f32_16x16x32_bf16, fp32 accumulation).
//
// Every node-level linear of the two layers is a set of 128x128 channel-mixing blocks applied to 128-channel rows
// of ir_mul features (one row per (node, component)): linear_up, linear (with the density division), skip_tp per
// species (fast_layers.SpeciesSkip, fast_layers.py:41-105 -- here the species rows are gathered by per-species
// row lists instead of computing every species and selecting), the product-block linear, and their transposes in
// the backward passes.  For each output component j of one launch:
//     out[out_row(r), comp_j] (= or +=) scale(r) * sum_q in[in_row(r), src_{j,q}] @ W[w_{j,q}]
//
// Split products.  Every fp32 operand is the sum of three bf16 values, x = x0 + x1 + x2 with x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1) (round to nearest even; the differences are exact in fp32), so that
// |x - x0 - x1 - x2| <= 2^-27 |x|.  A product a b is taken as the six bf16 products a_i b_j with i + j <= 2; the
// omitted ones are below 3 * 2^-24 |a b|, the size of an fp32 rounding, and every sum is accumulated in fp32.
// Six 16x16x32 bf16 products take 96 cycles against 256 for the same K = 32 in v_mfma_f32_16x16x4f32.  The
// weights are split once on the host; the input rows are split as they are loaded.
//
// Launch: grid (n_comp, ceil(rows / (256 n_blk)), n_groups), components fastest: the workgroups of one row block
// are dispatched together, so an output row is written and an input row is read by neighbouring workgroups
// (measured: 4-15 % less linear time than row blocks fastest).  1024 threads = 16 waves, each wave 16 rows x 128
// columns (8 MFMA tiles) of each of its n_blk row blocks; the weight block (3 bf16 planes of 128 x 128, 96 KiB)
// is staged in LDS in the lane order of the B operand.  16 waves of one workgroup per CU = 4 waves per SIMD.
// Weight blocks: plane p of block b at bf16 offset (3 b + p) 16384; element W[k][n], k = 32 t + 8 g + u,
// n = 16 nt + i, at (((t * 8 + nt) * 4 + g) * 16 + i) * 8 + u, so that lane (i, g) reads its 8 k-values of step t
// and tile nt as one 16-byte LDS read, the 16 lanes of a group reading 256 consecutive bytes (no bank conflicts);
// the A operand of lane (row, g) is in[row][32 t + 8 g .. + 7], loaded coalesced and passed through 2.5 KiB of
// LDS rows per wave (mm_lin_load_a, mm_lin_stage_a); a row past the last one reads logical row 0 and is not stored.
#include "common.h"

#include <algorithm>

#define MM_LIN_MAX_COMP 48
#define MM_LIN_MAX_SRC 3
#define MM_LIN_NW 16
#define MM_LIN_BLOCK_ROWS (16 * MM_LIN_NW)
#define MM_LIN_AS 40   // LDS row stride (floats) of a wave's A staging rows
// a launch keeps at least this many workgroups (4 per CU) when it groups row blocks per workgroup
#define MM_LIN_MIN_WG 1024

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx8 __attribute__((ext_vector_type(8)));

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
  const uint4* W;         // weight blocks: 3 bf16 planes of 16384 values each (6144 x 16 B per block)
  const float* row_scale; // nullable: per logical row id
  int scale_mode;         // 0: scale = row_scale[id]; 1: scale = 1 / (row_scale[id] + 1)
  const int* list;        // nullable: per group g, list[g * list_stride + r] = logical row id
  const int* list_count;  // per group row count (device): with list, or alone for one group of rows 0 .. n - 1
  long list_stride;
  int n_rows;             // without list
  int w_group_stride;     // weight block offset of group g (species)
  int in_cb;              // 0: input rows component-major; n > 0: 16-channel-block-major rows [8][n][16], a
                          // source chunk at in_off = 128 k being component k of every block
  int accumulate;
  int n_comp;
  MMLinComp comp[MM_LIN_MAX_COMP];
};

struct MMLinRows {
  bool valid;
  long in_row;
};

__device__ __forceinline__ void mm_lin_rows(const MMLinArgs& args, const int* list, int nrows, int row0, int wave,
                                            int i, MMLinRows& rw) {
  const int r = row0 + wave * 16 + i;
  rw.valid = r < nrows;
  const int rid = rw.valid ? (list ? list[r] : r) : 0;
  rw.in_row = args.in_rows ? (long)args.in_rows[rid] : (long)rid;
}

// Input rows of one source, loaded coalesced: lane L reads rows L >> 3 and 8 + (L >> 3) of the wave's 16, floats
// 32 t + 4 (L & 7) .. + 3 of the source chunk, into a[2 t] and a[2 t + 1] (t = 0..3): 8 lanes read 128 contiguous
// bytes of a row.  (In the MFMA operand layout the 16 lanes of a row group would read 16 different rows, which the
// texture path serves one lane per clock.)  mm_lin_stage_a passes step t through the wave's LDS rows into the
// operand layout.
// With channel-block-major input rows (in_cb = n components per block), chunk float q = 32 t + 4 (L & 7) of
// component k lies at (q >> 4) 16 n + 16 k + (q & 15): every lane's 4 floats stay contiguous.
__device__ __forceinline__ void mm_lin_load_a(const MMLinArgs& args, const MMLinRows& rw, int in_off, int lane,
                                              floatx4 (&a)[8]) {
  const long r0 = __shfl(rw.in_row, lane >> 3), r1 = __shfl(rw.in_row, 8 + (lane >> 3));
  const int qb = 4 * (lane & 7);
  const int n = args.in_cb;
  const int base = n ? (qb >> 4) * 16 * n + 16 * (in_off >> 7) + (qb & 15) : in_off + qb;
  const int tstep = n ? 32 * n : 32;
  const float* __restrict__ p0 = args.in + r0 * args.in_stride + base;
  const float* __restrict__ p1 = args.in + r1 * args.in_stride + base;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    a[2 * t] = *(const floatx4*)(p0 + tstep * t);
    a[2 * t + 1] = *(const floatx4*)(p1 + tstep * t);
  }
}

// A operand of step t: lane (i, g) gets in[row i][32 t + 8 g .. + 7], through the wave's LDS rows (row stride
// MM_LIN_AS floats: the 16-byte reads of the 16 rows fall in different banks)
__device__ __forceinline__ floatx8 mm_lin_stage_a(const floatx4 (&a)[8], int t, int lane, int i, int g,
                                                  float* __restrict__ as) {
  mm_wave_lds_sync();   // the previous step's reads are done
  *(floatx4*)(as + (lane >> 3) * MM_LIN_AS + 4 * (lane & 7)) = a[2 * t];
  *(floatx4*)(as + (8 + (lane >> 3)) * MM_LIN_AS + 4 * (lane & 7)) = a[2 * t + 1];
  mm_wave_lds_sync();
  const floatx4 xa = *(const floatx4*)(as + i * MM_LIN_AS + 8 * g);
  const floatx4 xb = *(const floatx4*)(as + i * MM_LIN_AS + 8 * g + 4);
  return floatx8{xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
}

// x = x0 + x1 + x2 (bf16, round to nearest even; both differences are exact in fp32)
__device__ __forceinline__ void mm_split3_bf16(const floatx8& x, bf16x8& x0, bf16x8& x1, bf16x8& x2) {
  x0 = __builtin_convertvector(x, bf16x8);
  const floatx8 r1 = x - __builtin_convertvector(x0, floatx8);
  x1 = __builtin_convertvector(r1, bf16x8);
  const floatx8 r2 = r1 - __builtin_convertvector(x1, floatx8);
  x2 = __builtin_convertvector(r2, bf16x8);
}

// A workgroup handles n_blk consecutive row blocks of one output component.  A weight block is staged in LDS only
// when it is not the one already there: once for all row blocks with a single source, n_src - 1 times per row block
// after the first with several (their order alternates between row blocks).
__global__ void __launch_bounds__(64 * MM_LIN_NW) mm_linear_kernel(MMLinArgs args, int n_blk) {
  __shared__ uint4 Wl[3 * 2048];
  __shared__ float As_all[MM_LIN_NW * 16 * MM_LIN_AS];   // per wave: 16 rows of one K-step
  const MMLinComp& cp = args.comp[blockIdx.x];   // kernel-argument memory, read with uniform indices
  const int grp = blockIdx.z;
  const int nrows = args.list_count ? min(args.list_count[grp], args.n_rows) : args.n_rows;
  const int blk0 = blockIdx.y * n_blk;
  if (blk0 * MM_LIN_BLOCK_ROWS >= nrows) return;
  const int blk1 = min(blk0 + n_blk, (nrows + MM_LIN_BLOCK_ROWS - 1) / MM_LIN_BLOCK_ROWS);
  const int* __restrict__ list = args.list ? args.list + (size_t)grp * args.list_stride : nullptr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  float* __restrict__ as = As_all + wave * 16 * MM_LIN_AS;
  const int n_src = cp.n_src;
  int staged = -1;   // weight block held in LDS (wave-uniform)
  MMLinRows rw;
  mm_lin_rows(args, list, nrows, blk0 * MM_LIN_BLOCK_ROWS, wave, i, rw);
  for (int blk = blk0; blk < blk1; ++blk) {
    const int row0 = blk * MM_LIN_BLOCK_ROWS;
    floatx4 acc[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
    // odd row blocks take the sources in reverse order, so that the block in LDS at the end of one row block is
    // the first one the next needs (n_src - 1 stagings per row block instead of n_src; the order depends only on
    // the row block, so every launch partition sums a row in the same order)
    for (int qq = 0; qq < n_src; ++qq) {
      const int q = (blk & 1) ? n_src - 1 - qq : qq;
      floatx4 a[8];
      mm_lin_load_a(args, rw, cp.in_off[q], lane, a);
      const int widx = cp.w_idx[q] + grp * args.w_group_stride;
      if (widx != staged) {
        const uint4* __restrict__ Wg = args.W + (size_t)widx * 6144;
        __syncthreads();
        for (int j = threadIdx.x; j < 6144; j += 64 * MM_LIN_NW) Wl[j] = Wg[j];
        __syncthreads();
        staged = widx;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const floatx8 x = mm_lin_stage_a(a, t, lane, i, g, as);
        bf16x8 a0, a1, a2;
        mm_split3_bf16(x, a0, a1, a2);
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const int o = ((t * 8 + nt) * 4 + g) * 16 + i;
          const bf16x8 b0 = __builtin_bit_cast(bf16x8, Wl[o]);
          const bf16x8 b1 = __builtin_bit_cast(bf16x8, Wl[2048 + o]);
          const bf16x8 b2 = __builtin_bit_cast(bf16x8, Wl[4096 + o]);
          // smallest terms first
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b0, acc[nt], 0, 0, 0);
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b2, acc[nt], 0, 0, 0);
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc[nt], 0, 0, 0);
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b0, acc[nt], 0, 0, 0);
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b1, acc[nt], 0, 0, 0);
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc[nt], 0, 0, 0);
        }
      }
    }
    // D layout of the 16x16 tile: lane (i, g) holds rows 4 g + v (v = 0..3) of column i.  The row indices and
    // scales of the four rows are loaded before any store, and an accumulating launch reads the eight old values
    // of a row together (one memory round trip per row, not one per value).  A lane past the last row uses
    // logical row 0 (there is one) for its loads and stores nothing.
    bool ok[4];
    int id[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int rr = row0 + wave * 16 + 4 * g + v;
      ok[v] = rr < nrows;
      id[v] = ok[v] ? (list ? list[rr] : rr) : 0;
    }
    float* op[4];
    float sc[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const long orow = args.out_rows ? (long)args.out_rows[id[v]] : (long)id[v];
      op[v] = args.out + orow * args.out_stride + cp.out_off + i;
      sc[v] = 1.f;
      if (args.row_scale)
        sc[v] = args.scale_mode == 1 ? 1.f / (args.row_scale[id[v]] + 1.f) : args.row_scale[id[v]];
    }
    if (args.accumulate) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (!ok[v]) continue;
        float old[8];
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) old[nt] = op[v][16 * nt];
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) op[v][16 * nt] = old[nt] + sc[v] * acc[nt][v];
      }
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (!ok[v]) continue;
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) op[v][16 * nt] = sc[v] * acc[nt][v];
      }
    }
    if (blk + 1 < blk1) mm_lin_rows(args, list, nrows, row0 + MM_LIN_BLOCK_ROWS, wave, i, rw);
  }
}

// Flat argument form for the C ABI: comp table as int arrays [n_comp][MM_LIN_MAX_SRC] etc.
extern "C" int mm_linear(const float* in, long in_stride, const int* in_rows, float* out, long out_stride,
                         const int* out_rows, const void* W, const float* row_scale, int scale_mode,
                         const int* list, const int* list_count, long list_stride, int n_groups, int w_group_stride,
                         int n_rows_max, int accumulate, int n_comp, const int* comp_nsrc, const int* comp_in_off,
                         const int* comp_w_idx, const int* comp_out_off, int in_cb, hipStream_t stream) {
  MM_CHECK_ARG(n_comp >= 1 && n_comp <= MM_LIN_MAX_COMP, "n_comp out of range");
  MM_CHECK_ARG(n_groups >= 1 && n_rows_max >= 0, "bad sizes");
  MM_CHECK_ARG(list == nullptr || list_count != nullptr, "a row list needs its counts");
  MM_CHECK_ARG(list != nullptr || list_count == nullptr || n_groups == 1, "a device row count without a list is for "
               "one group");
  MM_CHECK_ARG(list != nullptr || n_groups == 1, "groups need row lists");
  MM_CHECK_ARG(in_stride % 4 == 0, "input row stride must be a multiple of 4 floats");
  MM_CHECK_ARG(in_cb >= 0 && (in_cb == 0 || in_stride >= 128L * in_cb), "channel-block-major rows: in_cb >= 0 "
               "components per block, rows of at least 128 in_cb floats");
  MMLinArgs a;
  a.in = in;
  a.in_stride = in_stride;
  a.in_rows = in_rows;
  a.out = out;
  a.out_stride = out_stride;
  a.out_rows = out_rows;
  a.W = (const uint4*)W;
  a.row_scale = row_scale;
  a.scale_mode = scale_mode;
  a.list = list;
  a.list_count = list_count;
  a.list_stride = list_stride;
  a.n_rows = n_rows_max;
  a.w_group_stride = w_group_stride;
  a.in_cb = in_cb;
  a.accumulate = accumulate;
  a.n_comp = n_comp;
  for (int j = 0; j < n_comp; ++j) {
    MM_CHECK_ARG(comp_nsrc[j] >= 1 && comp_nsrc[j] <= MM_LIN_MAX_SRC, "n_src out of range");
    a.comp[j].n_src = comp_nsrc[j];
    for (int q = 0; q < MM_LIN_MAX_SRC; ++q) {
      a.comp[j].in_off[q] = comp_in_off[j * MM_LIN_MAX_SRC + q];
      a.comp[j].w_idx[q] = comp_w_idx[j * MM_LIN_MAX_SRC + q];
      MM_CHECK_ARG(q >= comp_nsrc[j] || a.comp[j].in_off[q] % 4 == 0, "source offsets must be multiples of 4");
      MM_CHECK_ARG(q >= comp_nsrc[j] || in_cb == 0 || (a.comp[j].in_off[q] % 128 == 0 &&
                   a.comp[j].in_off[q] / 128 < in_cb), "channel-block-major sources are whole components < in_cb");
    }
    a.comp[j].out_off = comp_out_off[j];
  }
  if (n_rows_max == 0) return MM_OK;
  // row blocks per workgroup: as many as keep at least MM_LIN_MIN_WG workgroups in the launch (at most 8)
  const long n_blocks = (n_rows_max + MM_LIN_BLOCK_ROWS - 1) / MM_LIN_BLOCK_ROWS;
  const long per_blk = (long)n_comp * n_groups;
  const int n_blk = (int)std::max(1L, std::min(8L, n_blocks * per_blk / MM_LIN_MIN_WG));
  dim3 grid(n_comp, (unsigned)((n_blocks + n_blk - 1) / n_blk), n_groups);
  hipLaunchKernelGGL(mm_linear_kernel, grid, dim3(64 * MM_LIN_NW), 0, stream, a, n_blk);
  return mm::launch_status("mm_linear");
}

// Layer-1 edge convolution in the exact "density projection" (ACE) form, on MFMA.
//
// In layer 1 the sender features depend only on the sender's species s and the radial weights are linear in the
// last hidden layer of the radial MLP:  W_e[w, c] = sum_q ht_q(r_e) A3[q, w, c], with ht = h * f_cut.  So the
// message of receiver i factors as
//     A[i, m, c] = coef_l(m) sum_{s,q} B_i[s, q, m] A3[q, l(m), c] Xs[s, c],
//     B_i[s, q, m] = sum_{e: recv = i, species(send) = s} ht_q(r_e) Y_m(e)                  (64 x 16 per species)
// (the reference's ace_layer1.py:1-104 states the identity).  The per-edge work is the outer product ht x Y;
// the 64 -> 128-channel maps (and the following linear / skip_tp) become one GEMM per atom (mm_linear).
//
// Harmonics: both kernels read the 16-byte edge vector (unit vector, r) and evaluate Y(u) once per edge into the
// wave's LDS rows (the forward for 64-slot batches, the backward for each 16-edge tile), from which the MFMA
// operands are read (instead of storing and re-reading 64 B of harmonics per edge in global memory).
//
// Edge order: each wave lists its receiver's edges grouped by sender species in LDS.  In the forward the groups are
// padded to 8 slots, so that a pair of 4-edge steps holds one species and only that species' MFMAs issue (instead
// of one MFMA per species with the other species' lanes zeroed).  In the backward the groups are not padded: a
// 16-edge tile holds one species except at a group boundary, where it issues one MFMA set per species present.
//
// mm_ace1_fwd: one wave per receiver; B_i accumulated with v_mfma_f32_16x16x4f32 taking 4 edges per step:
//   A operand (16 q x 4 edges) = ht, lane (i, g) -> q = 16 mt + i of edge g; B operand (4 edges x 16 m) = Y.
//   Output layout B[i][m][s * 64 + q] (S_pad species blocks, pad species written as 0), rho[i] = sum of the edge
//   densities.
// mm_ace1_bwd: given gB = dL/dB, per edge dL/dY_m = sum_q ht_q gB[s_e, q, m] and dL/dr = sum_m Y_m
//   sum_q ht'_q gB[s_e, q, m]: two GEMMs per tile of 16 edges (A operand = ht or ht' of edge i at q = 4 k + g,
//   B operand = gB), then a 16-lane sum over m.  Writes part[e][0] = dL/dr, part[e][1 + m] = dL/dY_m.  The table
//   rows are loaded coalesced and ht, ht' reach the MFMA layout through LDS (see the backward section below).
//   gB is read in the MFMA operand order: gB[i][m][s * 64 + 16 g + k] = dL/dB[i, s, q = 4 k + g, m] (mm_linear
//   writes it so, through a column permutation of its weights).
// ht is a cubic spline per knot interval: float4 (a0..a3) coef[row][64], row = table * (M - 1) + interval.
#include "common.h"
#include "gen/sh.h"

#define MM_ACE_H 64
#define MM_ACE_MAX_S 4
#define MM_ACE_YB 64     // slots per harmonic batch (one per lane)
#define MM_ACE_SEG 224   // edges of one species-grouped segment of a receiver
#define MM_ACE_SLOTS 256 // slots of a segment's record list: MM_ACE_SEG edges + at most 7 pad slots per species
#define MM_ACE_BSEG 256  // edges of one segment of a receiver in the backward (4 per lane, 16 tiles)

// Species-grouped records of the segment [eb, eb + n) of a receiver's edges (n <= MM_ACE_SEG), built by one wave in
// its LDS list `rec` (one float4 per slot): rec[slot] = {t, table row, edge offset within the segment, density} for
// an edge and {0, row 0, -1, 0} for a pad slot.  The edges of species s (the sender species, .z of the layer-1 edge
// record) fill the slots [first[s], first[s + 1]) in their CSR order, and every group starts at a multiple of 8, so
// a pair of 4-slot steps of the forward holds one species: the MFMAs of the other species are skipped.  The segment's
// records are loaded once (four 16-byte loads per lane, issued together) and grouped from registers.  first[] is
// wave-uniform.
template <int S>
__device__ __forceinline__ void mm_ace_group(const floatx4* __restrict__ e_pk, int eb, int n, int lane,
                                             floatx4* __restrict__ rec, int (&first)[S + 1]) {
  static_assert(MM_ACE_SEG <= 4 * 64 && MM_ACE_SEG + 7 * MM_ACE_MAX_S <= MM_ACE_SLOTS - 4, "segment sizes");
  floatx4 r[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) r[b] = e_pk[eb + min(64 * b + lane, n - 1)];   // (clamped: every load issued)
  int slot = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    first[s] = slot;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (64 * b >= n) break;   // (wave-uniform)
      const int j = 64 * b + lane;
      const bool in = j < n && __float_as_int(r[b].z) == s;
      const unsigned long long mask = __ballot(in);
      if (in) {
        floatx4 q = r[b];
        q.z = __int_as_float(j);
        rec[slot + __popcll(mask & ((1ull << lane) - 1ull))] = q;
      }
      slot += __popcll(mask);
    }
    const int pad = (8 - (slot & 7)) & 7;
    if (lane < pad) rec[slot + lane] = floatx4{0.f, 0.f, __int_as_float(-1), 0.f};
    slot += pad;
  }
  first[S] = slot;
  // the slots beyond the last group hold pad records too, so a step's rows may be loaded past the end
  for (int j = slot + lane; j < MM_ACE_SLOTS; j += 64) rec[j] = floatx4{0.f, 0.f, __int_as_float(-1), 0.f};
  mm_wave_lds_sync();
}

// lane j: harmonics of the edge vector u (has: the lane's slot holds an edge) into yrow[j * 16 .. + 15]
__device__ __forceinline__ void mm_ace_y_store(const floatx4& u, bool has, int lane, float* __restrict__ yrow) {
  mm_wave_lds_sync();   // the previous batch has been read
  if (has) {
    float Y[16];
    mm_sh16(u.x, u.y, u.z, Y);
    floatx4* __restrict__ d = (floatx4*)(yrow + lane * 16);
    d[0] = floatx4{Y[0], Y[1], Y[2], Y[3]};
    d[1] = floatx4{Y[4], Y[5], Y[6], Y[7]};
    d[2] = floatx4{Y[8], Y[9], Y[10], Y[11]};
    d[3] = floatx4{Y[12], Y[13], Y[14], Y[15]};
  }
  mm_wave_lds_sync();
}

// edge vector of slot sl of the segment starting at eb (has = false for a pad slot or sl >= nslot, whose load reads
// the segment's first edge: the load is unconditional)
__device__ __forceinline__ floatx4 mm_ace_slot_u(int sl, int nslot, int eb, const floatx4* __restrict__ rec,
                                                 const floatx4* __restrict__ e_u, bool& has) {
  const int oj = sl < nslot ? __float_as_int(rec[sl].z) : -1;
  has = oj >= 0;
  return e_u[eb + max(oj, 0)];
}

// the four table rows of the forward step at slot sl (lane (i16, g): slot sl + g, features 16 mt + i16)
__device__ __forceinline__ void mm_ace_fwd_rows(const floatx4* __restrict__ tab, const floatx4* __restrict__ rec,
                                                int sl, int g, int i16, floatx4 (&c)[4]) {
  const floatx4* __restrict__ tp = tab + (size_t)__float_as_int(rec[sl + g].y) * MM_ACE_H + i16;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) c[mt] = tp[16 * mt];
}

// one forward step: the 4 slots at sl (all of the species whose accumulators acc are) into B's accumulators
__device__ __forceinline__ void mm_ace_fwd_step(const floatx4 (&c)[4], const floatx4* __restrict__ rec,
                                                const float* __restrict__ yrow, int sl, int g, int i16,
                                                floatx4 (&acc)[4], float& dsum) {
  const floatx4 pk = rec[sl + g];
  // a pad slot holds row 0 (finite) and density 0; its h is zeroed by a factor
  const bool valid = __float_as_int(pk.z) >= 0;
  const float y = valid ? yrow[((sl + g) & (MM_ACE_YB - 1)) * 16 + i16] : 0.f;
  const float t = pk.x;
  if (i16 == 0) dsum += pk.w;
  const float vf = valid ? 1.f : 0.f;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const float h = vf * fmaf(fmaf(fmaf(c[mt].w, t, c[mt].z), t, c[mt].y), t, c[mt].x);
    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(h, y, acc[mt], 0, 0, 0);
  }
}

template <int S>
__global__ void __launch_bounds__(256) mm_ace1_fwd_kernel(const int* __restrict__ rowptr, int nC,
                                                          const floatx4* __restrict__ e_pk,
                                                          const floatx4* __restrict__ e_u,
                                                          const floatx4* __restrict__ tab, int S_pad,
                                                          float* __restrict__ Bout, float* __restrict__ rho) {
  __shared__ float yrows[4 * MM_ACE_YB * 16];
  __shared__ floatx4 recs[4 * MM_ACE_SLOTS];
  float* __restrict__ yrow = yrows + (threadIdx.x >> 6) * (MM_ACE_YB * 16);
  floatx4* __restrict__ rec = recs + (threadIdx.x >> 6) * MM_ACE_SLOTS;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= nC) return;   // the kernel synchronises only within a wave
  const int lane = threadIdx.x & 63, i16 = lane & 15, g = lane >> 4;
  const int e0 = rowptr[i], e1 = rowptr[i + 1];
  floatx4 acc[S][4];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[s][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float dsum = 0.f;
  for (int eb = e0; eb < e1; eb += MM_ACE_SEG) {
    const int n = min(MM_ACE_SEG, e1 - eb);
    int first[S + 1];
    mm_ace_group<S>(e_pk, eb, n, lane, rec, first);
    const int nslot = first[S];
    // software pipeline over pairs of steps: buffer A holds the rows of the even steps, B of the odd ones, and
    // each buffer is reloaded for the step two ahead right after its use (no register copies of loads in flight,
    // which would make the compiler wait for them); the edge vectors of a 64-slot harmonic batch are loaded
    // during the batch before.  A pair of steps lies in one species group, whose accumulators are known at
    // compile time in the loop over that group.
    floatx4 cA[4], cB[4];
    mm_ace_fwd_rows(tab, rec, 0, g, i16, cA);
    __builtin_amdgcn_sched_barrier(0);
    mm_ace_fwd_rows(tab, rec, 4, g, i16, cB);
    __builtin_amdgcn_sched_barrier(0);
    bool u_has;
    floatx4 u = mm_ace_slot_u(lane, nslot, eb, rec, e_u, u_has);
    int k = 0;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      for (; k < first[s + 1]; k += 8) {
        if ((k & (MM_ACE_YB - 1)) == 0) {   // (wave-uniform)
          mm_ace_y_store(u, u_has, lane, yrow);
          u = mm_ace_slot_u(k + MM_ACE_YB + lane, nslot, eb, rec, e_u, u_has);
        }
        mm_ace_fwd_step(cA, rec, yrow, k, g, i16, acc[s], dsum);
        __builtin_amdgcn_sched_barrier(0);
        mm_ace_fwd_rows(tab, rec, min(k + 8, MM_ACE_SLOTS - 4), g, i16, cA);
        __builtin_amdgcn_sched_barrier(0);
        mm_ace_fwd_step(cB, rec, yrow, k + 4, g, i16, acc[s], dsum);
        __builtin_amdgcn_sched_barrier(0);
        mm_ace_fwd_rows(tab, rec, min(k + 12, MM_ACE_SLOTS - 4), g, i16, cB);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    mm_wave_lds_sync();   // the next segment's records replace these
  }
  // C layout: lane (j = i16, g) holds rows 4 g + v (q within the 16-block mt) of column m = j
  float* __restrict__ op = Bout + (size_t)i * 16 * S_pad * MM_ACE_H + (size_t)i16 * S_pad * MM_ACE_H + 4 * g;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) *(floatx4*)(op + s * MM_ACE_H + 16 * mt) = acc[s][mt];
  for (int s = S; s < S_pad; ++s)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) *(floatx4*)(op + s * MM_ACE_H + 16 * mt) = floatx4{0.f, 0.f, 0.f, 0.f};
  dsum += __shfl_xor(dsum, 16);
  dsum += __shfl_xor(dsum, 32);
  if (lane == 0) rho[i] = dsum;
}

// ------------------------------------------------------------------------------------------------ backward
// A segment of up to MM_ACE_BSEG edges of one receiver is staged in the wave's LDS, its edges listed by sender
// species (slots [first[s], first[s + 1]) hold species s, CSR order within a species, no padding between groups):
// rec[slot] = {t, table row, edge offset in the segment, 0} and uv[slot] = the edge vector; slots beyond the segment
// hold pad records (row 0, edge -1).  A tile of 16 slots holds one species except at a group boundary, so most
// tiles issue one species' MFMAs instead of one set per species with the other species' lanes zeroed.
//
// Table rows are loaded coalesced: in half kh of a tile, load j (< 8) of a lane reads feature q = 32 kh + (lane & 31)
// of slot 2 j + (lane >> 5), so each half-wave reads 512 contiguous bytes of one row (in the MFMA layout, lane
// (i, g) would need edge i's row and the 16 lanes of a row group would read 16 different rows, which the texture
// path serves one lane per clock).  The cubic is evaluated in that layout and h, h' are passed to the MFMA layout
// through the wave's LDS (hT[edge i][g][k], 2 KiB each for one half).
template <int S>
__device__ __forceinline__ void ace_bwd_stage(const floatx4* __restrict__ e_pk, const floatx4* __restrict__ e_u,
                                              int sb, int n, int lane, floatx4* __restrict__ rec,
                                              floatx4* __restrict__ uv, int (&first)[S + 1]) {
  floatx4 r[4], u[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {   // (clamped: every load issued)
    const int j = sb + min(64 * b + lane, n - 1);
    r[b] = e_pk[j];
    u[b] = e_u[j];
  }
  mm_wave_lds_sync();   // the previous segment has been read
  int slot = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    first[s] = slot;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (64 * b >= n) break;   // (wave-uniform)
      const int j = 64 * b + lane;
      const bool in = j < n && __float_as_int(r[b].z) == s;
      const unsigned long long mask = __ballot(in);
      if (in) {
        const int sl = slot + __popcll(mask & ((1ull << lane) - 1ull));
        rec[sl] = floatx4{r[b].x, r[b].y, __int_as_float(j), 0.f};
        uv[sl] = u[b];
      }
      slot += __popcll(mask);
    }
  }
  first[S] = slot;
  for (int j = slot + lane; j < MM_ACE_BSEG; j += 64) {
    rec[j] = floatx4{0.f, 0.f, __int_as_float(-1), 0.f};
    uv[j] = floatx4{0.f, 0.f, 1.f, 0.f};
  }
  mm_wave_lds_sync();
}

// species of slot sl (wave-uniform when sl is)
template <int S>
__device__ __forceinline__ int ace_species_of(int sl, const int (&first)[S + 1]) {
  int sp = 0;
#pragma unroll
  for (int s = 1; s < S; ++s) sp += sl >= first[s] ? 1 : 0;
  return sp;
}

// coalesced rows of half kh of the tile at slot tb (see above); tb <= MM_ACE_BSEG - 16
__device__ __forceinline__ void ace_bwd_load_half(const floatx4* __restrict__ tab, const floatx4* __restrict__ rec,
                                                  int tb, int kh, int lane, floatx4 (&c)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = __float_as_int(rec[tb + 2 * j + (lane >> 5)].y);
    c[j] = tab[(size_t)row * MM_ACE_H + 32 * kh + (lane & 31)];
  }
}

// h and h' of half kh from its coalesced rows, into hT / hpT[edge i][g][k] (feature 32 kh + 4 k + g), then read back
// in the MFMA layout: lane (i16, g) gets h[k] = h(edge i16, feature 32 kh + 4 k + g), k < 8
__device__ __forceinline__ void ace_bwd_h_half(const floatx4 (&c)[8], const floatx4* __restrict__ rec, int tb,
                                               int lane, int i16, int g, float* __restrict__ hT,
                                               float* __restrict__ hpT, float (&h)[8], float (&hp)[8]) {
  const int qh = lane & 31;
  const int wofs = (lane >> 5) * 32 + (qh & 3) * 8 + (qh >> 2);   // (edge 2 j + (lane >> 5), g = qh & 3, k = qh >> 2)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float t = rec[tb + 2 * j + (lane >> 5)].x;
    hT[64 * j + wofs] = fmaf(fmaf(fmaf(c[j].w, t, c[j].z), t, c[j].y), t, c[j].x);
    hpT[64 * j + wofs] = fmaf(fmaf(3.f * c[j].w, t, 2.f * c[j].z), t, c[j].y);
  }
  mm_wave_lds_sync();
  const floatx4* __restrict__ hr = (const floatx4*)(hT + (i16 * 4 + g) * 8);
  const floatx4* __restrict__ hpr = (const floatx4*)(hpT + (i16 * 4 + g) * 8);
  const floatx4 h0 = hr[0], h1 = hr[1], p0 = hpr[0], p1 = hpr[1];
  h[0] = h0.x; h[1] = h0.y; h[2] = h0.z; h[3] = h0.w; h[4] = h1.x; h[5] = h1.y; h[6] = h1.z; h[7] = h1.w;
  hp[0] = p0.x; hp[1] = p0.y; hp[2] = p0.z; hp[3] = p0.w; hp[4] = p1.x; hp[5] = p1.y; hp[6] = p1.z; hp[7] = p1.w;
  mm_wave_lds_sync();   // read before the next half overwrites hT
}

// the MFMAs of half kh: K-steps 8 kh + k of dY (A operand h) and dYp (A operand h'), one set per species present in
// the tile (s_lo .. s_hi, wave-uniform), the lanes of other species (and pad slots, se = -1) zeroed
template <int S>
__device__ __forceinline__ void ace_bwd_mfma_half(const float (&h)[8], const float (&hp)[8], int se, int s_lo,
                                                  int s_hi, const float (&gb)[S][16], int kh, floatx4& dY,
                                                  floatx4& dYp) {
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (s < s_lo || s > s_hi) continue;   // (wave-uniform)
    const float fs = se == s ? 1.f : 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      dY = __builtin_amdgcn_mfma_f32_16x16x4f32(h[k] * fs, gb[s][8 * kh + k], dY, 0, 0, 0);
      dYp = __builtin_amdgcn_mfma_f32_16x16x4f32(hp[k] * fs, gb[s][8 * kh + k], dYp, 0, 0, 0);
    }
  }
}

// part rows of a tile: lane (i16 = m, g) holds dL/dY_m of the slots 4 g + v, whose edges are ev[v] (-1: none), and,
// in every lane, dL/dr of those edges
__device__ __forceinline__ void ace_bwd_store(float* __restrict__ part, const int (&ev)[4], int i16,
                                              const floatx4& dY, const float (&gr)[4]) {
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (ev[v] >= 0) {
      float* __restrict__ pp = part + (size_t)ev[v] * 17;
      pp[1 + i16] = dY[v];
      if (i16 == 0) pp[0] = gr[v];
    }
  }
}

// One wave per receiver, tiles of 16 slots of its species-ordered segments.  The loop is software-pipelined by
// halves of a tile: the next tile's first-half rows are loaded once this tile's first half has been evaluated, its
// second-half rows once this tile's second half has been, so half a tile of rows (8 loads per lane) is in flight
// at any time, and a buffer is reloaded only after its last use (no register copies of loads in flight, which would
// make the compiler wait for them).  The part rows of a tile are stored during the next tile, before its row loads,
// so that waiting for rows never waits for fresh stores (the wait counter counts both, in order).
template <int S>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S <= 2 ? 3 : 2)))
mm_ace1_bwd_kernel(const int* __restrict__ rowptr, int nC, const floatx4* __restrict__ e_pk,
                   const floatx4* __restrict__ e_u, const floatx4* __restrict__ tab, int S_pad,
                   const float* __restrict__ gB, float inv_h, float* __restrict__ part) {
  __shared__ floatx4 recs[4 * MM_ACE_BSEG];
  __shared__ floatx4 uvs[4 * MM_ACE_BSEG];
  __shared__ float yts[4 * 16 * 16];
  __shared__ float hts[4 * 2 * 16 * 32];
  const int w = threadIdx.x >> 6;
  floatx4* __restrict__ rec = recs + w * MM_ACE_BSEG;
  floatx4* __restrict__ uv = uvs + w * MM_ACE_BSEG;
  float* __restrict__ yt = yts + w * 256;
  float* __restrict__ hT = hts + w * 1024;
  float* __restrict__ hpT = hT + 512;
  const int i = blockIdx.x * 4 + w;
  if (i >= nC) return;
  const int lane = threadIdx.x & 63, i16 = lane & 15, g = lane >> 4;
  const int e0 = rowptr[i], e1 = rowptr[i + 1];
  if (e0 >= e1) return;
  int n = min(MM_ACE_BSEG, e1 - e0);
  int first[S + 1];
  ace_bwd_stage<S>(e_pk, e_u, e0, n, lane, rec, uv, first);
  // B operand of step k (4 q x 16 m): lane (j = i16, g) holds dL/dB[i, s, q = 4 k + g, m = j].  gB stores it in
  // this operand order, gB[i][m][s * 64 + 16 g + k], so a lane's 16 values of one species are 64 contiguous bytes
  // (four 16-byte loads per species instead of sixteen 4-byte loads).
  float gb[S][16];
  const floatx4* __restrict__ gp =
      (const floatx4*)(gB + (size_t)i * 16 * S_pad * MM_ACE_H + (size_t)i16 * S_pad * MM_ACE_H + 16 * g);
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const floatx4 wv = gp[s * (MM_ACE_H / 4) + kk];
      gb[s][4 * kk] = wv.x;
      gb[s][4 * kk + 1] = wv.y;
      gb[s][4 * kk + 2] = wv.z;
      gb[s][4 * kk + 3] = wv.w;
    }
  floatx4 sdY = {0.f, 0.f, 0.f, 0.f};
  float sgr[4] = {0.f, 0.f, 0.f, 0.f};
  int sev[4] = {-1, -1, -1, -1};   // edges of the tile whose part rows are pending (-1: none)
  for (int sb = e0; sb < e1; sb += MM_ACE_BSEG) {
    if (sb != e0) {
      // the pending rows name edges of the previous segment, whose records the stage replaces: store them first
      ace_bwd_store(part, sev, i16, sdY, sgr);
#pragma unroll
      for (int v = 0; v < 4; ++v) sev[v] = -1;
      n = min(MM_ACE_BSEG, e1 - sb);
      ace_bwd_stage<S>(e_pk, e_u, sb, n, lane, rec, uv, first);
    }
    floatx4 cA[8], cB[8];
    __builtin_amdgcn_sched_barrier(0);   // the loop's wait counts assume the first half issued first
    ace_bwd_load_half(tab, rec, 0, 0, lane, cA);
    __builtin_amdgcn_sched_barrier(0);
    ace_bwd_load_half(tab, rec, 0, 1, lane, cB);
    __builtin_amdgcn_sched_barrier(0);
    for (int tb = 0; tb < n; tb += 16) {
      const int tbn = min(tb + 16, MM_ACE_BSEG - 16);   // next tile's rows (after the last: pad rows, unused)
      const int s_lo = ace_species_of<S>(tb, first), s_hi = ace_species_of<S>(min(tb + 15, n - 1), first);
      const int se = tb + i16 < n ? ace_species_of<S>(tb + i16, first) : -1;
      // harmonics of the tile's 16 edges: lane j < 16 evaluates slot tb + j into yt[j][m]
      {
        const floatx4 uu = uv[tb + i16];
        float Y[16];
        mm_sh16(uu.x, uu.y, uu.z, Y);
        if (lane < 16) {
          floatx4* __restrict__ d = (floatx4*)(yt + lane * 16);
          d[0] = floatx4{Y[0], Y[1], Y[2], Y[3]};
          d[1] = floatx4{Y[4], Y[5], Y[6], Y[7]};
          d[2] = floatx4{Y[8], Y[9], Y[10], Y[11]};
          d[3] = floatx4{Y[12], Y[13], Y[14], Y[15]};
        }
      }
      floatx4 dY = {0.f, 0.f, 0.f, 0.f}, dYp = {0.f, 0.f, 0.f, 0.f};
      float h[8], hp[8];
      ace_bwd_h_half(cA, rec, tb, lane, i16, g, hT, hpT, h, hp);
      __builtin_amdgcn_sched_barrier(0);
      ace_bwd_store(part, sev, i16, sdY, sgr);   // the previous tile's results
      ace_bwd_load_half(tab, rec, tbn, 0, lane, cA);
      __builtin_amdgcn_sched_barrier(0);
      ace_bwd_mfma_half<S>(h, hp, se, s_lo, s_hi, gb, 0, dY, dYp);
      ace_bwd_h_half(cB, rec, tb, lane, i16, g, hT, hpT, h, hp);
      __builtin_amdgcn_sched_barrier(0);
      ace_bwd_load_half(tab, rec, tbn, 1, lane, cB);
      __builtin_amdgcn_sched_barrier(0);
      ace_bwd_mfma_half<S>(h, hp, se, s_lo, s_hi, gb, 1, dY, dYp);
      // C layout: lane (j = i16 = m, g) holds slots tb + 4 g + v of column m
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int sl = tb + 4 * g + v;
        const int ej = __float_as_int(rec[sl].z);
        const float yv = ej >= 0 ? yt[(4 * g + v) * 16 + i16] : 0.f;
        sgr[v] = mm_row_sum16(dYp[v] * yv) * mm_spline_dxdr(rec[sl].x, inv_h);
        sev[v] = ej >= 0 ? sb + ej : -1;
      }
      sdY = dY;
    }
  }
  ace_bwd_store(part, sev, i16, sdY, sgr);
}

template <int S>
static void launch_fwd(dim3 grid, hipStream_t stream, const int* rowptr, int nC, const float* e_pk, const float* e_u,
                       const float* tab, int S_pad, float* Bout, float* rho) {
  hipLaunchKernelGGL(mm_ace1_fwd_kernel<S>, grid, dim3(256), 0, stream, rowptr, nC, (const floatx4*)e_pk,
                     (const floatx4*)e_u,
                     (const floatx4*)tab, S_pad, Bout, rho);
}

template <int S>
static void launch_bwd(dim3 grid, hipStream_t stream, const int* rowptr, int nC, const float* e_pk, const float* e_u,
                       const float* tab, int S_pad, const float* gB, float inv_h, float* part) {
  hipLaunchKernelGGL(mm_ace1_bwd_kernel<S>, grid, dim3(256), 0, stream, rowptr, nC, (const floatx4*)e_pk,
                     (const floatx4*)e_u,
                     (const floatx4*)tab, S_pad, gB, inv_h, part);
}

extern "C" int mm_ace1_fwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* tab, int S,
                           int S_pad, float* B, float* rho, hipStream_t stream) {
  MM_CHECK_ARG(nC >= 0 && S >= 1 && S <= MM_ACE_MAX_S && S_pad >= S, "bad sizes (1 <= S <= 4, S_pad >= S)");
  if (nC == 0) return MM_OK;
  const dim3 grid((nC + 3) / 4);
  switch (S) {
    case 1: launch_fwd<1>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, B, rho); break;
    case 2: launch_fwd<2>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, B, rho); break;
    case 3: launch_fwd<3>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, B, rho); break;
    default: launch_fwd<4>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, B, rho); break;
  }
  return mm::launch_status("mm_ace1_fwd");
}

extern "C" int mm_ace1_bwd(const int* rowptr, int nC, const float* e_pk, const float* e_u, const float* tab, int S,
                           int S_pad, const float* gB, float inv_h, float* part, hipStream_t stream) {
  MM_CHECK_ARG(nC >= 0 && S >= 1 && S <= MM_ACE_MAX_S && S_pad >= S, "bad sizes (1 <= S <= 4, S_pad >= S)");
  if (nC == 0) return MM_OK;
  const dim3 grid((nC + 3) / 4);
  switch (S) {
    case 1: launch_bwd<1>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, gB, inv_h, part); break;
    case 2: launch_bwd<2>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, gB, inv_h, part); break;
    case 3: launch_bwd<3>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, gB, inv_h, part); break;
    default: launch_bwd<4>(grid, stream, rowptr, nC, e_pk, e_u, tab, S_pad, gB, inv_h, part); break;
  }
  return mm::launch_status("mm_ace1_bwd");
}

// samples [3, M, D] (values, values at r + eps, at r - eps) -> coef[tab][k][d] float4 (a0..a3 in t), the
// interpolant of mm_spline_coeffs in a flat layout (no channel blocks).
__global__ void mm_spline_coeffs_flat_kernel(const double* __restrict__ samples, int M, int D, double eps, double h,
                                             int tab, float* __restrict__ coef) {
  const long idx = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (idx >= (long)(M - 1) * D) return;
  const int k = (int)(idx / D), d = (int)(idx % D);
  const double* V = samples;
  const double* Vp = samples + (size_t)M * D;
  const double* Vm = samples + (size_t)2 * M * D;
  const double v0 = V[(size_t)k * D + d], v1 = V[(size_t)(k + 1) * D + d];
  const double g0 = (Vp[(size_t)k * D + d] - Vm[(size_t)k * D + d]) / (2 * eps) * h;
  const double g1 = (Vp[(size_t)(k + 1) * D + d] - Vm[(size_t)(k + 1) * D + d]) / (2 * eps) * h;
  float* p = coef + 4 * (((size_t)tab * (M - 1) + k) * D + d);
  p[0] = (float)v0;
  p[1] = (float)g0;
  p[2] = (float)(-3 * v0 - 2 * g0 + 3 * v1 - g1);
  p[3] = (float)(2 * v0 + g0 - 2 * v1 + g1);
}

extern "C" int mm_spline_coeffs_flat(const double* samples, int M, int D, double eps, double h, int tab, float* coef,
                                     hipStream_t stream) {
  MM_CHECK_ARG(M >= 2 && D >= 1 && tab >= 0, "bad sizes");
  const long n = (long)(M - 1) * D;
  hipLaunchKernelGGL(mm_spline_coeffs_flat_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, samples,
                     M, D, eps, h, tab, coef);
  return mm::launch_status("mm_spline_coeffs_flat");
}

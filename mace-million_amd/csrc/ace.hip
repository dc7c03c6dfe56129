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
// Harmonics: both kernels read the 16-byte edge vector (unit vector, r) and evaluate Y(u) once per edge: lane j of
// a wave evaluates edge eb + j of a 64-edge batch into the wave's LDS rows (16 floats per edge), from which the
// MFMA operands are read (instead of storing and re-reading 64 B of harmonics per edge in global memory).
//
// Edge order of the forward: each wave lists its receiver's edges grouped by sender species (mm_ace_group), so that
// a step of 4 edges holds one species and only that species' MFMAs issue (instead of one MFMA per species with the
// other species' lanes zeroed).  The backward keeps the CSR order: grouping its 16-edge tiles the same way halved
// its MFMAs for water but lengthened its per-tile latency chain (order -> edge record -> table rows) and measured
// slower (2.04 -> 2.17 ms per launch at configuration 5).
//
// mm_ace1_fwd: one wave per receiver; B_i accumulated with v_mfma_f32_16x16x4f32 taking 4 edges per step:
//   A operand (16 q x 4 edges) = ht, lane (i, g) -> q = 16 mt + i of edge g; B operand (4 edges x 16 m) = Y.
//   Output layout B[i][m][s * 64 + q] (S_pad species blocks, pad species written as 0), rho[i] = sum of the edge
//   densities.
// mm_ace1_bwd: given gB = dL/dB, per edge dL/dY_m = sum_q ht_q gB[s_e, q, m] and dL/dr = sum_m Y_m
//   sum_q ht'_q gB[s_e, q, m]: two GEMMs per tile of 16 edges (A operand = ht or ht' of edge i at q = 4 k + g,
//   B operand = gB), then a 16-lane sum over m.  Writes part[e][0] = dL/dr, part[e][1 + m] = dL/dY_m.
// ht is a cubic spline per knot interval: float4 (a0..a3) coef[row][64], row = table * (M - 1) + interval.
#include "common.h"
#include "gen/sh.h"

#define MM_ACE_H 64
#define MM_ACE_MAX_S 4
#define MM_ACE_YB 64     // slots per harmonic batch (one per lane)
#define MM_ACE_SEG 240   // edges of one species-grouped segment of a receiver
#define MM_ACE_SLOTS 256 // slots of a segment's order list: MM_ACE_SEG edges + at most 3 pad slots per species

// Species-grouped order of the segment [eb, eb + n) of a receiver's edges (n <= MM_ACE_SEG), built by one wave in
// its LDS list `order`: order[slot] = edge offset within the segment, -1 for a pad slot.  The edges of species s
// (the sender species, .z of the layer-1 edge record) fill the slots [first[s], first[s + 1]) in their CSR order,
// and every group starts at a multiple of 4, so a 4-slot step of the forward holds one species: the MFMAs of the
// other species are skipped.  first[] is wave-uniform.
template <int S>
__device__ __forceinline__ void mm_ace_group(const int* __restrict__ pk_i, int eb, int n, int lane,
                                             int* __restrict__ order, int (&first)[S + 1]) {
  int slot = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    first[s] = slot;
    for (int b = 0; b < n; b += 64) {
      const int j = b + lane;
      const bool in = j < n && pk_i[4 * (eb + j) + 2] == s;
      const unsigned long long mask = __ballot(in);
      if (in) order[slot + __popcll(mask & ((1ull << lane) - 1ull))] = j;
      slot += __popcll(mask);
    }
    const int pad = (4 - (slot & 3)) & 3;
    if (lane < pad) order[slot + lane] = -1;
    slot += pad;
  }
  first[S] = slot;
  mm_wave_lds_sync();
}

// lane j: harmonics of the edge in slot sb + j (if any) into yrow[j * 16 .. + 15]
__device__ __forceinline__ void mm_ace_y_batch(int sb, int nslot, int eb, int lane, const int* __restrict__ order,
                                               const floatx4* __restrict__ e_u, float* __restrict__ yrow) {
  mm_wave_lds_sync();   // the previous batch has been read
  const int sl = sb + lane;
  const int oj = sl < nslot ? order[sl] : -1;
  if (oj >= 0) {
    const floatx4 u = e_u[eb + oj];
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

// (backward, CSR order) lane j: harmonics of edge eb + j (if it exists) into yrow[j * 16 .. + 15]; the edge vector of the next batch is
// loaded one batch ahead (u_next)
__device__ __forceinline__ void mm_ace_y_batch_csr(int eb, int e1, int lane, const floatx4* __restrict__ e_u,
                                               floatx4& u_next, float* __restrict__ yrow) {
  mm_wave_lds_sync();   // the previous batch has been read
  const int ej = eb + lane;
  if (ej < e1) {
    const floatx4 u = u_next;
    if (ej + MM_ACE_YB < e1) u_next = e_u[ej + MM_ACE_YB];
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

// species of slot sl (wave-uniform when sl is)
template <int S>
__device__ __forceinline__ int mm_ace_species_of(int sl, const int (&first)[S + 1]) {
  int sp = 0;
#pragma unroll
  for (int s = 1; s < S; ++s) sp += sl >= first[s] ? 1 : 0;
  return __builtin_amdgcn_readfirstlane(sp);
}

template <int S>
__global__ void __launch_bounds__(256) mm_ace1_fwd_kernel(const int* __restrict__ rowptr, int nC,
                                                          const floatx4* __restrict__ e_pk,
                                                          const floatx4* __restrict__ e_u,
                                                          const floatx4* __restrict__ tab, int S_pad,
                                                          float* __restrict__ Bout, float* __restrict__ rho) {
  __shared__ float yrows[4 * MM_ACE_YB * 16];
  __shared__ int orders[4 * MM_ACE_SLOTS];
  float* __restrict__ yrow = yrows + (threadIdx.x >> 6) * (MM_ACE_YB * 16);
  int* __restrict__ order = orders + (threadIdx.x >> 6) * MM_ACE_SLOTS;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= nC) return;   // the kernel synchronises only within a wave
  const int lane = threadIdx.x & 63, i16 = lane & 15, g = lane >> 4;
  const int e0 = rowptr[i], e1 = rowptr[i + 1];
  const int* __restrict__ pk_i = (const int*)e_pk;
  floatx4 acc[S][4];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[s][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float dsum = 0.f;
  for (int eb = e0; eb < e1; eb += MM_ACE_SEG) {
    const int n = min(MM_ACE_SEG, e1 - eb);
    int first[S + 1];
    mm_ace_group<S>(pk_i, eb, n, lane, order, first);
    const int nslot = first[S];
    int oj_n = order[g];                                  // the step's slots are read one step ahead
    floatx4 pk_n = oj_n >= 0 ? e_pk[eb + oj_n] : floatx4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nslot; k += 4) {
      if ((k & (MM_ACE_YB - 1)) == 0) mm_ace_y_batch(k, nslot, eb, lane, order, e_u, yrow);   // (wave-uniform)
      const int oj = oj_n;
      const floatx4 pk = pk_n;
      if (k + 4 < nslot) {
        oj_n = order[k + 4 + g];
        pk_n = oj_n >= 0 ? e_pk[eb + oj_n] : floatx4{0.f, 0.f, 0.f, 0.f};
      }
      const bool valid = oj >= 0;
      const float y = valid ? yrow[((k + g) & (MM_ACE_YB - 1)) * 16 + i16] : 0.f;
      const floatx4* __restrict__ tp = tab + (size_t)(valid ? __float_as_int(pk.y) : 0) * MM_ACE_H + i16;
      const float t = pk.x;
      if (i16 == 0 && valid) dsum += pk.w;
      // the step's four table rows are loaded together, before any use: a pad lane reads row 0 (finite) and its
      // h is zeroed by a factor, so no load sits behind a branch on the slot's validity
      const float vf = valid ? 1.f : 0.f;
      floatx4 c[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) c[mt] = tp[16 * mt];
      __builtin_amdgcn_sched_barrier(0);
      const int sp = mm_ace_species_of<S>(k, first);     // the step's 4 slots hold one species
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const float h = vf * fmaf(fmaf(fmaf(c[mt].w, t, c[mt].z), t, c[mt].y), t, c[mt].x);
#pragma unroll
        for (int s = 0; s < S; ++s)
          if (s == sp) acc[s][mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(h, y, acc[s][mt], 0, 0, 0);
      }
    }
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

// part rows of the 16-edge tile starting at tb: lane (i16 = m, g) holds dL/dY_m of edges tb + 4 g + v and, in every
// lane, dL/dr of those edges
__device__ __forceinline__ void ace_bwd_store(float* __restrict__ part, int tb, int e1, int g, int i16,
                                              const floatx4& dY, const float (&gr)[4]) {
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int ev = tb + 4 * g + v;
    if (ev < e1) {
      float* __restrict__ pp = part + (size_t)ev * 17;
      pp[1 + i16] = dY[v];
      if (i16 == 0) pp[0] = gr[v];
    }
  }
}

template <int S>
__global__ void __launch_bounds__(256) mm_ace1_bwd_kernel(const int* __restrict__ rowptr, int nC,
                                                          const floatx4* __restrict__ e_pk,
                                                          const floatx4* __restrict__ e_u,
                                                          const floatx4* __restrict__ tab, int S_pad,
                                                          const float* __restrict__ gB, float inv_h,
                                                          float* __restrict__ part) {
  __shared__ float yrows[4 * MM_ACE_YB * 16];
  float* __restrict__ yrow = yrows + (threadIdx.x >> 6) * (MM_ACE_YB * 16);
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= nC) return;
  const int lane = threadIdx.x & 63, i16 = lane & 15, g = lane >> 4;
  const int e0 = rowptr[i], e1 = rowptr[i + 1];
  // B operand of step k (4 q x 16 m): lane (j = i16, g) holds gB[i][m = j][s * 64 + 4 k + g]
  float gb[S][16];
  const float* __restrict__ gp = gB + (size_t)i * 16 * S_pad * MM_ACE_H + (size_t)i16 * S_pad * MM_ACE_H + g;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int k = 0; k < 16; ++k) gb[s][k] = gp[s * MM_ACE_H + 4 * k];
  // the packed record of the next tile is loaded one tile ahead; the tile's harmonics before its MFMAs
  floatx4 pk_n = e0 + i16 < e1 ? e_pk[e0 + i16] : floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 u_next = e0 + lane < e1 ? e_u[e0 + lane] : floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 sdY = {0.f, 0.f, 0.f, 0.f};
  float sgr[4] = {0.f, 0.f, 0.f, 0.f};
  int stb = -1;
  for (int tb = e0; tb < e1; tb += 16) {
    if (((tb - e0) & (MM_ACE_YB - 1)) == 0) mm_ace_y_batch_csr(tb, e1, lane, e_u, u_next, yrow);   // (wave-uniform)
    const int e = tb + i16;          // A-operand row: edge i16 of the tile
    const bool valid = e < e1;
    const floatx4 pk = pk_n;
    if (e + 16 < e1) pk_n = e_pk[e + 16];
    float yv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int ev = tb + 4 * g + v;
      yv[v] = ev < e1 ? yrow[((ev - e0) & (MM_ACE_YB - 1)) * 16 + i16] : 0.f;
    }
    const int se = valid ? __float_as_int(pk.z) : -1;
    const floatx4* __restrict__ tp = tab + (size_t)(valid ? __float_as_int(pk.y) : 0) * MM_ACE_H + g;
    const float t = pk.x;
    // the tile's 16 table rows are loaded together, before any use (one memory latency per tile); a pad lane reads
    // row 0 (finite) and its A operands are zeroed by the species factors
    floatx4 c[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) c[k] = tp[4 * k];
    if (stb >= 0) ace_bwd_store(part, stb, e1, g, i16, sdY, sgr);   // the previous tile's results
    __builtin_amdgcn_sched_barrier(0);
    float fs[S];   // 1 for the species of this lane's edge, else 0
#pragma unroll
    for (int s = 0; s < S; ++s) fs[s] = se == s ? 1.f : 0.f;
    floatx4 dY = {0.f, 0.f, 0.f, 0.f}, dYp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float h = fmaf(fmaf(fmaf(c[k].w, t, c[k].z), t, c[k].y), t, c[k].x);
      const float hp = fmaf(fmaf(3.f * c[k].w, t, 2.f * c[k].z), t, c[k].y);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        dY = __builtin_amdgcn_mfma_f32_16x16x4f32(h * fs[s], gb[s][k], dY, 0, 0, 0);
        dYp = __builtin_amdgcn_mfma_f32_16x16x4f32(hp * fs[s], gb[s][k], dYp, 0, 0, 0);
      }
    }
    // C layout: lane (j = i16 = m, g) holds edges tb + 4 g + v of column m
#pragma unroll
    for (int v = 0; v < 4; ++v) sgr[v] = mm_row_sum16(dYp[v] * yv[v]) * inv_h;
    sdY = dY;
    stb = tb;
  }
  if (stb >= 0) ace_bwd_store(part, stb, e1, g, i16, sdY, sgr);
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

// Per-edge geometry of a receiver chunk and the per-edge gradient assembly.
//
// mm_edge_geom_rij / mm_edge_geom_pos: edge vector (fp64 in, fp32 out, as the reference's rij.to(dtype),
// mliap_threepass.py:326) stored as (unit vector, length) -- the convolutions and the ACE kernels evaluate the
// spherical harmonics from it; e_Y (optional, null on the production path) receives the 16 harmonics --, local
// receiver index, and one packed record per edge
// for the convolutions: (t, spline interval row = table(pair) * (M - 1) + k, feature row of the sender, edge
// density d = tanh((B(r) . w / sqrt(nb))^2) f_cut(r)) (fast_layers.py:154-156, 179-183, 190-192); d'(r) separately.
// mm_edge_grad: dL/dv_e = dL/dr u + (I - u u^T) grad_u(sum_m dL/dY_m Y_m) / r, with dL/dr and dL/dY summed
// over the 8 channel blocks of the convolution backward and the density term g_rho[recv] * d'(r) added.
#include "common.h"
#include "gen/sh.h"

#define MM_MAX_BESSEL 16

struct MMDensity {
  float w[MM_MAX_BESSEL];   // density weights / sqrt(nb)
  int nb;
  float r_max;
  int p;
};

// sin(n theta) and cos(n theta) for n = 1..nb come from one fp64 sincos(theta) and the rotation
// (s, c) <- (s cos theta + c sin theta, c cos theta - s sin theta) in fp64: exact to fp32 rounding, where
// sincosf(n * theta) in fp32 first rounds the argument n * theta (up to 8 pi), and measured 15 % less kernel time
// together with x^p by repeated multiplication instead of powf.
__device__ __forceinline__ void mm_density(float r, const MMDensity& dp, float& d, float& dd) {
  const float pi = 3.14159265358979323846f;
  const float pref = sqrtf(2.0f / dp.r_max);
  float s0 = 0.f, s1 = 0.f;   // density pre-activation and its derivative
  const float ir = 1.0f / r;
  double s_1, c_1;
  sincos(3.14159265358979323846 * (double)r / (double)dp.r_max, &s_1, &c_1);
  double s_n = s_1, c_n = c_1;
  for (int n = 1; n <= dp.nb; ++n) {
    const float sn = (float)s_n, cn = (float)c_n;
    const double s_next = s_n * c_1 + c_n * s_1;
    c_n = c_n * c_1 - s_n * s_1;
    s_n = s_next;
    const float b = pref * sn * ir;
    const float db = pref * (n * pi / dp.r_max * cn * ir - sn * ir * ir);
    s0 = fmaf(dp.w[n - 1], b, s0);
    s1 = fmaf(dp.w[n - 1], db, s1);
  }
  const float x = r / dp.r_max;
  float f = 0.f, df = 0.f;
  if (x < 1.f) {
    const float p = (float)dp.p;
    float xp = 1.f;   // x^p (p is a small integer)
    for (int k = 0; k < dp.p; ++k) xp *= x;
    f = 1.f - 0.5f * (p + 1.f) * (p + 2.f) * xp + p * (p + 2.f) * xp * x - 0.5f * p * (p + 1.f) * xp * x * x;
    const float xp1 = xp / x;      // x^(p-1)
    df = (-0.5f * p * (p + 1.f) * (p + 2.f) * xp1 + p * (p + 1.f) * (p + 2.f) * xp
          - 0.5f * p * (p + 1.f) * (p + 2.f) * xp * x) / dp.r_max;
  }
  const float q = s0 * s0;
  const float th2 = tanhf(q);
  d = th2 * f;
  dd = (1.f - th2 * th2) * 2.f * s0 * s1 * f + th2 * df;
}

// Spline coordinate of a length r: x = clamp((r - r_lo) / h, 0, M - 1 - 1e-4), interval k = floor(x), t = x - k
// (the clamp of spline_w._coords, spline_w.py:18-27).  The tables hold M - 1 intervals, so k is also clamped to
// M - 2: for M >= 4096 the fp32 value M - 1 - 1e-4 rounds to M - 1, and floor(x) alone would index one interval
// past the table (then t = x - k = 1, the right end of the last interval).
// A length below r_lo gets t = -0: W is W(r_lo) there (the same value as t = +0), and the backward kernels read
// the sign as "dx/dr = 0" (mm_spline_dxdr).  The reference's backward takes the table's slope at the clamped end
// (spline_w.py:63-79), a force that is not the derivative of its energy there.
struct MMSpline {
  int M;
  float r_lo, inv_h;
};

__device__ __forceinline__ void mm_geom_common(int e, float vx, float vy, float vz, int recv, int send,
                                               const int* __restrict__ node_spec, int S,
                                               const int* __restrict__ pair_map, const MMDensity& dp,
                                               const MMSpline& sp, int x_from_spec, float4* __restrict__ e_u,
                                               float* __restrict__ e_Y, float4* __restrict__ e_pk,
                                               int* __restrict__ e_recv, float* __restrict__ e_dd) {
  const float r = sqrtf(vx * vx + vy * vy + vz * vz);
  const float ir = 1.0f / r;
  e_u[e] = make_float4(vx * ir, vy * ir, vz * ir, r);
  if (e_Y) {
    float Y[16];
    mm_sh16(vx * ir, vy * ir, vz * ir, Y);
    float4* __restrict__ yp = (float4*)(e_Y + (size_t)e * 16);
    yp[0] = make_float4(Y[0], Y[1], Y[2], Y[3]);
    yp[1] = make_float4(Y[4], Y[5], Y[6], Y[7]);
    yp[2] = make_float4(Y[8], Y[9], Y[10], Y[11]);
    yp[3] = make_float4(Y[12], Y[13], Y[14], Y[15]);
  }
  const int tab = pair_map[node_spec[send] * S + node_spec[recv]];
  const float xr = (r - sp.r_lo) * sp.inv_h;
  const float x = fminf(fmaxf(xr, 0.f), (float)(sp.M - 1) - 1e-4f);
  const float kf = fminf(floorf(x), (float)(sp.M - 2));
  const int row = tab * (sp.M - 1) + (int)kf;
  const float t = xr < 0.f ? -0.f : x - kf;
  const int xsrc = x_from_spec ? node_spec[send] : send;
  e_recv[e] = recv;
  float d, dd;
  mm_density(r, dp, d, dd);
  e_pk[e] = make_float4(t, __int_as_float(row), __int_as_float(xsrc), d);
  e_dd[e] = dd;
}

__global__ void mm_edge_geom_rij_kernel(int E, const double* __restrict__ rij, const int* __restrict__ pair_i, int a,
                                        const int* __restrict__ ls, const int* __restrict__ node_spec, int S,
                                        const int* __restrict__ pair_map, MMDensity dp, MMSpline sp, int x_from_spec,
                                        float4* e_u, float* e_Y, float4* e_pk, int* e_recv, float* e_dd,
                                        const int* __restrict__ E_dev) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (E_dev ? *E_dev : E)) return;   // E_dev: the edge count in device memory (graph replays)
  const float vx = (float)rij[3 * (size_t)e + 0];
  const float vy = (float)rij[3 * (size_t)e + 1];
  const float vz = (float)rij[3 * (size_t)e + 2];
  mm_geom_common(e, vx, vy, vz, pair_i[e] - a, ls[e], node_spec, S, pair_map, dp, sp, x_from_spec, e_u, e_Y,
                 e_pk, e_recv, e_dd);
}

// x_i - x_j - L * rint((x_i - x_j) / L), every operation rounded separately (no FMA contraction), as torch's
// System.min_image on the CPU
__device__ __forceinline__ double mm_mic_f64(double xi, double xj, double L) {
#pragma clang fp contract(off)
  const double x = xi - xj;
  return x - L * rint(x / L);
}

// standalone path: v = minimum image of x_recv - x_send in fp64 (receiver_chunk_mace.py:110-111, 194)
__global__ void mm_edge_geom_pos_kernel(int E, const double* __restrict__ pos, double bx, double by, double bz,
                                        const int* __restrict__ recv_local, int a, const int* __restrict__ ls,
                                        const int* __restrict__ nodes, const int* __restrict__ node_spec, int S,
                                        const int* __restrict__ pair_map, MMDensity dp, MMSpline sp,
                                        int x_from_spec, float4* e_u, float* e_Y, float4* e_pk, int* e_recv,
                                        float* e_dd, const int* __restrict__ E_dev) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (E_dev ? *E_dev : E)) return;   // E_dev: the edge count in device memory (graph replays)
  const int rl = recv_local[e];
  const int sl = ls[e];
  const long gi = nodes[rl], gj = nodes[sl];
  double v[3];
  const double b[3] = {bx, by, bz};
#pragma unroll
  for (int k = 0; k < 3; ++k) v[k] = mm_mic_f64(pos[3 * gi + k], pos[3 * gj + k], b[k]);
  (void)a;
  mm_geom_common(e, (float)v[0], (float)v[1], (float)v[2], rl, sl, node_spec, S, pair_map, dp, sp, x_from_spec,
                 e_u, e_Y, e_pk, e_recv, e_dd);
}

__global__ void mm_edge_grad_kernel(int E, const float* __restrict__ part, long part_stride, int n_part,
                                    const float* __restrict__ g_rho, const int* __restrict__ e_recv,
                                    const float* __restrict__ e_dd, const float4* __restrict__ e_u,
                                    float* __restrict__ pf, int accumulate, const int* __restrict__ E_dev) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (E_dev ? *E_dev : E)) return;   // E_dev: the edge count in device memory (graph replays)
  float g[17];
#pragma unroll
  for (int j = 0; j < 17; ++j) g[j] = 0.f;
  for (int cb = 0; cb < n_part; ++cb) {
    const float* __restrict__ pp = part + (size_t)cb * part_stride + (size_t)e * 17;
#pragma unroll
    for (int j = 0; j < 17; ++j) g[j] += pp[j];
  }
  const float gr = g[0] + (g_rho ? g_rho[e_recv[e]] * e_dd[e] : 0.f);
  const float4 u = e_u[e];
  const float ux = u.x, uy = u.y, uz = u.z;
  const float ir = 1.0f / u.w;
  float G[3];
  mm_sh16_grad(ux, uy, uz, g + 1, G);
  const float ug = ux * G[0] + uy * G[1] + uz * G[2];
  const float gx = gr * ux + (G[0] - ug * ux) * ir;
  const float gy = gr * uy + (G[1] - ug * uy) * ir;
  const float gz = gr * uz + (G[2] - ug * uz) * ir;
  float* __restrict__ o = pf + 3 * (size_t)e;
  if (accumulate) {
    o[0] += gx;
    o[1] += gy;
    o[2] += gz;
  } else {
    o[0] = gx;
    o[1] = gy;
    o[2] = gz;
  }
}

static int make_density(MMDensity& dp, const float* w, int nb, float r_max, int p) {
  if (nb < 1 || nb > MM_MAX_BESSEL) return MM_EINVAL;
  for (int i = 0; i < MM_MAX_BESSEL; ++i) dp.w[i] = i < nb ? w[i] : 0.f;
  dp.nb = nb;
  dp.r_max = r_max;
  dp.p = p;
  return MM_OK;
}

extern "C" int mm_edge_geom_rij(int E, const int* E_dev, const double* rij, const int* pair_i, int a,
                                const int* ls, const int* node_spec, int S, const int* pair_map, const float* dens_w,
                                int nb, float r_max, int p_cut, int M, float r_lo, float inv_h, int x_from_spec,
                                float* e_u, float* e_Y, float* e_pk, int* e_recv, float* e_dd, hipStream_t stream) {
  MM_CHECK_ARG(E >= 0 && S >= 1 && M >= 2, "bad sizes");
  MMDensity dp;
  MM_CHECK_ARG(make_density(dp, dens_w, nb, r_max, p_cut) == MM_OK, "nb out of range");
  const MMSpline sp{M, r_lo, inv_h};
  if (E == 0) return MM_OK;
  hipLaunchKernelGGL(mm_edge_geom_rij_kernel, dim3((E + 255) / 256), dim3(256), 0, stream, E, rij, pair_i, a, ls,
                     node_spec, S, pair_map, dp, sp, x_from_spec, (float4*)e_u, e_Y, (float4*)e_pk, e_recv,
                     e_dd, E_dev);
  return mm::launch_status("mm_edge_geom_rij");
}

extern "C" int mm_edge_geom_pos(int E, const int* E_dev, const double* pos, const double* box,
                                const int* recv_local, int a, const int* ls, const int* nodes, const int* node_spec,
                                int S, const int* pair_map, const float* dens_w, int nb, float r_max, int p_cut, int M,
                                float r_lo, float inv_h, int x_from_spec, float* e_u, float* e_Y, float* e_pk,
                                int* e_recv, float* e_dd, hipStream_t stream) {
  MM_CHECK_ARG(E >= 0 && S >= 1 && box != nullptr && M >= 2, "bad sizes");
  MMDensity dp;
  MM_CHECK_ARG(make_density(dp, dens_w, nb, r_max, p_cut) == MM_OK, "nb out of range");
  const MMSpline sp{M, r_lo, inv_h};
  if (E == 0) return MM_OK;
  hipLaunchKernelGGL(mm_edge_geom_pos_kernel, dim3((E + 255) / 256), dim3(256), 0, stream, E, pos, box[0], box[1],
                     box[2], recv_local, a, ls, nodes, node_spec, S, pair_map, dp, sp, x_from_spec, (float4*)e_u,
                     e_Y, (float4*)e_pk, e_recv, e_dd, E_dev);
  return mm::launch_status("mm_edge_geom_pos");
}

extern "C" int mm_edge_grad(int E, const int* E_dev, const float* part, long part_stride, int n_part,
                            const float* g_rho, const int* e_recv, const float* e_dd, const float* e_u, float* pf,
                            int accumulate, hipStream_t stream) {
  MM_CHECK_ARG(E >= 0 && n_part >= 0, "bad sizes");
  if (E == 0) return MM_OK;
  hipLaunchKernelGGL(mm_edge_grad_kernel, dim3((E + 255) / 256), dim3(256), 0, stream, E, part, part_stride, n_part,
                     g_rho, e_recv, e_dd, (const float4*)e_u, pf, accumulate, E_dev);
  return mm::launch_status("mm_edge_grad");
}

// Spline tables of the radial weights W(r) = MLP(Bessel(r)) * f_cut(r), sampled in fp64 on the GPU.
//
// Restates the reference's table construction (conv_spline.build_tables, conv_spline.py:230-249, and
// spline_radial._sample, spline_radial.py:116-151): values on a uniform grid of M knots in [r_lo, r_hi] and
// derivatives by central differences with eps = 1e-5 (r_hi - r_lo), all in fp64.  The table consumed by the
// convolution kernels holds, per knot interval k and weight column d, the coefficients of the cubic Hermite
// interpolant written as a polynomial in t = (r - r_k) / h in [0, 1):
//   a0 = V_k, a1 = G_k, a2 = -3 V_k - 2 G_k + 3 V_k+1 - G_k+1, a3 = 2 V_k + G_k - 2 V_k+1 + G_k+1   (G = h dW/dr),
// i.e. the same interpolant as the reference's (TV, TG) Hermite form, rounded to fp32 once per coefficient.
// Layout: float4 coef[cb = d%128/16][tab][k][w = d/128][d%16] so that each XCD's channel block is contiguous.
#include "common.h"

#define MM_MLP_MAXH 128
#define MM_MLP_MAXB 16

// One workgroup per grid point: Bessel features, three hidden layers (silu_n), last layer, cutoff.
__global__ void __launch_bounds__(256) mm_radial_mlp_f64_kernel(int n_pts, const double* __restrict__ r_pts,
                                                                const double* __restrict__ W0,
                                                                const double* __restrict__ W1,
                                                                const double* __restrict__ W2,
                                                                const double* __restrict__ W3, int nb, int H, int D,
                                                                double r_max, int p, double cst,
                                                                double* __restrict__ out) {
  __shared__ double B[MM_MLP_MAXB];
  __shared__ double h[2][MM_MLP_MAXH];
  const int pt = blockIdx.x;
  if (pt >= n_pts) return;
  const double r = r_pts[pt];
  const double pi = 3.14159265358979323846;
  if (threadIdx.x < nb) B[threadIdx.x] = sqrt(2.0 / r_max) * sin((threadIdx.x + 1) * pi * r / r_max) / r;
  __syncthreads();
  if (threadIdx.x < H) {
    double s = 0;
    for (int k = 0; k < nb; ++k) s += B[k] * W0[k * H + threadIdx.x];
    s /= sqrt((double)nb);
    h[0][threadIdx.x] = cst * s / (1.0 + exp(-s));
  }
  __syncthreads();
  const double* Ws[2] = {W1, W2};
  for (int l = 0; l < 2; ++l) {
    if (threadIdx.x < H) {
      double s = 0;
      for (int k = 0; k < H; ++k) s += h[l & 1][k] * Ws[l][k * H + threadIdx.x];
      s /= sqrt((double)H);
      h[(l + 1) & 1][threadIdx.x] = cst * s / (1.0 + exp(-s));
    }
    __syncthreads();
  }
  const double x = r / r_max;
  double f = 0.0;
  if (x < 1.0) {
    const double pp = (double)p;
    f = 1.0 - 0.5 * (pp + 1) * (pp + 2) * pow(x, pp) + pp * (pp + 2) * pow(x, pp + 1) -
        0.5 * pp * (pp + 1) * pow(x, pp + 2);
  }
  const double* hl = h[0];   // after two hidden updates the last activation is in h[0]
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    double s = 0;
    for (int k = 0; k < H; ++k) s += hl[k] * W3[(size_t)k * D + d];
    out[(size_t)pt * D + d] = s / sqrt((double)H) * f;
  }
}

extern "C" int mm_radial_mlp_f64(int n_pts, const double* r_pts, const double* W0, const double* W1,
                                 const double* W2, const double* W3, int nb, int H, int D, double r_max, int p,
                                 double cst, double* out, hipStream_t stream) {
  MM_CHECK_ARG(n_pts >= 0 && nb >= 1 && nb <= MM_MLP_MAXB && H >= 1 && H <= MM_MLP_MAXH && D >= 1, "bad sizes");
  if (n_pts == 0) return MM_OK;
  hipLaunchKernelGGL(mm_radial_mlp_f64_kernel, dim3(n_pts), dim3(256), 0, stream, n_pts, r_pts, W0, W1, W2, W3, nb,
                     H, D, r_max, p, cst, out);
  return mm::launch_status("mm_radial_mlp_f64");
}

// samples [3, M, D]: W(r_k), W(r_k + eps), W(r_k - eps).  Writes the interval coefficients of table `tab`.
__global__ void mm_spline_coeffs_kernel(const double* __restrict__ samples, int M, int nW, double eps, double h,
                                        int tab, int n_tab, float* __restrict__ coef) {
  const int D = nW * MM_C;
  const long idx = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (idx >= (long)(M - 1) * D) return;
  const int k = (int)(idx / D), d = (int)(idx % D);
  const double* V = samples;
  const double* Vp = samples + (size_t)M * D;
  const double* Vm = samples + (size_t)2 * M * D;
  const double v0 = V[(size_t)k * D + d], v1 = V[(size_t)(k + 1) * D + d];
  const double g0 = (Vp[(size_t)k * D + d] - Vm[(size_t)k * D + d]) / (2 * eps) * h;
  const double g1 = (Vp[(size_t)(k + 1) * D + d] - Vm[(size_t)(k + 1) * D + d]) / (2 * eps) * h;
  const double a2 = -3 * v0 - 2 * g0 + 3 * v1 - g1;
  const double a3 = 2 * v0 + g0 - 2 * v1 + g1;
  const int w = d / MM_C, c = d % MM_C, cb = c / MM_CB, cl = c % MM_CB;
  const size_t o = ((((size_t)cb * n_tab + tab) * (M - 1) + k) * nW + w) * MM_CB + cl;
  float* p = coef + 4 * o;
  p[0] = (float)v0;
  p[1] = (float)g0;
  p[2] = (float)a2;
  p[3] = (float)a3;
}

extern "C" int mm_spline_coeffs(const double* samples, int M, int nW, double eps, double h, int tab, int n_tab,
                                float* coef, hipStream_t stream) {
  MM_CHECK_ARG(M >= 2 && nW >= 1 && tab >= 0 && tab < n_tab, "bad sizes");
  const long n = (long)(M - 1) * nW * MM_C;
  hipLaunchKernelGGL(mm_spline_coeffs_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, samples, M,
                     nW, eps, h, tab, n_tab, coef);
  return mm::launch_status("mm_spline_coeffs");
}

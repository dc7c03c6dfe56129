// Shared definitions of the MI355X (gfx950) three-pass MACE library.
//
// Conventions of every extern "C" entry point (declared in include/mace_million_amd.h):
//   * returns 0 on success, a negative MM_E* code on failure; mm_last_error() gives the text of the last failure
//     of the calling thread;
//   * takes device pointers, element counts and a hipStream_t; launches work on that stream; never allocates,
//     never frees, never synchronises (so every entry point can be captured into a hipGraph);
//   * all buffers belong to the caller.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#define MM_OK 0
#define MM_EINVAL -1
#define MM_ELAUNCH -2
#define MM_ERANGE -3

namespace mm {
void set_error(const std::string& msg);
int launch_status(const char* what);   // hipGetLastError() -> status code (records the message)
}  // namespace mm

#define MM_CHECK_ARG(cond, msg)                 \
  do {                                          \
    if (!(cond)) {                              \
      mm::set_error(std::string(__func__) + ": " + (msg)); \
      return MM_EINVAL;                         \
    }                                           \
  } while (0)

// channel count of the model (128 for the MACE-MPA-0 architecture); the generated kernels assume it
#define MM_C 128
// channel blocks: one per XCD of the MI355X (8 XCDs); a block of CB channels stays on one XCD's L2
#define MM_NCB 8
#define MM_CB 16

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int mm_xcd_channel_block() {
  // workgroups are dispatched round-robin over the 8 XCDs: blockIdx.x % 8 selects the XCD, and with it the
  // channel block whose table slice that XCD keeps in its L2
  return blockIdx.x & (MM_NCB - 1);
}

// dx/dr of an edge's spline coordinate x = (r - r_lo) / h: inv_h inside the table; zero for a length below the
// table start, which the geometry kernels mark with t = -0 (x clamped to 0, so W is W(r_lo) and does not vary with
// r there: a zero derivative keeps the forces the derivative of the energy that the forward evaluates).
__device__ __forceinline__ float mm_spline_dxdr(float t, float inv_h) {
  return __float_as_int(t) < 0 ? 0.f : inv_h;
}

// DPP (data-parallel primitive) lane moves inside a row of 16 lanes; used for channel reductions without LDS.
template <int CTRL>
__device__ __forceinline__ float mm_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the (bitwise identical) sum.
__device__ __forceinline__ float mm_row_sum16(float v) {
  v += mm_dpp<0xB1>(v);    // quad_perm [1, 0, 3, 2]: pairs within a quad
  v += mm_dpp<0x4E>(v);    // quad_perm [2, 3, 0, 1]: quad sums
  v += mm_dpp<0x141>(v);   // row_half_mirror: lane i <- 7 - i within each 8-lane half: 8-lane sums
  v += mm_dpp<0x140>(v);   // row_mirror: lane i <- 15 - i: 16-lane sums
  return v;
}

// Orders the LDS accesses of the lanes of one wave: what a lane wrote before the call is seen by every lane's reads
// after it.  One wave's LDS instructions execute in program order; the fences keep the compiler from moving
// accesses across the call (no s_barrier: the lanes of other waves are not waited for).
__device__ __forceinline__ void mm_wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Four float adds to LDS (p[0], p[16], p[32], p[48]) through 32-bit compare-and-swap, issued together; a lane
// repeats only the adds whose swap lost a race.  The native LDS float atomic add (ds_add_f32) runs far below
// the integer LDS atomics on this GPU (measured), so float sums shared by the waves of a workgroup use this.
__device__ __forceinline__ void mm_lds_add4_f32(float* p, float v0, float v1, float v2, float v3) {
  unsigned* u = (unsigned*)p;
  unsigned a0 = u[0], a1 = u[16], a2 = u[32], a3 = u[48];
  unsigned r0 = atomicCAS(u, a0, __float_as_uint(__uint_as_float(a0) + v0));
  unsigned r1 = atomicCAS(u + 16, a1, __float_as_uint(__uint_as_float(a1) + v1));
  unsigned r2 = atomicCAS(u + 32, a2, __float_as_uint(__uint_as_float(a2) + v2));
  unsigned r3 = atomicCAS(u + 48, a3, __float_as_uint(__uint_as_float(a3) + v3));
  while (r0 != a0) { a0 = r0; r0 = atomicCAS(u, a0, __float_as_uint(__uint_as_float(a0) + v0)); }
  while (r1 != a1) { a1 = r1; r1 = atomicCAS(u + 16, a1, __float_as_uint(__uint_as_float(a1) + v1)); }
  while (r2 != a2) { a2 = r2; r2 = atomicCAS(u + 32, a2, __float_as_uint(__uint_as_float(a2) + v2)); }
  while (r3 != a3) { a3 = r3; r3 = atomicCAS(u + 48, a3, __float_as_uint(__uint_as_float(a3) + v3)); }
}

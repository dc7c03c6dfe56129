// Library-wide entry points: error reporting and version.
#include "common.h"

#include <cstring>

namespace {
thread_local std::string g_last_error;
}

namespace mm {
void set_error(const std::string& msg) { g_last_error = msg; }

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return MM_ELAUNCH;
  }
  return MM_OK;
}
}  // namespace mm

extern "C" const char* mm_last_error(void) { return g_last_error.c_str(); }

// Version of the argument conventions; the host binding refuses a library of another version (an older library
// given the buffers of a newer host reads them with the wrong layout).  2: mm_linear weight blocks as three bf16
// planes.  3: mm_ace1_fwd / mm_ace1_bwd take the edge vectors (unit vector, r) instead of stored harmonics.
// 4: the edge-geometry and edge-gradient entry points take a device edge count.  5: mm_ace1_bwd reads gB in its
// MFMA operand order.  6: the mm_tpw_*_bwd kernels write one dL/dY partial per channel half (1 or 2), not 8.
// 7: mm_conv2_bwd / mm_conv2_bwd_det write dL/dX in 16-channel-block-major rows; mm_linear takes in_cb.
extern "C" int mm_version(void) { return 7; }

// Channel count and channel-block geometry the generated kernels were built for.
extern "C" int mm_build_info(int* channels, int* channel_blocks, int* block_channels) {
  if (channels) *channels = MM_C;
  if (channel_blocks) *channel_blocks = MM_NCB;
  if (block_channels) *block_channels = MM_CB;
  return MM_OK;
}

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

extern "C" int mm_version(void) { return 1; }

// Channel count and channel-block geometry the generated kernels were built for.
extern "C" int mm_build_info(int* channels, int* channel_blocks, int* block_channels) {
  if (channels) *channels = MM_C;
  if (channel_blocks) *channel_blocks = MM_NCB;
  if (block_channels) *block_channels = MM_CB;
  return MM_OK;
}

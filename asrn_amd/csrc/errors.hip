// Error reporting shared by every entry point: a thread-local last message.
#include "common.h"

namespace asrn {

static thread_local char g_msg[1024] = "";

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return 1;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

}  // namespace asrn

extern "C" const char* asrn_hip_last_error(void) { return asrn::g_msg; }
extern "C" int32_t asrn_hip_abi_version(void) { return 2; }

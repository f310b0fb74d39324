// Error slot, version and workspace sizing of the C ABI (include/loopsgl_tok.h).
#include <stdarg.h>
#include <stdio.h>

#include "lsg_capi_internal.h"

namespace lsg {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(LSG_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return LSG_OK;
}

}  // namespace lsg

extern "C" const char* lsg_last_error(void) { return lsg::g_err; }

extern "C" int lsg_version(void) { return 1; }

// Exit-compaction workspace: the call serial number and an error flag (padded
// to 256 B), then one 64-bit published count per workgroup of four rows (padded
// to 256 B).
extern "C" size_t lsg_workspace_bytes(int op, int64_t B) {
  if ((op != LSG_OP_EXIT_GATE && op != LSG_OP_REL_CHANGE) || B < 0) return 0;
  const size_t tiles = B > 0 ? (size_t)((B + 3) / 4) : 1;  // an empty batch still launches one workgroup
  return 256 + ((tiles * 8 + 255) / 256) * 256;
}

// Library-wide C-ABI plumbing: version, last-error reporting.
#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

static thread_local char g_last_error[512] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

}  // namespace hc

extern "C" const char* hc_last_error(void) { return hc::g_last_error; }

extern "C" int hc_version(void) { return HC_ABI_VERSION; }

extern "C" int hc_tile_tokens(void) { return HC_TILE; }

extern "C" int hc_head_dim(void) { return HC_HEAD_DIM; }

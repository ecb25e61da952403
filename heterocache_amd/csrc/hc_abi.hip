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

extern "C" int hc_read_status(int32_t* status, int clear, int32_t* value, void* stream) {
  hc::clear_error();
  if (!status) return hc::set_error(HC_ERR_INVALID, "hc_read_status: null status");
  hipStream_t s = (hipStream_t)stream;
  int32_t word = 0;
  if (hipMemcpyAsync(&word, status, sizeof(word), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return hc::set_error(HC_ERR_HIP, "hc_read_status: %s", hipGetErrorString(hipGetLastError()));
  if (value) *value = word;
  if (clear && word != 0) {
    static const int32_t zero = 0;
    if (hipMemcpyAsync(status, &zero, sizeof(zero), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return hc::set_error(HC_ERR_HIP, "hc_read_status: %s", hipGetErrorString(hipGetLastError()));
  }
  if (word & 1) return hc::set_error(HC_ERR_CAPACITY, "a row was at capacity when a token was appended (status 0x%x)", word);
  return HC_OK;
}

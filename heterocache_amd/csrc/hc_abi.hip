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

namespace hc {

// Streaming-read ceiling of the device, the yardstick of the HBM-bound
// kernels: every thread sums 16-byte nontemporal loads in a grid-stride
// loop, one load in flight per thread and many waves per SIMD (the shape
// that read fastest among 1-8 loads per thread and 2-16 workgroups per CU).
// The sink is written only when the sum equals one arbitrary value (never,
// for the zero-filled buffer the bench passes), so the loads are kept.
__global__ __launch_bounds__(256) void stream_read_kernel(const f32x4* __restrict__ p, size_t n,
                                                          float* __restrict__ sink) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) acc += __builtin_nontemporal_load(p + i);
  const float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  if (s == -1.2345e-37f) sink[0] = s;
}

}  // namespace hc

extern "C" int hc_stream_read(const void* src, size_t bytes, float* sink, int workgroups_per_cu, void* stream) {
  hc::clear_error();
  if (!src || !sink || bytes < 16 || (bytes % 16) != 0 || (reinterpret_cast<uintptr_t>(src) % 16) != 0)
    return hc::set_error(HC_ERR_INVALID, "hc_stream_read: need a 16-byte aligned buffer of a multiple of 16 bytes");
  if (workgroups_per_cu < 1 || workgroups_per_cu > 64)
    return hc::set_error(HC_ERR_INVALID, "hc_stream_read: workgroups_per_cu=%d (1..64)", workgroups_per_cu);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return hc::set_error(HC_ERR_HIP, "hc_stream_read: device query failed");
  hipLaunchKernelGGL(hc::stream_read_kernel, dim3((unsigned)(cus * workgroups_per_cu)), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const hc::f32x4*>(src), bytes / 16, sink);
  return hc::check_launch("hc_stream_read");
}

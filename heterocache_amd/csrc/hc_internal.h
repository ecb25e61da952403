// Host-side helpers shared by the C-ABI entry points: status codes, the
// thread-local last-error message and launch checking.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "hc.h"

namespace hc {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(HC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return HC_OK;
}

size_t decode_workspace_bytes_rows(int rows, int group, int64_t num_parts);
int64_t decode_num_parts(const int* host_row_len, int rows, int chunk_tiles);

}  // namespace hc

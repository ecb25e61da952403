// Head-analysis pooling: the per-head attention vectors from which the
// head-classification JSON is built (tools/get_cluster.py:13-56).
//
//   out[b*Hout + h][t] = avg_pool_k( mean_{g<group} attn[b, h*group + g, t] ),  t < span
//
// Zero padding of kernel/2 on both sides with divisor `kernel`
// (F.avg_pool1d, count_include_pad).  With 16-bit inputs the group mean is
// rounded to the input type first, as the reference's torch.mean on the
// saved tensor leaves it.  One thread per output position; the work is a
// few MB per layer, latency-bound.
#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

template <typename T>
__global__ __launch_bounds__(256) void head_pool_kernel(const T* __restrict__ attn, int64_t batch_stride,
                                                        int64_t head_stride, int heads_out, int group, int span,
                                                        int kernel, float* __restrict__ out) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int job = blockIdx.y;  // b * heads_out + h
  if (t >= span) return;
  const int b = job / heads_out, h = job % heads_out;
  const T* base = attn + b * batch_stride + (int64_t)h * group * head_stride;
  const int p = kernel / 2;
  float acc = 0.f;
  for (int d = -p; d <= p; ++d) {
    const int u = t + d;
    if (u < 0 || u >= span) continue;
    float m = 0.f;
    for (int g = 0; g < group; ++g) m += Elem<T>::to_f32(base[g * head_stride + u]);
    m /= (float)group;
    if constexpr (sizeof(T) == 2) m = Elem<T>::to_f32(Elem<T>::from_f32(m));
    acc += m;
  }
  out[(int64_t)job * span + t] = acc / (float)kernel;
}

}  // namespace hc

using namespace hc;

extern "C" int hc_head_pool(int dtype, const void* attn, int64_t batch_stride, int64_t head_stride, int batch,
                            int heads_out, int group, int span, int kernel, float* out, void* stream) {
  clear_error();
  if (dtype != HC_DTYPE_F32 && dtype != HC_DTYPE_BF16 && dtype != HC_DTYPE_F16)
    return set_error(HC_ERR_INVALID, "hc_head_pool: unknown dtype %d", dtype);
  if (batch < 0 || heads_out < 0 || group < 1 || span < 0 || kernel < 1 || (kernel & 1) == 0)
    return set_error(HC_ERR_INVALID, "hc_head_pool: batch=%d heads_out=%d group=%d span=%d kernel=%d", batch,
                     heads_out, group, span, kernel);
  if (batch == 0 || heads_out == 0 || span == 0) return HC_OK;
  if (!attn || !out) return set_error(HC_ERR_INVALID, "hc_head_pool: null pointer argument");
  if ((int64_t)batch * heads_out > 65535) return set_error(HC_ERR_INVALID, "hc_head_pool: too many rows");
  const dim3 grid((span + 255) / 256, batch * heads_out);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case HC_DTYPE_F32:
      hipLaunchKernelGGL(head_pool_kernel<float>, grid, dim3(256), 0, s, (const float*)attn, batch_stride,
                         head_stride, heads_out, group, span, kernel, out);
      break;
    case HC_DTYPE_BF16:
      hipLaunchKernelGGL(head_pool_kernel<__bf16>, grid, dim3(256), 0, s, (const __bf16*)attn, batch_stride,
                         head_stride, heads_out, group, span, kernel, out);
      break;
    default:
      hipLaunchKernelGGL(head_pool_kernel<_Float16>, grid, dim3(256), 0, s, (const _Float16*)attn, batch_stride,
                         head_stride, heads_out, group, span, kernel, out);
  }
  return check_launch("hc_head_pool");
}

// RMSNorm of the hybrid stack around the Bolt-3 layers (block norms, final norm, q/k norms of
// the softmax-anchor layers): y = (x * rsqrt(mean(x^2) + eps)) * w, fp32 statistic, each product
// rounded in fp32, the result cast to the storage dtype once (vsa_lm/surgery.py:48-52).  One
// wavefront per row, 8 elements per 16-byte load; four rows per 256-thread workgroup.
#include "bolt3_common.h"
#include "bolt3_amd.h"

namespace b3 {

template <typename T, typename W>
__global__ void __launch_bounds__(256) rms_norm_kernel(b3_rms_norm_args a) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;   // whole wavefronts; no barrier below
  const T* x = reinterpret_cast<const T*>(a.x) + row * a.x_row_stride;
  T* y = reinterpret_cast<T*>(a.y) + row * a.y_row_stride;
  const W* w = reinterpret_cast<const W*>(a.w);
  const int n8 = a.dim / 8;
  float ss = 0.f;
  for (int i = lane; i < n8; i += 64) {
    Vec8<T> v;
    v.load(x + 8 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = v.get(e);
      ss += f * f;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float r = 1.0f / sqrtf(div_rn(ss, (float)a.dim) + a.eps);
  for (int i = lane; i < n8; i += 64) {
    Vec8<T> v;
    v.load(x + 8 * i);
    Vec8<T> o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.set(e, mul_rn(mul_rn(v.get(e), r), St<W>::ld(w + 8 * i + e)));
    o.store(y + 8 * i);
  }
}

template <typename T>
static int launch_rms(const b3_rms_norm_args& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  if (a.w_dtype == B3_F32) hipLaunchKernelGGL((rms_norm_kernel<T, float>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((rms_norm_kernel<T, uint16_t>), grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int bolt3_rms_norm(const b3_rms_norm_args* a, void* stream) {
  if (!a || a->rows < 0 || a->dim <= 0 || a->dim % 8 || !a->x || !a->w || !a->y) return B3_ERR_ARG;
  if ((a->dtype != B3_F32 && a->dtype != B3_BF16) || (a->w_dtype != B3_F32 && a->w_dtype != B3_BF16))
    return B3_ERR_UNSUPPORTED;
  const int64_t es = a->dtype == B3_BF16 ? 2 : 4;
  if (a->x_row_stride < a->dim || a->y_row_stride < a->dim || (a->x_row_stride * es) % 16 ||
      (a->y_row_stride * es) % 16 || reinterpret_cast<uintptr_t>(a->x) % 16 || reinterpret_cast<uintptr_t>(a->y) % 16)
    return B3_ERR_ARG;
  if (a->rows == 0) return 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return a->dtype == B3_BF16 ? b3::launch_rms<uint16_t>(*a, st) : b3::launch_rms<float>(*a, st);
}

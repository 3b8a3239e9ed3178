// Backward of Bolt3Attn's head preparation (the inverse direction of heads_kernel), one pass over
// the token rows: RoPE transposes, the q / k RMSNorm backward, the gates' derivatives, and the
// packed gradient dz of the projection output [q | k | v | beta | eta | pad] in the storage
// dtype.  Replaces the autograd of vsa_lm/config/bolt3.py:196-215 (projections' outputs through
// the norms, RoPE and gates) and vsa_lm/surgery.py:48-52, :86-93.
//
// One workgroup of four wavefronts takes RPB token rows; a wavefront takes four heads of a row at
// a time (all their loads issued before the first sum), lane j holding the RoPE pair (j, j + HD/2),
// so the rotation's transpose is lane-local and the norm statistics are wavefront sums.
#include <math.h>

#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {
namespace hbwd {

constexpr int NT = 256;
constexpr int RPB = 2;     // token rows per workgroup (more workgroups in flight beat longer ones)

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// norm backward of one head row: y = x * rsqrt(mean(x^2) + eps) * w; g = dL/dy at features
// (j, j + half); returns dL/dx in g and adds dL/dw to dw
__device__ __forceinline__ void rms_bwd_pair(float& g0, float& g1, float x0, float x1, float w0, float w1, float eps,
                                             int hd, float& dw0, float& dw1) {
  const float ss = wsum(x0 * x0 + x1 * x1);
  const float r = 1.0f / sqrtf(ss / (float)hd + eps);
  const float gw0 = g0 * w0, gw1 = g1 * w1;
  const float m = wsum(gw0 * x0 + gw1 * x1) / (float)hd;
  dw0 += g0 * x0 * r;
  dw1 += g1 * x1 * r;
  const float r3 = r * r * r;
  g0 = r * gw0 - x0 * r3 * m;
  g1 = r * gw1 - x1 * r3 * m;
}

template <typename T>
__global__ void __launch_bounds__(NT) heads_bwd_kernel(b3_heads_bwd_args a) {
  __shared__ float red[2][4][128];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int HD = a.HD, half = HD / 2, H = a.H, HKV = a.HKV;
  const bool on = lane < half;
  const int j = on ? lane : 0;
  const float invf = a.inv_freq[j];
  const float qw0 = a.has_qk_norm ? a.qn_w[j] : 0.f, qw1 = a.has_qk_norm ? a.qn_w[j + half] : 0.f;
  const float kw0 = a.has_qk_norm ? a.kn_w[j] : 0.f, kw1 = a.has_qk_norm ? a.kn_w[j + half] : 0.f;
  float dqw0 = 0.f, dqw1 = 0.f, dkw0 = 0.f, dkw1 = 0.f;
  const long long BT = (long long)a.B * a.T;
  const long long BH = (long long)a.B * HKV;
  for (int rr = 0; rr < RPB; ++rr) {
    const long long row = (long long)blockIdx.x * RPB + rr;
    if (row >= BT) break;
    const int b = (int)(row / a.T), t = (int)(row % a.T);
    T* dz = reinterpret_cast<T*>(a.dz) + row * a.dz_row_stride;
    float sn, cs;
    sincos_rope((float)t * invf, &sn, &cs);   // the forward RoPE's own values
    // query heads u = w + 4 i, four at a time: every load of the four first, then the sums
    for (int i0 = 0; i0 < H; i0 += 16) {
      float q0[4], q1[4], r0[4], r1[4], x0[4], x1[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int u = i0 + w + 4 * k;
        const bool ok = on && u < H;
        const long long base = (((long long)b * H + min(u, H - 1)) * a.T + t) * HD;
        q0[k] = ok ? a.d_q_raw[base + j] : 0.f;
        q1[k] = ok ? a.d_q_raw[base + j + half] : 0.f;
        r0[k] = ok ? a.d_q_rope[base + j] : 0.f;
        r1[k] = ok ? a.d_q_rope[base + j + half] : 0.f;
        x0[k] = x1[k] = 0.f;
        if (a.has_qk_norm && ok) {
          const T* lq = reinterpret_cast<const T*>(a.lin_q) + row * a.lin_q_row_stride + (long long)u * HD;
          x0[k] = St<T>::ld(lq + j);
          x1[k] = St<T>::ld(lq + j + half);
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int u = i0 + w + 4 * k;
        if (u >= H) break;   // uniform over the wavefront
        float g0 = q0[k] + (r0[k] * cs + r1[k] * sn), g1 = q1[k] + (r1[k] * cs - r0[k] * sn);
        if (a.has_qk_norm) rms_bwd_pair(g0, g1, x0[k], x1[k], qw0, qw1, a.q_eps, HD, dqw0, dqw1);
        if (on) {
          dz[(long long)u * HD + j] = St<T>::from_f(g0);
          dz[(long long)u * HD + j + half] = St<T>::from_f(g1);
        }
      }
    }
    // kv heads hk = w + 4 i, four at a time: keys, then values
    for (int i0 = 0; i0 < HKV; i0 += 16) {
      float k0[4], k1[4], c0[4], c1[4], x0[4], x1[4], v0[4], v1[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int hk = i0 + w + 4 * k;
        const bool ok = on && hk < HKV;
        const long long bh = (long long)b * HKV + min(hk, HKV - 1);
        const long long base = (bh * a.T + t) * HD;
        k0[k] = ok ? a.d_k_own[base + j] + a.d_k_next[base + j] : 0.f;
        k1[k] = ok ? a.d_k_own[base + j + half] + a.d_k_next[base + j + half] : 0.f;
        v0[k] = ok ? a.d_v_own[base + j] + a.d_v_next[base + j] : 0.f;
        v1[k] = ok ? a.d_v_own[base + j + half] + a.d_v_next[base + j + half] : 0.f;
        if (ok && a.d_sink_k && t < a.n_sinks)
          for (int cc = 0; cc < a.n_chunks; ++cc) {
            const long long sb = (((long long)cc * BH + bh) * a.n_sinks + t) * HD;
            k0[k] += a.d_sink_k[sb + j];
            k1[k] += a.d_sink_k[sb + j + half];
            v0[k] += a.d_sink_v[sb + j];
            v1[k] += a.d_sink_v[sb + j + half];
          }
        c0[k] = c1[k] = 0.f;
        if (ok && a.d_k_chain) {
          c0[k] = a.d_k_chain[base + j];
          c1[k] = a.d_k_chain[base + j + half];
          v0[k] += a.d_v_chain[base + j];
          v1[k] += a.d_v_chain[base + j + half];
        }
        x0[k] = x1[k] = 0.f;
        if (a.has_qk_norm && ok) {
          const T* lk = reinterpret_cast<const T*>(a.lin_k) + row * a.lin_k_row_stride + (long long)hk * HD;
          x0[k] = St<T>::ld(lk + j);
          x1[k] = St<T>::ld(lk + j + half);
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int hk = i0 + w + 4 * k;
        if (hk >= HKV) break;   // uniform over the wavefront
        float g0 = c0[k] + (k0[k] * cs + k1[k] * sn), g1 = c1[k] + (k1[k] * cs - k0[k] * sn);
        if (a.has_qk_norm) rms_bwd_pair(g0, g1, x0[k], x1[k], kw0, kw1, a.k_eps, HD, dkw0, dkw1);
        if (on) {
          dz[(long long)(H + hk) * HD + j] = St<T>::from_f(g0);
          dz[(long long)(H + hk) * HD + j + half] = St<T>::from_f(g1);
          dz[(long long)(H + HKV + hk) * HD + j] = St<T>::from_f(v0[k]);
          dz[(long long)(H + HKV + hk) * HD + j + half] = St<T>::from_f(v1[k]);
        }
      }
    }
    // gates and the zero pad
    const int g_off = (H + 2 * HKV) * HD;
    for (int c = tid; c < a.dz_cols - g_off; c += NT) {
      float v = 0.f;
      if (c < HKV) {
        const long long bh = (long long)b * HKV + c;
        const float bt = a.beta[bh * a.T + t];
        v = a.d_beta ? a.d_beta[bh * a.T + t] * bt * (1.0f - bt) : 0.f;
      } else if (c < HKV + H) {
        const long long i = ((long long)b * H + (c - HKV)) * a.T + t;
        const float e = a.eta[i];
        v = a.d_eta[i] * (1.0f - e * e);
      }
      dz[g_off + c] = St<T>::from_f(v);
    }
  }
  if (!a.has_qk_norm) return;
  if (on) {
    red[0][w][j] = dqw0;
    red[0][w][j + half] = dqw1;
    red[1][w][j] = dkw0;
    red[1][w][j + half] = dkw1;
  }
  __syncthreads();
  if (tid < HD) {
    a.d_qn_w[(long long)blockIdx.x * HD + tid] = red[0][0][tid] + red[0][1][tid] + red[0][2][tid] + red[0][3][tid];
    a.d_kn_w[(long long)blockIdx.x * HD + tid] = red[1][0][tid] + red[1][1][tid] + red[1][2][tid] + red[1][3][tid];
  }
}

}  // namespace hbwd
}  // namespace b3

extern "C" int32_t bolt3_heads_bwd_blocks(int32_t B, int32_t T) {
  if (B <= 0 || T <= 0) return 0;
  return (int32_t)(((long long)B * T + b3::hbwd::RPB - 1) / b3::hbwd::RPB);
}

extern "C" int bolt3_heads_bwd(const b3_heads_bwd_args* a, void* stream) {
  if (!a) return B3_ERR_ARG;
  if (a->dtype != B3_F32 && a->dtype != B3_BF16) return B3_ERR_UNSUPPORTED;
  if (a->HD != 64 && a->HD != 128) return B3_ERR_UNSUPPORTED;
  if (a->B <= 0 || a->T <= 0 || a->H <= 0 || a->HKV <= 0 || a->H % a->HKV || a->n_sinks < 0 || a->n_chunks < 0)
    return B3_ERR_ARG;
  const long long need = (long long)(a->H + 2 * a->HKV) * a->HD + a->HKV + a->H;
  if (a->dz_cols < need || a->dz_row_stride < a->dz_cols) return B3_ERR_ARG;
  if (!a->d_q_raw || !a->d_q_rope || !a->d_k_own || !a->d_k_next || !a->d_v_own || !a->d_v_next || !a->d_eta ||
      !a->beta || !a->eta || !a->inv_freq || !a->dz)
    return B3_ERR_ARG;
  if ((a->d_sink_k || a->d_sink_v) && (!a->d_sink_k || !a->d_sink_v || a->n_chunks <= 0 || a->n_sinks <= 0))
    return B3_ERR_ARG;
  if (a->has_qk_norm && (!a->lin_q || !a->lin_k || !a->qn_w || !a->kn_w || !a->d_qn_w || !a->d_kn_w ||
                         a->lin_q_row_stride < (long long)a->H * a->HD || a->lin_k_row_stride < (long long)a->HKV * a->HD))
    return B3_ERR_ARG;
  const int nb = bolt3_heads_bwd_blocks(a->B, a->T);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_BF16)
    hipLaunchKernelGGL(b3::hbwd::heads_bwd_kernel<uint16_t>, dim3(nb), dim3(b3::hbwd::NT), 0, st, *a);
  else
    hipLaunchKernelGGL(b3::hbwd::heads_bwd_kernel<float>, dim3(nb), dim3(b3::hbwd::NT), 0, st, *a);
  return (int)hipGetLastError();
}

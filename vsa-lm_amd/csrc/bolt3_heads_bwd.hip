// Backward of Bolt3Attn's head preparation (the inverse direction of heads_kernel), one pass over
// the token rows: RoPE transposes, the q / k RMSNorm backward, the gates' derivatives, and the
// packed gradient dz of the projection output [q | k | v | beta | eta | pad] in the storage
// dtype.  Replaces the autograd of vsa_lm/config/bolt3.py:196-215 (projections' outputs through
// the norms, RoPE and gates) and vsa_lm/surgery.py:48-52, :86-93.
//
// One workgroup of four wavefronts takes RPB token rows.  A head row is LPH = HD/8 lanes: lane e
// of a head holds features 4e .. 4e+3 and their RoPE partners HD/2 + 4e .., so the rotation's
// transpose is lane-local, every load and store moves four elements, and the norm statistics
// are sums over the head's lanes; a wavefront takes 64/LPH heads of a row at a time.
#include <math.h>

#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {
namespace hbwd {

constexpr int NT = 256;
constexpr int RPB = 2;     // token rows per workgroup (more workgroups in flight beat longer ones)

// four consecutive elements as floats / from floats (8-byte bf16 or 16-byte fp32 accesses)
__device__ __forceinline__ void ld4v(const uint16_t* p, float* o) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  o[0] = bf_lo(v.x); o[1] = bf_hi(v.x); o[2] = bf_lo(v.y); o[3] = bf_hi(v.y);
}
__device__ __forceinline__ void ld4v(const float* p, float* o) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
__device__ __forceinline__ void st4v(uint16_t* p, const float* v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
}
__device__ __forceinline__ void st4v(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void zero4(float* v) { v[0] = v[1] = v[2] = v[3] = 0.f; }

// sum over the L lanes of a head (aligned groups of L lanes)
template <int L>
__device__ __forceinline__ float gsum(float v) {
#pragma unroll
  for (int o = L / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// norm backward of one head row: y = x * rsqrt(mean(x^2) + eps) * w; g = dL/dy at this lane's
// features (4e.., HD/2 + 4e..); returns dL/dx in g and adds dL/dw to dw
template <int HD>
__device__ __forceinline__ void rms_bwd4(float* g0, float* g1, const float* x0, const float* x1, const float* w0,
                                         const float* w1, float eps, float* dw0, float* dw1) {
  constexpr int LPH = HD / 8;
  float ss = 0.f, m = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += x0[i] * x0[i] + x1[i] * x1[i];
  ss = gsum<LPH>(ss);
  const float r = 1.0f / sqrtf(ss / (float)HD + eps);
  float gw0[4], gw1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    gw0[i] = g0[i] * w0[i];
    gw1[i] = g1[i] * w1[i];
    m += gw0[i] * x0[i] + gw1[i] * x1[i];
  }
  m = gsum<LPH>(m) / (float)HD;
  const float r3 = r * r * r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dw0[i] += g0[i] * x0[i] * r;
    dw1[i] += g1[i] * x1[i] * r;
    g0[i] = r * gw0[i] - x0[i] * r3 * m;
    g1[i] = r * gw1[i] - x1[i] * r3 * m;
  }
}

template <typename T, int HD>
__global__ void __launch_bounds__(NT) heads_bwd_kernel(b3_heads_bwd_args a) {
  constexpr int HALF = HD / 2, LPH = HD / 8, HPW = 64 / LPH, HPB = 4 * HPW;   // heads per wavefront, workgroup
  __shared__ float red[2][4][HD];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int hl = lane / LPH, j = 4 * (lane % LPH);   // head slot of the lane; features j.., HALF + j..
  const int H = a.H, HKV = a.HKV;
  float invf[4], qw0[4], qw1[4], kw0[4], kw1[4];
  float dqw0[4], dqw1[4], dkw0[4], dkw1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    invf[i] = a.inv_freq[j + i];
    qw0[i] = a.has_qk_norm ? a.qn_w[j + i] : 0.f;
    qw1[i] = a.has_qk_norm ? a.qn_w[HALF + j + i] : 0.f;
    kw0[i] = a.has_qk_norm ? a.kn_w[j + i] : 0.f;
    kw1[i] = a.has_qk_norm ? a.kn_w[HALF + j + i] : 0.f;
    dqw0[i] = dqw1[i] = dkw0[i] = dkw1[i] = 0.f;
  }
  const long long BT = (long long)a.B * a.T;
  const long long BH = (long long)a.B * HKV;
  // the attention's row gradients, in the storage dtype
  const T* g_q_raw = static_cast<const T*>(a.d_q_raw);
  const T* g_q_rope = static_cast<const T*>(a.d_q_rope);
  const T* g_k_own = static_cast<const T*>(a.d_k_own);
  const T* g_k_next = static_cast<const T*>(a.d_k_next);
  const T* g_v_own = static_cast<const T*>(a.d_v_own);
  const T* g_v_next = static_cast<const T*>(a.d_v_next);
  const bool do_q = a.parts != 2, do_kv = a.parts != 1;
  for (int rr = 0; rr < RPB; ++rr) {
    const long long row = (long long)blockIdx.x * RPB + rr;
    if (row >= BT) break;
    const int b = (int)(row / a.T), t = (int)(row % a.T);
    T* dz = reinterpret_cast<T*>(a.dz) + row * a.dz_row_stride;
    float sn[4], cs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sincos_rope((float)t * invf[i], &sn[i], &cs[i]);   // the forward RoPE's own values
    // query heads u = i0 + HPW w + hl: every load first, then the sums
    for (int i0 = 0; i0 < (do_q ? H : 0); i0 += HPB) {
      const int u = i0 + HPW * w + hl;
      const bool ok = u < H;
      const long long base = (((long long)b * H + min(u, H - 1)) * a.T + t) * HD;
      float q0[4], q1[4], r0[4], r1[4], x0[4], x1[4];
      zero4(q0); zero4(q1); zero4(r0); zero4(r1); zero4(x0); zero4(x1);
      if (ok) {
        ld4v(g_q_raw + base + j, q0);
        ld4v(g_q_raw + base + HALF + j, q1);
        ld4v(g_q_rope + base + j, r0);
        ld4v(g_q_rope + base + HALF + j, r1);
        if (a.has_qk_norm) {
          const T* lq = reinterpret_cast<const T*>(a.lin_q) + row * a.lin_q_row_stride + (long long)u * HD;
          ld4v(lq + j, x0);
          ld4v(lq + HALF + j, x1);
        }
      }
      float g0[4], g1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g0[i] = q0[i] + (r0[i] * cs[i] + r1[i] * sn[i]);
        g1[i] = q1[i] + (r1[i] * cs[i] - r0[i] * sn[i]);
      }
      if (a.has_qk_norm) rms_bwd4<HD>(g0, g1, x0, x1, qw0, qw1, a.q_eps, dqw0, dqw1);
      if (ok) {
        st4v(dz + (long long)u * HD + j, g0);
        st4v(dz + (long long)u * HD + HALF + j, g1);
      }
    }
    // kv heads hk = i0 + HPW w + hl: keys (own + next chunk + sinks, the chain's gradient of the
    // un-roped keys, the norm) and values
    for (int i0 = 0; i0 < (do_kv ? HKV : 0); i0 += HPB) {
      const int hk = i0 + HPW * w + hl;
      const bool ok = hk < HKV;
      const long long bh = (long long)b * HKV + min(hk, HKV - 1);
      const long long base = (bh * a.T + t) * HD;
      float k0[4], k1[4], c0[4], c1[4], x0[4], x1[4], v0[4], v1[4];
      zero4(k0); zero4(k1); zero4(c0); zero4(c1); zero4(x0); zero4(x1); zero4(v0); zero4(v1);
      if (ok) {
        float p0[4], p1[4], n0[4], n1[4];
        ld4v(g_k_own + base + j, k0);
        ld4v(g_k_own + base + HALF + j, k1);
        ld4v(g_k_next + base + j, n0);
        ld4v(g_k_next + base + HALF + j, n1);
        ld4v(g_v_own + base + j, v0);
        ld4v(g_v_own + base + HALF + j, v1);
        ld4v(g_v_next + base + j, p0);
        ld4v(g_v_next + base + HALF + j, p1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          k0[i] += n0[i];
          k1[i] += n1[i];
          v0[i] += p0[i];
          v1[i] += p1[i];
        }
        if (a.d_sink_k && t < a.n_sinks)
          for (int cc = 0; cc < a.n_chunks; ++cc) {
            const long long sb = (((long long)cc * BH + bh) * a.n_sinks + t) * HD;
            float s0[4], s1[4], s2[4], s3[4];
            ld4v(a.d_sink_k + sb + j, s0);
            ld4v(a.d_sink_k + sb + HALF + j, s1);
            ld4v(a.d_sink_v + sb + j, s2);
            ld4v(a.d_sink_v + sb + HALF + j, s3);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              k0[i] += s0[i];
              k1[i] += s1[i];
              v0[i] += s2[i];
              v1[i] += s3[i];
            }
          }
        if (a.d_k_chain) {
          float s2[4], s3[4];
          ld4v(a.d_k_chain + base + j, c0);
          ld4v(a.d_k_chain + base + HALF + j, c1);
          ld4v(a.d_v_chain + base + j, s2);
          ld4v(a.d_v_chain + base + HALF + j, s3);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v0[i] += s2[i];
            v1[i] += s3[i];
          }
        }
        if (a.has_qk_norm) {
          const T* lk = reinterpret_cast<const T*>(a.lin_k) + row * a.lin_k_row_stride + (long long)hk * HD;
          ld4v(lk + j, x0);
          ld4v(lk + HALF + j, x1);
        }
      }
      float g0[4], g1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g0[i] = c0[i] + (k0[i] * cs[i] + k1[i] * sn[i]);
        g1[i] = c1[i] + (k1[i] * cs[i] - k0[i] * sn[i]);
      }
      if (a.has_qk_norm) rms_bwd4<HD>(g0, g1, x0, x1, kw0, kw1, a.k_eps, dkw0, dkw1);
      if (ok) {
        st4v(dz + (long long)(H + hk) * HD + j, g0);
        st4v(dz + (long long)(H + hk) * HD + HALF + j, g1);
        st4v(dz + (long long)(H + HKV + hk) * HD + j, v0);
        st4v(dz + (long long)(H + HKV + hk) * HD + HALF + j, v1);
      }
    }
    // gates and the zero pad (part 1: the eta columns; part 2: beta and the pad)
    const int g_off = (H + 2 * HKV) * HD;
    for (int c = tid; c < a.dz_cols - g_off; c += NT) {
      if ((c >= HKV && c < HKV + H) ? !do_q : !do_kv) continue;
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
  // norm-weight partials: over the wavefront's head slots, then over the wavefronts
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int o = LPH; o < 64; o <<= 1) {
      dqw0[i] += __shfl_xor(dqw0[i], o, 64);
      dqw1[i] += __shfl_xor(dqw1[i], o, 64);
      dkw0[i] += __shfl_xor(dkw0[i], o, 64);
      dkw1[i] += __shfl_xor(dkw1[i], o, 64);
    }
  if (hl == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[0][w][j + i] = dqw0[i];
      red[0][w][HALF + j + i] = dqw1[i];
      red[1][w][j + i] = dkw0[i];
      red[1][w][HALF + j + i] = dkw1[i];
    }
  }
  __syncthreads();
  if (tid < HD) {
    if (do_q)
      a.d_qn_w[(long long)blockIdx.x * HD + tid] = red[0][0][tid] + red[0][1][tid] + red[0][2][tid] + red[0][3][tid];
    if (do_kv)
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
  if (a->parts < 0 || a->parts > 2) return B3_ERR_ARG;
  const long long need = (long long)(a->H + 2 * a->HKV) * a->HD + a->HKV + a->H;
  if (a->dz_cols < need || a->dz_row_stride < a->dz_cols || a->dz_row_stride % 4) return B3_ERR_ARG;
  if (!a->d_q_raw || !a->d_q_rope || !a->d_k_own || !a->d_k_next || !a->d_v_own || !a->d_v_next || !a->d_eta ||
      !a->beta || !a->eta || !a->inv_freq || !a->dz)
    return B3_ERR_ARG;
  if ((a->d_sink_k || a->d_sink_v) && (!a->d_sink_k || !a->d_sink_v || a->n_chunks <= 0 || a->n_sinks <= 0))
    return B3_ERR_ARG;
  if (a->has_qk_norm && (!a->lin_q || !a->lin_k || !a->qn_w || !a->kn_w || !a->d_qn_w || !a->d_kn_w ||
                         a->lin_q_row_stride < (long long)a->H * a->HD || a->lin_k_row_stride < (long long)a->HKV * a->HD ||
                         a->lin_q_row_stride % 4 || a->lin_k_row_stride % 4))
    return B3_ERR_ARG;
  const int nb = bolt3_heads_bwd_blocks(a->B, a->T);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  using namespace b3::hbwd;
  if (a->dtype == B3_BF16) {
    if (a->HD == 128) hipLaunchKernelGGL((heads_bwd_kernel<uint16_t, 128>), dim3(nb), dim3(NT), 0, st, *a);
    else hipLaunchKernelGGL((heads_bwd_kernel<uint16_t, 64>), dim3(nb), dim3(NT), 0, st, *a);
  } else {
    if (a->HD == 128) hipLaunchKernelGGL((heads_bwd_kernel<float, 128>), dim3(nb), dim3(NT), 0, st, *a);
    else hipLaunchKernelGGL((heads_bwd_kernel<float, 64>), dim3(nb), dim3(NT), 0, st, *a);
  }
  return (int)hipGetLastError();
}

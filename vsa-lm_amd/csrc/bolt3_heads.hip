// Head preparation: split the packed projection row into q/k/v heads, apply
// the optional q/k RMSNorm, RoPE at integer positions, and the beta/eta gates.
//
// Replaces the elementwise part of Bolt3Attn.forward between the projections
// and the chunk loop: head_qkv's q/k RMSNorm (vsa_lm/config/bolt3.py:64-65,
// vsa_lm/surgery.py:49-53), LlamaRoPE (vsa_lm/surgery.py:86-93, applied at
// vsa_lm/config/bolt3.py:197 and :347) and the gates
// sigmoid(beta_proj x), tanh(eta_proj x) (vsa_lm/config/bolt3.py:198-199, :348-349).
//
// One workgroup per token row; a head is handled by HD/2 lanes, lane i owning
// the RoPE pair (i, i + HD/2).  Every value is rounded to the storage type at
// the same points as the reference's per-op evaluation.
#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

template <typename T, int HD>
__global__ void __launch_bounds__(256) heads_kernel(b3_heads_args a) {
  constexpr int HALF = HD / 2;
  constexpr int UNITS = 256 / HALF;  // heads processed per pass
  const int t = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x;
  const T* row = reinterpret_cast<const T*>(a.lin) + ((long long)b * a.T + t) * a.lin_row_stride;
  const float pos = (float)(a.pos0 + t);

  const int n_units = a.H + 2 * a.HKV;
  const int unit_in_pass = tid / HALF;
  const int i = tid % HALF;
  const float inv = a.inv_freq[i];
  const float ang = mul_rn(pos, inv);
  float sn, cs;
  sincos_rope(ang, &sn, &cs);
  const float c = St<T>::rnd(cs), s = St<T>::rnd(sn);

  for (int u0 = 0; u0 < n_units; u0 += UNITS) {
    const int u = u0 + unit_in_pass;
    const bool live = u < n_units;
    int kind = 0, h = 0;  // 0: q, 1: k, 2: v
    if (live) {
      if (u < a.H) { kind = 0; h = u; }
      else if (u < a.H + a.HKV) { kind = 1; h = u - a.H; }
      else { kind = 2; h = u - a.H - a.HKV; }
    }
    const int col = kind == 0 ? h * HD : (kind == 1 ? (a.H + h) * HD : (a.H + a.HKV + h) * HD);
    float x0 = 0.f, x1 = 0.f;
    if (live) {
      x0 = St<T>::ld(row + col + i);
      x1 = St<T>::ld(row + col + i + HALF);
    }
    // RMSNorm over the head (q and k only, when the module has q/k norms).
    float ss = x0 * x0 + x1 * x1;
#pragma unroll
    for (int o = HALF / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (live && kind < 2 && a.has_qk_norm) {
      const float* w = kind == 0 ? a.qn_w : a.kn_w;
      const float r = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
      x0 = St<T>::rnd(mul_rn(mul_rn(x0, r), w[i]));
      x1 = St<T>::rnd(mul_rn(mul_rn(x1, r), w[i + HALF]));
    }
    if (!live) continue;
    if (kind == 2) {
      T* o = reinterpret_cast<T*>(a.v.p) + b * a.v.sb + h * a.v.sh + (long long)t * HD;
      o[i] = St<T>::from_f(x0);
      o[i + HALF] = St<T>::from_f(x1);
      continue;
    }
    // out = x*cos + rotate_half(x)*sin, each product and the sum rounded.
    const float r0 = St<T>::rnd(add_rn(St<T>::rnd(mul_rn(x0, c)), St<T>::rnd(mul_rn(-x1, s))));
    const float r1 = St<T>::rnd(add_rn(St<T>::rnd(mul_rn(x1, c)), St<T>::rnd(mul_rn(x0, s))));
    const b3_tensor_out& raw = kind == 0 ? a.q_raw : a.k_raw;
    const b3_tensor_out& rot = kind == 0 ? a.q_rope : a.k_rope;
    if (raw.p) {
      T* o = reinterpret_cast<T*>(raw.p) + b * raw.sb + h * raw.sh + (long long)t * HD;
      o[i] = St<T>::from_f(x0);
      o[i + HALF] = St<T>::from_f(x1);
    }
    T* o = reinterpret_cast<T*>(rot.p) + b * rot.sb + h * rot.sh + (long long)t * HD;
    o[i] = St<T>::from_f(r0);
    o[i + HALF] = St<T>::from_f(r1);
  }

  // Gates: beta = sigmoid(.) per kv head, eta = tanh(.) per query head, stored as
  // fp32 copies of the storage-type values.
  const int gcol = (a.H + 2 * a.HKV) * HD;
  for (int g = tid; g < a.HKV + a.H; g += 256) {
    const float z = St<T>::ld(row + gcol + g);
    if (g < a.HKV) {
      const float val = St<T>::rnd(1.0f / (1.0f + expf(-z)));
      a.beta.p[b * a.beta.sb + g * a.beta.sh + t] = val;
    } else {
      const int hq = g - a.HKV;
      const float val = St<T>::rnd(tanhf(z));
      a.eta.p[b * a.eta.sb + hq * a.eta.sh + t] = val;
    }
  }
  if (a.pos_out && b == 0 && tid == 0) a.pos_out[t] = pos;
}

template <typename T>
static int launch_heads(const b3_heads_args& a, hipStream_t st) {
  dim3 grid(a.T, a.B), block(256);
  if (a.HD == 64) hipLaunchKernelGGL((heads_kernel<T, 64>), grid, block, 0, st, a);
  else if (a.HD == 128) hipLaunchKernelGGL((heads_kernel<T, 128>), grid, block, 0, st, a);
  else return B3_ERR_UNSUPPORTED;
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int bolt3_heads(const b3_heads_args* a, void* stream) {
  if (!a || a->T <= 0 || a->B <= 0 || a->HKV <= 0) return B3_ERR_ARG;
  if (a->H % a->HKV != 0 || !a->q_rope.p || !a->k_rope.p || !a->v.p || !a->beta.p || !a->eta.p || !a->lin ||
      !a->inv_freq)
    return B3_ERR_ARG;
  if (a->has_qk_norm && (!a->qn_w || !a->kn_w)) return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return b3::launch_heads<float>(*a, st);
  if (a->dtype == B3_BF16) return b3::launch_heads<uint16_t>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

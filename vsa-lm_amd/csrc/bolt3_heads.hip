// Head preparation: split the packed projection row into q/k/v heads, apply
// the optional q/k RMSNorm, RoPE at integer positions, and the beta/eta gates.
//
// Replaces the elementwise part of Bolt3Attn.forward between the projections
// and the chunk loop: head_qkv's q/k RMSNorm (vsa_lm/config/bolt3.py:64-65,
// vsa_lm/surgery.py:49-53), LlamaRoPE (vsa_lm/surgery.py:86-93, applied at
// vsa_lm/config/bolt3.py:197 and :347) and the gates
// sigmoid(beta_proj x), tanh(eta_proj x) (vsa_lm/config/bolt3.py:198-199, :348-349).
//
// Layout: a workgroup handles TOK consecutive tokens of one batch row.  A head unit
// (q, k or v head of one token) is handled by HD/16 lanes; lane p owns the RoPE pairs
// (8p..8p+7, HD/2+8p..HD/2+8p+7), so every load and store is a 16-byte vector and the
// RMS statistic is a 3- (HD=128) or 2-step (HD=64) shuffle sum.  The rounded cos / sin
// of the TOK positions come from an LDS table filled once per workgroup.  Every value is
// rounded to the storage type at the same points as the reference's per-op evaluation.
#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int HEADS_TOK = 4;    // tokens per workgroup
constexpr int HEADS_NT = 256;   // threads per workgroup

template <typename T, int HD>
__global__ void __launch_bounds__(HEADS_NT) heads_kernel(b3_heads_args a) {
  constexpr int HALF = HD / 2, P8 = HALF / 8;   // lanes per head unit
  __shared__ float cs_tab[HEADS_TOK][HALF], sn_tab[HEADS_TOK][HALF];
  const int b = blockIdx.y, t0 = blockIdx.x * HEADS_TOK;
  const int tid = threadIdx.x;
  const int ntok = min(HEADS_TOK, a.T - t0);

  for (int it = tid; it < HEADS_TOK * HALF; it += HEADS_NT) {
    const int tt = it / HALF, i = it % HALF;
    float sn, cs;
    sincos_rope(mul_rn((float)(a.pos0 + t0 + tt), a.inv_freq[i]), &sn, &cs);
    cs_tab[tt][i] = St<T>::rnd(cs);
    sn_tab[tt][i] = St<T>::rnd(sn);
    if constexpr (St<T>::is_bf16)
      if (a.rope_cs && b == 0 && t0 + tt < a.T) a.rope_cs[(long long)(t0 + tt) * HALF + i] = pack_bf2(cs, sn);
  }
  __syncthreads();

  // units: q heads 0..H-1, then k heads, then v heads; `parts` selects q or k/v
  const int parts = a.parts == 0 ? 3 : a.parts;
  const int u_begin = (parts & 1) ? 0 : a.H;
  const int u_end = (parts & 2) ? a.H + 2 * a.HKV : a.H;
  const int n_units = u_end - u_begin;
  const bool split = a.lin_kv != nullptr;
  const int items = HEADS_TOK * n_units * P8;   // P8 consecutive threads share one (token, unit)
  for (int it = tid; it < items; it += HEADS_NT) {
    const int p = it % P8, unit = u_begin + (it / P8) % n_units, tt = it / (P8 * n_units);
    if (tt >= ntok) continue;   // uniform across the P8 lanes of the unit
    const int t = t0 + tt;
    const long long tok = (long long)b * a.T + t;
    const T* row = (split && unit >= a.H)
                       ? reinterpret_cast<const T*>(a.lin_kv) + tok * a.lin_kv_row_stride + (unit - a.H) * HD
                       : reinterpret_cast<const T*>(a.lin) + tok * a.lin_row_stride + unit * HD;
    Vec8<T> x0, x1;
    x0.load(row + 8 * p);
    x1.load(row + HALF + 8 * p);
    const int kind = unit < a.H ? 0 : (unit < a.H + a.HKV ? 1 : 2);   // q, k, v
    const int h = kind == 0 ? unit : (kind == 1 ? unit - a.H : unit - a.H - a.HKV);
    if (kind == 2) {
      T* o = reinterpret_cast<T*>(a.v.p) + b * a.v.sb + h * a.v.sh + (long long)t * HD;
      x0.store(o + 8 * p);
      x1.store(o + HALF + 8 * p);
      continue;
    }
    // RMSNorm over the head (fp32 statistic), then weight, one rounding
    if (a.has_qk_norm) {
      float u8[8], w8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u8[e] = x0.get(e);
        w8[e] = x1.get(e);
      }
      float ss = sumsq_pair8(u8, w8);
#pragma unroll
      for (int o = P8 / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
      const float* wt = kind == 0 ? a.qn_w : a.kn_w;
      const float r = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x0.set(e, mul_rn(mul_rn(x0.get(e), r), wt[8 * p + e]));
        x1.set(e, mul_rn(mul_rn(x1.get(e), r), wt[HALF + 8 * p + e]));
      }
    }
    const b3_tensor_out& raw = kind == 0 ? a.q_raw : a.k_raw;
    const b3_tensor_out& rot = kind == 0 ? a.q_rope : a.k_rope;
    if (raw.p) {
      T* o = reinterpret_cast<T*>(raw.p) + b * raw.sb + h * raw.sh + (long long)t * HD;
      x0.store(o + 8 * p);
      x1.store(o + HALF + 8 * p);
    }
    // out = x*cos + rotate_half(x)*sin, each product and the sum rounded
    Vec8<T> r0, r1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c = cs_tab[tt][8 * p + e], sn = sn_tab[tt][8 * p + e];
      const float u = x0.get(e), w = x1.get(e);
      r0.set(e, add_rn(St<T>::rnd(mul_rn(u, c)), St<T>::rnd(mul_rn(-w, sn))));
      r1.set(e, add_rn(St<T>::rnd(mul_rn(w, c)), St<T>::rnd(mul_rn(u, sn))));
    }
    T* o = reinterpret_cast<T*>(rot.p) + b * rot.sb + h * rot.sh + (long long)t * HD;
    r0.store(o + 8 * p);
    r1.store(o + HALF + 8 * p);
  }

  // Gates: beta = sigmoid(.) per kv head, eta = tanh(.) per query head, stored as fp32
  // copies of the storage-type values.
  const int g_begin = (parts & 2) ? 0 : a.HKV, g_end = (parts & 1) ? a.HKV + a.H : a.HKV;
  const int ng = g_end - g_begin;
  for (int it = tid; it < HEADS_TOK * ng; it += HEADS_NT) {
    const int tt = it / ng, g = g_begin + it % ng;
    if (tt >= ntok) continue;
    const int t = t0 + tt;
    const long long tok = (long long)b * a.T + t;
    float z;
    if (a.gates) z = St<T>::ld(reinterpret_cast<const T*>(a.gates) + tok * a.gates_row_stride + g);
    else if (!split) z = St<T>::ld(reinterpret_cast<const T*>(a.lin) + tok * a.lin_row_stride + (a.H + 2 * a.HKV) * HD + g);
    else if (g < a.HKV) z = St<T>::ld(reinterpret_cast<const T*>(a.lin_kv) + tok * a.lin_kv_row_stride + 2 * a.HKV * HD + g);
    else z = St<T>::ld(reinterpret_cast<const T*>(a.lin) + tok * a.lin_row_stride + a.H * HD + (g - a.HKV));
    if (g < a.HKV) {
      a.beta.p[b * a.beta.sb + g * a.beta.sh + t] = St<T>::rnd(1.0f / (1.0f + expf(-z)));
    } else {
      a.eta.p[b * a.eta.sb + (g - a.HKV) * a.eta.sh + t] = St<T>::rnd(tanhf(z));
    }
  }
  if (a.pos_out && (parts & 2) && b == 0 && tid < ntok) a.pos_out[t0 + tid] = (float)(a.pos0 + t0 + tid);
}

template <typename T>
static int launch_heads(const b3_heads_args& a, hipStream_t st) {
  dim3 grid((a.T + HEADS_TOK - 1) / HEADS_TOK, a.B), block(HEADS_NT);
  if (a.HD == 64) hipLaunchKernelGGL((heads_kernel<T, 64>), grid, block, 0, st, a);
  else if (a.HD == 128) hipLaunchKernelGGL((heads_kernel<T, 128>), grid, block, 0, st, a);
  else return B3_ERR_UNSUPPORTED;
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int bolt3_heads(const b3_heads_args* a, void* stream) {
  if (!a || a->T <= 0 || a->B <= 0 || a->HKV <= 0) return B3_ERR_ARG;
  const int parts = a->parts == 0 ? 3 : a->parts;
  if (parts < 0 || parts > 3 || a->H % a->HKV != 0 || !a->inv_freq) return B3_ERR_ARG;
  if ((parts & 1) && (!a->q_rope.p || !a->eta.p || !a->lin)) return B3_ERR_ARG;
  if (a->gates && a->gates_row_stride < a->HKV + a->H) return B3_ERR_ARG;
  if ((parts & 2) && (!a->k_rope.p || !a->v.p || !a->beta.p || (!a->lin && !a->lin_kv))) return B3_ERR_ARG;
  if (a->has_qk_norm && (!a->qn_w || !a->kn_w)) return B3_ERR_ARG;
  if (a->rope_cs && (a->dtype != B3_BF16 || reinterpret_cast<uintptr_t>(a->rope_cs) % 4)) return B3_ERR_ARG;
  // 16-byte vector moves: projection rows and head rows must start 16-byte aligned
  const int64_t es = a->dtype == B3_BF16 ? 2 : 4;
  if (a->lin && ((a->lin_row_stride * es) % 16 || reinterpret_cast<uintptr_t>(a->lin) % 16)) return B3_ERR_ARG;
  if (a->lin_kv && ((a->lin_kv_row_stride * es) % 16 || reinterpret_cast<uintptr_t>(a->lin_kv) % 16)) return B3_ERR_ARG;
  const b3_tensor_out* outs[5] = {&a->q_raw, &a->q_rope, &a->k_raw, &a->k_rope, &a->v};
  for (const b3_tensor_out* o : outs)
    if (o->p && (reinterpret_cast<uintptr_t>(o->p) % 16 || (o->sb * es) % 16 || (o->sh * es) % 16)) return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return b3::launch_heads<float>(*a, st);
  if (a->dtype == B3_BF16) return b3::launch_heads<uint16_t>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

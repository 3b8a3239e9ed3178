// One-token decode step of a Bolt-3 layer (t_s == 1 branch of
// Bolt3Decoder.step, vsa_lm/config/bolt3.py:346-402).
//
// Per (batch row, kv head) workgroup:
//   1. head prep of the new token (q/k RMSNorm, RoPE at `pos`, beta/eta
//      gates) and its append to the window ring (roped and un-roped key,
//      value, beta, position);
//   2. fp32 scores of the G query heads against sinks, attractor slots
//      (cached roped keys + kappa*log(mass) bias) and the whole window;
//   3. one fp32 softmax per head, probabilities rounded to the storage dtype,
//      value read;
//   4. the M_res readout eta * RMSNorm(normalize(q_raw) M (1-gamma)/sqrt(HD)).
// The step is bound by reading the window, the slots and M_res once; every
// load is a 16-byte vector load spread over HD/8 lanes per key.
#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int DNT = 256;
constexpr int GMAX = 8;
constexpr int NKMAX = 4 + 128 + 4 * 128 + 8;

template <typename T, int HD>
struct DecSmem {
  float q[GMAX][HD];       // roped query (values of the storage dtype)
  float qr[GMAX][HD];      // un-roped query
  float kn[HD];            // new roped key (for its own score)
  float s[GMAX][NKMAX];    // scores, then probabilities
  float red[16][GMAX][HD]; // partial sums of the value read / readout
  float eta[GMAX];
  float stat[GMAX][2];
};

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* out) {
  if constexpr (St<T>::is_bf16) {
    const u16x8 v = *reinterpret_cast<const u16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = bf2f(v[i]);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

template <typename T, int HD>
__global__ void __launch_bounds__(DNT) decode_kernel(b3_decode_args a) {
  __shared__ DecSmem<T, HD> sm;
  constexpr int HALF = HD / 2;
  constexpr int TPK = HD / 8;           // threads per key
  constexpr int KPAR = DNT / TPK;       // keys in flight
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x;
  const T* row = reinterpret_cast<const T*>(a.lin) + (long long)b * a.lin_row_stride;
  const float pos = (float)a.pos;
  const int new_idx = a.b_start + a.b_len;
  const long long wbase = (long long)b * a.w_sb + (long long)hkv * a.w_sh;

  // ---- 1. head prep: units 0..G-1 query heads, G key, G+1 value
  {
    const int i = tid % HALF;
    float sn, cs;
    sincos_rope(mul_rn(pos, a.inv_freq[i]), &sn, &cs);
    const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
    constexpr int UNITS = DNT / HALF;
    for (int u0 = 0; u0 < G + 2; u0 += UNITS) {
      const int u = u0 + tid / HALF;
      const bool live = u < G + 2;
      const int kind = u < G ? 0 : (u == G ? 1 : 2);
      const int col = kind == 0 ? (hkv * G + u) * HD : (kind == 1 ? (a.H + hkv) * HD : (a.H + a.HKV + hkv) * HD);
      float x0 = live ? St<T>::ld(row + col + i) : 0.f;
      float x1 = live ? St<T>::ld(row + col + i + HALF) : 0.f;
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
        T* o = reinterpret_cast<T*>(a.win_v) + wbase + (long long)new_idx * HD;
        o[i] = St<T>::from_f(x0);
        o[i + HALF] = St<T>::from_f(x1);
        continue;
      }
      const float r0 = St<T>::rnd(add_rn(St<T>::rnd(mul_rn(x0, c)), St<T>::rnd(mul_rn(-x1, si))));
      const float r1 = St<T>::rnd(add_rn(St<T>::rnd(mul_rn(x1, c)), St<T>::rnd(mul_rn(x0, si))));
      if (kind == 0) {
        sm.q[u][i] = r0; sm.q[u][i + HALF] = r1;
        sm.qr[u][i] = x0; sm.qr[u][i + HALF] = x1;
      } else {
        T* kr = reinterpret_cast<T*>(a.win_kr) + wbase + (long long)new_idx * HD;
        T* kp = reinterpret_cast<T*>(a.win_kp) + wbase + (long long)new_idx * HD;
        kr[i] = St<T>::from_f(x0); kr[i + HALF] = St<T>::from_f(x1);
        kp[i] = St<T>::from_f(r0); kp[i + HALF] = St<T>::from_f(r1);
        sm.kn[i] = r0; sm.kn[i + HALF] = r1;
      }
    }
    const int gcol = (a.H + 2 * a.HKV) * HD;
    if (tid == 0) {
      const float z = St<T>::ld(row + gcol + hkv);
      a.win_beta[b * a.wb_sb + hkv * a.wb_sh + new_idx] = St<T>::rnd(1.0f / (1.0f + expf(-z)));
      if (bh == 0 && a.win_pos) a.win_pos[new_idx] = pos;
    }
    if (tid < G) sm.eta[tid] = St<T>::rnd(tanhf(St<T>::ld(row + gcol + a.HKV + hkv * G + tid)));
  }
  __threadfence_block();
  __syncthreads();

  // ---- 2. scores over [sinks | slots | window A | window B (incl. new token)]
  const int ns = a.n_sink_keys, nsl = a.has_slots ? a.S : 0, na = a.a_len, nb = a.b_len + 1;
  const int nk = ns + nsl + na + nb;
  const float scale = 1.0f / sqrtf((float)HD);
  const T* sink_k = reinterpret_cast<const T*>(a.sink_k);
  const T* slot_k = reinterpret_cast<const T*>(a.slot_k) + (long long)bh * a.S * HD;
  const T* win_k = reinterpret_cast<const T*>(a.win_kp) + wbase;
  auto key_ptr = [&](int kidx) -> const T* {
    if (kidx < ns) return sink_k + (long long)b * a.s_sb + (long long)hkv * a.s_sh + (long long)kidx * HD;
    kidx -= ns;
    if (kidx < nsl) return slot_k + (long long)kidx * HD;
    kidx -= nsl;
    if (kidx < na) return win_k + (long long)(a.a_start + kidx) * HD;
    kidx -= na;
    return win_k + (long long)(a.b_start + kidx) * HD;
  };
  const int sub = tid % TPK, grp = tid / TPK;
  for (int k0 = 0; k0 < nk; k0 += KPAR) {
    const int kidx = k0 + grp;
    float kv[8];
    if (kidx < nk) load8<T>(key_ptr(kidx) + 8 * sub, kv);
    else {
#pragma unroll
      for (int i = 0; i < 8; ++i) kv[i] = 0.f;
    }
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d += sm.q[g][8 * sub + i] * kv[i];
#pragma unroll
      for (int o = TPK / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, 64);
      if (sub == 0 && kidx < nk) {
        float x = mul_rn(d, scale);
        if (kidx >= ns && kidx < ns + nsl) x = add_rn(x, a.slot_bias[(long long)bh * a.S + (kidx - ns)]);
        sm.s[g][kidx] = x;
      }
    }
  }
  __syncthreads();

  // ---- 3. softmax per head (one wavefront per head), probabilities in the storage dtype
  {
    const int lane = tid & 63, wv = tid >> 6;
    for (int g = wv; g < G; g += DNT / 64) {
      float mx = -INFINITY;
      for (int k = lane; k < nk; k += 64) mx = fmaxf(mx, sm.s[g][k]);
      mx = wave_reduce(mx, [](float x, float y) { return fmaxf(x, y); });
      float sum = 0.f;
      for (int k = lane; k < nk; k += 64) {
        const float e = expf(sm.s[g][k] - mx);
        sm.s[g][k] = e;
        sum += e;
      }
      sum = wave_sum(sum);
      const float rs = 1.0f / sum;
      for (int k = lane; k < nk; k += 64) sm.s[g][k] = St<T>::rnd(mul_rn(sm.s[g][k], rs));
    }
  }
  __syncthreads();

  // ---- value read: y[g][d] = sum_k p[g][k] v[k][d]
  {
    const T* sink_v = reinterpret_cast<const T*>(a.sink_v);
    const T* slot_v = reinterpret_cast<const T*>(a.slot_v) + (long long)bh * a.S * HD;
    const T* win_v = reinterpret_cast<const T*>(a.win_v) + wbase;
    float acc[GMAX][8];
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    for (int kidx = grp; kidx < nk; kidx += KPAR) {
      const T* p;
      int kk = kidx;
      if (kk < ns) p = sink_v + (long long)b * a.s_sb + (long long)hkv * a.s_sh + (long long)kk * HD;
      else if ((kk -= ns) < nsl) p = slot_v + (long long)kk * HD;
      else if ((kk -= nsl) < na) p = win_v + (long long)(a.a_start + kk) * HD;
      else p = win_v + (long long)(a.b_start + kk - na) * HD;
      float vv[8];
      load8<T>(p + 8 * sub, vv);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g < G) {
          const float pg = sm.s[g][kidx];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] += pg * vv[i];
        }
      }
    }
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) sm.red[grp % 16][g][8 * sub + i] = 0.f;
    __syncthreads();
    // groups beyond 16 (HD == 64) fold onto the first 16 rows in two rounds
    for (int rnd = 0; rnd < KPAR / 16; ++rnd) {
      if (grp / 16 == rnd)
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int i = 0; i < 8; ++i) sm.red[grp % 16][g][8 * sub + i] += acc[g][i];
      __syncthreads();
    }
  }
  // sum the partials: thread (g, d); the attention output reuses the query storage
  for (int it = tid; it < G * HD; it += DNT) {
    const int g = it / HD, d = it % HD;
    float s = 0.f;
    for (int r = 0; r < 16; ++r) s += sm.red[r][g][d];
    sm.q[g][d] = St<T>::rnd(s);
  }
  __syncthreads();

  // ---- 4. readout
  const bool has_m = a.m_res != nullptr;
  if (has_m) {
    const float* M = a.m_res + (long long)bh * HD * HD;
    // normalized raw query
    {
      const int lane = tid & 63, wv = tid >> 6;
      for (int g = wv; g < G; g += DNT / 64) {
        float ss = 0.f;
        for (int d = lane; d < HD; d += 64) ss += sm.qr[g][d] * sm.qr[g][d];
        ss = wave_sum(ss);
        if (lane == 0) sm.stat[g][0] = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      }
    }
    __syncthreads();
    constexpr int CG = DNT / HD;  // c-groups
    const int d = tid % HD, cg = tid / HD;
    float acc[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) acc[g] = 0.f;
    for (int c = cg; c < HD; c += CG) {
      const float m = M[(long long)c * HD + d];
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) acc[g] += sm.qr[g][c] * m;
    }
    for (int g = 0; g < G; ++g) sm.red[cg][g][d] = acc[g];
    __syncthreads();
    const float coef = div_rn(1.0f - a.gamma[hkv], sqrtf((float)HD));
    for (int it = tid; it < G * HD; it += DNT) {
      const int g = it / HD, dd = it % HD;
      float s = 0.f;
      for (int r = 0; r < CG; ++r) s += sm.red[r][g][dd];
      sm.red[8][g][dd] = mul_rn(s * sm.stat[g][0], coef);
    }
    __syncthreads();
    {
      const int lane = tid & 63, wv = tid >> 6;
      for (int g = wv; g < G; g += DNT / 64) {
        float ss = 0.f;
        for (int dd = lane; dd < HD; dd += 64) ss += sm.red[8][g][dd] * sm.red[8][g][dd];
        ss = wave_sum(ss);
        if (lane == 0) sm.stat[g][1] = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
      }
    }
    __syncthreads();
    for (int it = tid; it < G * HD; it += DNT) {
      const int g = it / HD, dd = it % HD;
      const float ymn = mul_rn(mul_rn(sm.red[8][g][dd], sm.stat[g][1]), a.res_w[dd]);
      sm.q[g][dd] = St<T>::rnd(add_rn(sm.q[g][dd], St<T>::rnd(mul_rn(sm.eta[g], ymn))));
    }
    __syncthreads();
  }

  // ---- write y[b][hq*HD + d]
  T* y = reinterpret_cast<T*>(a.y) + (long long)b * a.H * HD + (long long)hkv * G * HD;
  for (int it = tid; it < G * HD; it += DNT) y[it] = St<T>::from_f(sm.q[it / HD][it % HD]);
}

template <typename T, int HD>
static int launch_decode(const b3_decode_args& a, hipStream_t st) {
  hipLaunchKernelGGL((decode_kernel<T, HD>), dim3(a.B * a.HKV), dim3(DNT), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int bolt3_decode(const b3_decode_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->H % a->HKV != 0) return B3_ERR_ARG;
  if (a->H / a->HKV > b3::GMAX || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  const int nk = a->n_sink_keys + (a->has_slots ? a->S : 0) + a->a_len + a->b_len + 1;
  if (nk > b3::NKMAX || a->n_sink_keys < 0 || a->a_len < 0 || a->b_len < 0) return B3_ERR_UNSUPPORTED;
  if (!a->lin || !a->win_kr || !a->win_kp || !a->win_v || !a->win_beta || !a->inv_freq || !a->gamma || !a->res_w ||
      !a->y)
    return B3_ERR_ARG;
  if (a->has_slots && (!a->slot_k || !a->slot_v || !a->slot_bias)) return B3_ERR_ARG;
  if (a->n_sink_keys > 0 && (!a->sink_k || !a->sink_v)) return B3_ERR_ARG;
  if (a->has_qk_norm && (!a->qn_w || !a->kn_w)) return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return a->HD == 64 ? b3::launch_decode<float, 64>(*a, st) : b3::launch_decode<float, 128>(*a, st);
  if (a->dtype == B3_BF16)
    return a->HD == 64 ? b3::launch_decode<uint16_t, 64>(*a, st) : b3::launch_decode<uint16_t, 128>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

extern "C" const char* bolt3_version(void) { return "bolt3_amd 0.1 gfx950 (MFMA 32x32, wave64)"; }

// One-token decode step of a Bolt-3 layer (t_s == 1 branch of
// Bolt3Decoder.step, vsa_lm/config/bolt3.py:346-402).
//
// The step is bound by reading the window, the slots and M_res once, so it is
// split over many workgroups (flash-decoding):
//   decode_split_kernel, grid (NSPLIT + 1, B*HKV):
//     workgroups 0..NSPLIT-1 each take a contiguous range of the keys
//     [sinks | attractor slots | window A | window B + new token] of one
//     (batch, kv head): fp32 scores of the G query heads (q/k RMSNorm and RoPE
//     of the new token recomputed per workgroup), a local softmax, and the
//     value read with the probabilities rounded to the storage dtype; they
//     leave (max, sum, unnormalised output) per head in the workspace.  The
//     last range owns the new token: it appends its roped and un-roped key,
//     value, beta and position to the window ring.
//     workgroup NSPLIT computes the M_res readout
//     eta * RMSNorm(normalize(q_raw) M (1-gamma)/sqrt(HD)), rounded.
//   decode_combine_kernel, grid (B*HKV): merges the NSPLIT partial softmaxes,
//     rounds the attention output and adds the readout.
// Every key or value row is read as 16-byte vectors by HD/8 lanes, several rows
// per thread in flight.
#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int DNT = 256;        // threads per decode workgroup
constexpr int GMAX = 8;         // query heads per kv head
constexpr int NSPLIT = 4;       // key ranges per (batch, kv head)
constexpr int KCAP = 168;       // keys per range at most (4 sinks + 128 slots + two window halves of 256)
constexpr int NKMAX = NSPLIT * KCAP;

// per (bh): NSPLIT x G x (HD + 2) floats of partial softmax state, then G x HD readout floats
__host__ __device__ constexpr long long dec_ws_per_bh(int G, int HD) {
  return (long long)NSPLIT * G * (HD + 2) + (long long)G * HD;
}

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
struct SplitSmem {
  float q[GMAX][HD];          // roped queries (storage-dtype values)
  float qr[GMAX][HD];         // un-roped queries after the norm
  float kn[HD], vn[HD];       // new token's roped key and value
  float s[GMAX][KCAP];        // scores, then probabilities of this range
  float part[DNT / 64][GMAX][HD];   // per-wavefront partials of the value read; per row group of the readout
  float eta[GMAX];
  float stat[GMAX][2];
};

// Head preparation of the new token for G query heads (and, when `with_kv`, its key and
// value, appended to the window ring): RMSNorm (fp32 statistic, one rounding), RoPE at `pos`
// with per-op rounding.  HD/16 lanes per head unit, lane p owning the pairs
// (8p..8p+7, HD/2+8p..HD/2+8p+7).
template <typename T, int HD>
__device__ void prep_token(const b3_decode_args& a, SplitSmem<T, HD>& sm, int b, int hkv, int G, bool with_kv,
                           int tid) {
  constexpr int HALF = HD / 2, P8 = HALF / 8;
  const T* row = reinterpret_cast<const T*>(a.lin) + (long long)b * a.lin_row_stride;
  const int n_units = G + (with_kv ? 2 : 0);
  const float pos = (float)a.pos;
  const long long wbase = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const int ni = a.b_start + a.b_len;   // ring index of the new token
  for (int it = tid; it < n_units * P8; it += DNT) {
    const int p = it % P8, u = it / P8;
    const int kind = u < G ? 0 : (u == G ? 1 : 2);   // q, k, v
    const int col = kind == 0 ? (hkv * G + u) * HD : (kind == 1 ? (a.H + hkv) * HD : (a.H + a.HKV + hkv) * HD);
    float x0[8], x1[8];
    load8<T>(row + col + 8 * p, x0);
    load8<T>(row + col + HALF + 8 * p, x1);
    if (kind == 2) {
      T* vo = reinterpret_cast<T*>(a.win_v) + wbase + (long long)ni * HD;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sm.vn[8 * p + e] = x0[e];
        sm.vn[HALF + 8 * p + e] = x1[e];
        vo[8 * p + e] = St<T>::from_f(x0[e]);
        vo[HALF + 8 * p + e] = St<T>::from_f(x1[e]);
      }
      continue;
    }
    if (a.has_qk_norm) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x0[e] * x0[e] + x1[e] * x1[e];
#pragma unroll
      for (int o = P8 / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
      const float* w = kind == 0 ? a.qn_w : a.kn_w;
      const float r = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x0[e] = St<T>::rnd(mul_rn(mul_rn(x0[e], r), w[8 * p + e]));
        x1[e] = St<T>::rnd(mul_rn(mul_rn(x1[e], r), w[HALF + 8 * p + e]));
      }
    }
    float r0[8], r1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sn, cs;
      sincos_rope(mul_rn(pos, a.inv_freq[8 * p + e]), &sn, &cs);
      const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
      r0[e] = St<T>::rnd(add_rn(St<T>::rnd(mul_rn(x0[e], c)), St<T>::rnd(mul_rn(-x1[e], si))));
      r1[e] = St<T>::rnd(add_rn(St<T>::rnd(mul_rn(x1[e], c)), St<T>::rnd(mul_rn(x0[e], si))));
    }
    if (kind == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sm.q[u][8 * p + e] = r0[e];
        sm.q[u][HALF + 8 * p + e] = r1[e];
        sm.qr[u][8 * p + e] = x0[e];
        sm.qr[u][HALF + 8 * p + e] = x1[e];
      }
    } else {
      T* kr = reinterpret_cast<T*>(a.win_kr) + wbase + (long long)ni * HD;
      T* kp = reinterpret_cast<T*>(a.win_kp) + wbase + (long long)ni * HD;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sm.kn[8 * p + e] = r0[e];
        sm.kn[HALF + 8 * p + e] = r1[e];
        kr[8 * p + e] = St<T>::from_f(x0[e]);
        kr[HALF + 8 * p + e] = St<T>::from_f(x1[e]);
        kp[8 * p + e] = St<T>::from_f(r0[e]);
        kp[HALF + 8 * p + e] = St<T>::from_f(r1[e]);
      }
    }
  }
}

template <typename T, int HD>
__global__ void __launch_bounds__(DNT) decode_split_kernel(b3_decode_args a) {
  __shared__ SplitSmem<T, HD> sm;
  constexpr int TPK = HD / 8;        // lanes per key row
  constexpr int KPAR = DNT / TPK;    // rows per pass
  constexpr int U = 2;               // passes in flight
  const int split = blockIdx.x, bh = blockIdx.y, b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x;
  const long long wbase = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const int ns = a.n_sink_keys, nsl = a.has_slots ? a.S : 0, na = a.a_len, nbk = a.b_len + 1;
  const int nk = ns + nsl + na + nbk;
  float* ws = a.work + (long long)bh * dec_ws_per_bh(G, HD);
  const T* row = reinterpret_cast<const T*>(a.lin) + (long long)b * a.lin_row_stride;
  const int gcol = (a.H + 2 * a.HKV) * HD;

  if (split == NSPLIT) {
    // ---------------- M_res readout
    prep_token<T, HD>(a, sm, b, hkv, G, false, tid);
    if (tid < G) sm.eta[tid] = St<T>::rnd(tanhf(St<T>::ld(row + gcol + a.HKV + hkv * G + tid)));
    __syncthreads();
    if (!a.m_res) {
      for (int it = tid; it < G * HD; it += DNT) ws[NSPLIT * G * (HD + 2) + it] = 0.f;
      return;
    }
    {
      const int lane = tid & 63, wv = tid >> 6;
      for (int g = wv; g < G; g += DNT / 64) {
        float ss = 0.f;
        for (int d = lane; d < HD; d += 64) ss += sm.qr[g][d] * sm.qr[g][d];
        ss = wave_sum(ss);
        if (lane == 0) sm.stat[g][0] = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      }
    }
    const float* M = a.m_res + (long long)bh * HD * HD;
    constexpr int CG = DNT / HD;   // row groups of M
    const int d = tid % HD, cg = tid / HD;
    float acc[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) acc[g] = 0.f;
#pragma unroll 8
    for (int c = cg; c < HD; c += CG) {
      const float m = M[(long long)c * HD + d];
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) acc[g] += sm.qr[g][c] * m;
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) sm.part[cg][g][d] = acc[g];
    __syncthreads();
    const float coef = div_rn(1.0f - a.gamma[hkv], sqrtf((float)HD));
    for (int it = tid; it < G * HD; it += DNT) {
      const int g = it / HD, dd = it % HD;
      float s = 0.f;
      for (int r = 0; r < CG; ++r) s += sm.part[r][g][dd];
      sm.s[g][dd] = mul_rn(s * sm.stat[g][0], coef);   // scores area reused for ym
    }
    __syncthreads();
    {
      const int lane = tid & 63, wv = tid >> 6;
      for (int g = wv; g < G; g += DNT / 64) {
        float ss = 0.f;
        for (int dd = lane; dd < HD; dd += 64) ss += sm.s[g][dd] * sm.s[g][dd];
        ss = wave_sum(ss);
        if (lane == 0) sm.stat[g][1] = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
      }
    }
    __syncthreads();
    for (int it = tid; it < G * HD; it += DNT) {
      const int g = it / HD, dd = it % HD;
      const float ymn = mul_rn(mul_rn(sm.s[g][dd], sm.stat[g][1]), a.res_w[dd]);
      ws[NSPLIT * G * (HD + 2) + it] = St<T>::rnd(mul_rn(sm.eta[g], ymn));
    }
    return;
  }

  // ---------------- attention over one key range
  const int per = (nk + NSPLIT - 1) / NSPLIT;
  const int k0 = split * per, k1 = min(nk, k0 + per);
  const bool owns_new = split == (nk - 1) / per;   // the range holding the new token (key nk-1)
  prep_token<T, HD>(a, sm, b, hkv, G, owns_new, tid);
  if (owns_new && tid == 0) {
    const float z = St<T>::ld(row + gcol + hkv);
    a.win_beta[b * a.wb_sb + hkv * a.wb_sh + a.b_start + a.b_len] = St<T>::rnd(1.0f / (1.0f + expf(-z)));
    if (bh == 0 && a.win_pos) a.win_pos[a.b_start + a.b_len] = (float)a.pos;
  }
  __syncthreads();

  const float scale = 1.0f / sqrtf((float)HD);
  const T* sink_k = reinterpret_cast<const T*>(a.sink_k);
  const T* slot_k = reinterpret_cast<const T*>(a.slot_k) + (long long)bh * a.S * HD;
  const T* win_k = reinterpret_cast<const T*>(a.win_kp) + wbase;
  const T* sink_v = reinterpret_cast<const T*>(a.sink_v);
  const T* slot_v = reinterpret_cast<const T*>(a.slot_v) + (long long)bh * a.S * HD;
  const T* win_v = reinterpret_cast<const T*>(a.win_v) + wbase;
  // key kidx of the list -> row pointers (nullptr for the new token, held in LDS)
  auto rows = [&](int kidx, const T*& kp, const T*& vp) {
    int k = kidx;
    if (k < ns) {
      const long long o = (long long)b * a.s_sb + (long long)hkv * a.s_sh + (long long)k * HD;
      kp = sink_k + o;
      vp = sink_v + o;
      return;
    }
    k -= ns;
    if (k < nsl) { kp = slot_k + (long long)k * HD; vp = slot_v + (long long)k * HD; return; }
    k -= nsl;
    if (k < na) { kp = win_k + (long long)(a.a_start + k) * HD; vp = win_v + (long long)(a.a_start + k) * HD; return; }
    k -= na;
    if (k < a.b_len) { kp = win_k + (long long)(a.b_start + k) * HD; vp = win_v + (long long)(a.b_start + k) * HD; return; }
    kp = nullptr;
    vp = nullptr;
  };

  const int sub = tid % TPK, grp = tid / TPK;
  const int nloc = k1 - k0;
  // ---- scores
  for (int base = 0; base < nloc; base += KPAR * U) {
    float kv[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kl = base + u * KPAR + grp;
      const T* kp;
      const T* vp;
      if (kl < nloc) {
        rows(k0 + kl, kp, vp);
        if (kp) load8<T>(kp + 8 * sub, kv[u]);
        else {
#pragma unroll
          for (int i = 0; i < 8; ++i) kv[u][i] = sm.kn[8 * sub + i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) kv[u][i] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kl = base + u * KPAR + grp;
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d += sm.q[g][8 * sub + i] * kv[u][i];
#pragma unroll
        for (int o = TPK / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, 64);
        if (sub == 0 && kl < nloc) {
          float x = mul_rn(d, scale);
          const int kidx = k0 + kl;
          if (kidx >= ns && kidx < ns + nsl) x = add_rn(x, a.slot_bias[(long long)bh * a.S + (kidx - ns)]);
          sm.s[g][kl] = x;
        }
      }
    }
  }
  __syncthreads();
  // ---- local softmax per head (one wavefront per head): p~ = exp(x - m), rounded to the storage dtype
  {
    const int lane = tid & 63, wv = tid >> 6;
    for (int g = wv; g < G; g += DNT / 64) {
      float mx = -INFINITY;
      for (int k = lane; k < nloc; k += 64) mx = fmaxf(mx, sm.s[g][k]);
      mx = wave_reduce(mx, [](float x, float y) { return fmaxf(x, y); });
      float sum = 0.f;
      for (int k = lane; k < nloc; k += 64) {
        const float e = mx == -INFINITY ? 0.f : expf(sm.s[g][k] - mx);
        sm.s[g][k] = St<T>::rnd(e);
        sum += e;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        ws[(split * G + g) * (HD + 2) + HD] = mx;
        ws[(split * G + g) * (HD + 2) + HD + 1] = sum;
      }
    }
  }
  __syncthreads();
  // ---- value read: o[g][d] = sum_k p~[g][k] v[k][d]
  float acc[GMAX][8];
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  for (int base = 0; base < nloc; base += KPAR * U) {
    float vv[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kl = base + u * KPAR + grp;
      const T* kp;
      const T* vp;
      if (kl < nloc) {
        rows(k0 + kl, kp, vp);
        if (vp) load8<T>(vp + 8 * sub, vv[u]);
        else {
#pragma unroll
          for (int i = 0; i < 8; ++i) vv[u][i] = sm.vn[8 * sub + i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) vv[u][i] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kl = base + u * KPAR + grp;
      if (kl < nloc) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
          if (g < G) {
            const float pg = sm.s[g][kl];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] += pg * vv[u][i];
          }
      }
    }
  }
  // reduce the KPAR row groups: the groups of one wavefront (lanes sharing `sub`) by shuffles,
  // then the 4 wavefronts through two LDS rows
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
    if (g < G) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x = acc[g][i];
#pragma unroll
        for (int o = TPK; o < 64; o <<= 1) x += __shfl_xor(x, o, 64);
        acc[g][i] = x;
      }
    }
  const int wv = tid >> 6, lane = tid & 63;
  if (lane < TPK) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sm.part[wv][g][8 * sub + i] = acc[g][i];
      }
  }
  __syncthreads();
  for (int it = tid; it < G * HD; it += DNT) {
    const int g = it / HD, d = it % HD;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < DNT / 64; ++w) o += sm.part[w][g][d];
    ws[(split * G + g) * (HD + 2) + d] = o;
  }
}

// Merge the NSPLIT partial softmaxes of one (batch, kv head), round, add the readout.
template <typename T, int HD>
__global__ void __launch_bounds__(DNT) decode_combine_kernel(b3_decode_args a) {
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const float* ws = a.work + (long long)bh * dec_ws_per_bh(G, HD);
  T* y = reinterpret_cast<T*>(a.y) + (long long)b * a.H * HD + (long long)hkv * G * HD;
  for (int it = threadIdx.x; it < G * HD; it += DNT) {
    const int g = it / HD, d = it % HD;
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NSPLIT; ++s) m = fmaxf(m, ws[(s * G + g) * (HD + 2) + HD]);
    float l = 0.f, o = 0.f;
#pragma unroll
    for (int s = 0; s < NSPLIT; ++s) {
      const float ms = ws[(s * G + g) * (HD + 2) + HD];
      const float w = ms == -INFINITY ? 0.f : expf(ms - m);
      l += ws[(s * G + g) * (HD + 2) + HD + 1] * w;
      o += ws[(s * G + g) * (HD + 2) + d] * w;
    }
    const float att = St<T>::rnd(o / l);
    y[it] = St<T>::from_f(St<T>::rnd(add_rn(att, ws[NSPLIT * G * (HD + 2) + it])));
  }
}

template <typename T, int HD>
static int launch_decode(const b3_decode_args& a, hipStream_t st) {
  const int BH = a.B * a.HKV;
  hipLaunchKernelGGL((decode_split_kernel<T, HD>), dim3(NSPLIT + 1, BH), dim3(DNT), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((decode_combine_kernel<T, HD>), dim3(BH), dim3(DNT), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int64_t bolt3_decode_workspace_bytes(int32_t B, int32_t H, int32_t HKV, int32_t HD) {
  if (B <= 0 || HKV <= 0 || H % HKV != 0) return 0;
  return (int64_t)B * HKV * b3::dec_ws_per_bh(H / HKV, HD) * 4;
}

extern "C" int bolt3_decode(const b3_decode_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->H % a->HKV != 0) return B3_ERR_ARG;
  if (a->H / a->HKV > b3::GMAX || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  const int nk = a->n_sink_keys + (a->has_slots ? a->S : 0) + a->a_len + a->b_len + 1;
  if (nk > b3::NKMAX || a->n_sink_keys < 0 || a->a_len < 0 || a->b_len < 0) return B3_ERR_UNSUPPORTED;
  if (!a->lin || !a->win_kr || !a->win_kp || !a->win_v || !a->win_beta || !a->inv_freq || !a->gamma || !a->res_w ||
      !a->y || !a->work)
    return B3_ERR_ARG;
  if (a->work_bytes < bolt3_decode_workspace_bytes(a->B, a->H, a->HKV, a->HD)) return B3_ERR_WORKSPACE;
  if (a->has_slots && (!a->slot_k || !a->slot_v || !a->slot_bias)) return B3_ERR_ARG;
  if (a->n_sink_keys > 0 && (!a->sink_k || !a->sink_v)) return B3_ERR_ARG;
  if (a->has_qk_norm && (!a->qn_w || !a->kn_w)) return B3_ERR_ARG;
  // 16-byte rows: the projection row and every key / value row
  const int64_t es = a->dtype == B3_BF16 ? 2 : 4;
  if ((a->lin_row_stride * es) % 16 || reinterpret_cast<uintptr_t>(a->lin) % 16) return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return a->HD == 64 ? b3::launch_decode<float, 64>(*a, st) : b3::launch_decode<float, 128>(*a, st);
  if (a->dtype == B3_BF16)
    return a->HD == 64 ? b3::launch_decode<uint16_t, 64>(*a, st) : b3::launch_decode<uint16_t, 128>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

extern "C" const char* bolt3_version(void) { return "bolt3_amd 0.1 gfx950 (MFMA 32x32, wave64)"; }

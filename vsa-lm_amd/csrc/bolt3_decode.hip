// One-token decode step of a Bolt-3 layer (t_s == 1 branch of
// Bolt3Decoder.step, vsa_lm/config/bolt3.py:346-402).
//
// The step is bound by reading the window, the slots and M_res once:
//   decode_prep_kernel, grid (B*HKV): head preparation of the new token (q/k RMSNorm, RoPE,
//     beta/eta gates) from the projection row (or from the fp32 K-chunk partial products of
//     bolt3_decode_layer's projection); appends its roped and un-roped key, value, beta and
//     position to the window ring and leaves the roped and normalised un-roped queries,
//     1/|q_raw| and eta in the workspace.
//   bf16: decode_attn_kernel, grid (B*HKV): attention over
//     [sinks | attractor slots | window A | window B | new token] and the M_res readout of one
//     (batch, kv head) per workgroup, merged in LDS, y written.
//   fp32: decode_split_kernel, grid (ceil(keys / 128) + HD/32, B*HKV), 128-key pieces and
//     32-row readout pieces in parallel with fp32 MFMAs, then decode_combine_kernel, grid
//     (B*HKV), merges the partial softmaxes and finishes the readout.
// bolt3_decode_layer (bf16) adds the two projections around these: rowproj_kernel streams
// a weight once per step and leaves fp32 partial products per K chunk; the prep kernel sums
// those of the input projection and proj_reduce_kernel those of o_proj.
#include <utility>

#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

__device__ __forceinline__ void dec_dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
// ds_read_b64_tr_b16 as inline assembly (the compiler cannot separate these reads from the
// LDS-DMA destination and would wait for all outstanding loads before them); the results are
// used only after dec_lds_wait.
__device__ __forceinline__ u16x4 dec_read_tr(const uint16_t* p) {
  u16x4 r;
  const uint32_t addr = (uint32_t)(size_t)((__attribute__((address_space(3))) const uint16_t*)p);
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
__device__ __forceinline__ void dec_lds_wait(u16x4& a, u16x4& b) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }
// wait until at most N vector-memory operations of this wavefront are outstanding
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}

constexpr int DNT = 256;        // threads per decode workgroup
constexpr int DWAVES = DNT / 64;
constexpr int GMAX = 8;         // query heads per kv head
constexpr int KWG = 32 * DWAVES;   // keys per attention workgroup (one 32-key tile per wavefront)
constexpr int NKMAX = 4 + 128 + 2 * 256 + 8;
constexpr int NSPLIT_MAX = (NKMAX + KWG - 1) / KWG;
constexpr int NPART = NSPLIT_MAX;            // partial softmax states per (batch, kv head)
constexpr int RROWS = 32;       // rows of M_res per readout workgroup

// per (bh): NPART x G x (HD + 2) floats of partial softmax state, HD/RROWS x G x HD partial
// readout floats, G x 2 floats (1/|q_raw|, eta), then the prepared queries: G x HD roped
// (storage dtype, in G x HD float slots) and G x HD un-roped after the norm (fp32)
__host__ __device__ constexpr long long dec_ws_per_bh(int G, int HD) {
  return (long long)NPART * G * (HD + 2) + (long long)(HD / RROWS) * G * HD + 2LL * G + 2LL * G * HD;
}
__host__ __device__ constexpr long long dec_ws_q(int G, int HD) {   // offset of the prepared queries
  return (long long)NPART * G * (HD + 2) + (long long)(HD / RROWS) * G * HD + 2LL * G;
}
__host__ __device__ inline int dec_nsplit(int nk) { return (nk + KWG - 1) / KWG; }

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
  static constexpr int QS = HD + 4;   // query row stride (16-byte rows)
  static constexpr int VS = 32 + 1;   // V^T row stride of a key tile
  alignas(16) T qt[32 * QS];          // roped queries as MFMA operand rows; rows G.. zero
  float qr[GMAX][HD];                 // un-roped queries after the norm
  float bias[DWAVES][32];             // slot bias of each wavefront's key tile
  union {
    T vt[DWAVES][HD * VS];            // V^T of each wavefront's key tile
    float part[DNT / 64][GMAX][HD];   // readout row groups; per-wavefront outputs of the merge
  } u;
  float wm[DWAVES][GMAX], wl[DWAVES][GMAX];   // per-wavefront softmax max / sum
};

// Head preparation of the new token: its G query heads and its key and value, RMSNorm
// (fp32 statistic, one rounding) and RoPE at `pos` with per-op rounding.  HD/16 lanes per
// head unit, lane p owning the pairs (8p..8p+7, HD/2+8p..HD/2+8p+7).  The key (roped and
// un-roped), value, beta and position go to the window ring; the roped queries (storage
// dtype), the normalised un-roped queries (fp32), 1/|q_raw| and eta go to the workspace.
// Source of the projection row when it comes as fp32 partial products of K chunks
// (parts[chunk][b][c], chunk_stride floats apart): the row is the chunks added in order, plus
// the bias, rounded once.  parts == nullptr: the row is a.lin.
constexpr int LP_MAXC = 8;   // K chunks a projection row may come in (K <= 8 * 512)

struct LinParts {
  const float* parts;
  int n_chunks;
  long long chunk_stride;
  const uint16_t* bias;
};

// Where the prepared token goes: roped queries [G][HD] (storage dtype), normalised
// un-roped queries [G][HD] (fp32), (1/|q_raw|, eta) per head, and optionally copies of the
// new token's roped key and value rows (besides the window ring).
template <typename T>
struct PrepOut {
  T* q_rope;
  float* q_raw;
  float* stat;
  T* new_k;
  T* new_v;
};

// The step's position and window segments: the argument fields, or (graph-captured steps) the
// device descriptor, clamped so that every window index stays in [0, ring_cap).
struct StepView {
  int pos, a_start, a_len, b_start, b_len, n_sink, has_slots;
};
__device__ __forceinline__ StepView step_view(const b3_decode_args& a) {
  StepView v;
  if (a.step_desc) {
    const int32_t* d = a.step_desc;
    const int cap = a.ring_cap;
    v.pos = d[0];
    v.a_start = min(max(d[1], 0), cap);
    v.a_len = min(max(d[2], 0), cap - v.a_start);
    v.b_start = min(max(d[3], 0), cap - 1);
    v.b_len = min(max(d[4], 0), cap - 1 - v.b_start);   // the new token goes to b_start + b_len
    v.n_sink = min(max(d[5], 0), 4);
    v.has_slots = d[6] != 0;
  } else {
    v.pos = a.pos;
    v.a_start = a.a_start;
    v.a_len = a.a_len;
    v.b_start = a.b_start;
    v.b_len = a.b_len;
    v.n_sink = a.n_sink_keys;
    v.has_slots = a.has_slots;
  }
  return v;
}

// The head preparation of (batch, kv head) bh by the 128 threads tid = 0..127 (two whole
// wavefronts).  Softmax-anchor mode (win_beta == NULL): no gate columns, eta = 0, and the
// un-roped key is kept only when win_kr is set.
template <typename T, int HD>
__device__ __forceinline__ void prep_token(const b3_decode_args& a, const StepView& sv, const LinParts& lp, int bh,
                                           int tid, const PrepOut<T>& out) {
  constexpr int HALF = HD / 2, P8 = HALF / 8;
  const int b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const T* row = reinterpret_cast<const T*>(a.lin) + (long long)b * a.lin_row_stride;
  float* ws_stat = out.stat;
  T* q_rope = out.q_rope;
  float* q_raw = out.q_raw;
  const long long wbase = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const int ni = sv.b_start + sv.b_len;   // ring index of the new token
  const int gcol = (a.H + 2 * a.HKV) * HD;
  const int p = tid % P8, u = tid / P8;
  const bool live = u < G + 2;
  const int kind = u < G ? 0 : (u == G ? 1 : 2);   // q, k, v
  const int col = kind == 0 ? (hkv * G + u) * HD : (kind == 1 ? (a.H + hkv) * HD : (a.H + a.HKV + hkv) * HD);
  const bool norm = kind < 2 && a.has_qk_norm;
  float x0[8], x1[8], f[8], w0[8], w1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { x0[e] = 0.f; x1[e] = 0.f; f[e] = 0.f; w0[e] = 0.f; w1[e] = 0.f; }
  // element c of the projection row (8 consecutive ones for lin8)
  auto lin8 = [&](int c, float* out) {
    if (lp.parts) {
      const float* q = lp.parts + (long long)b * a.lin_row_stride + c;
      // every chunk's loads first (at most LP_MAXC chunks), then the sums in chunk order
      f32x4 pl[LP_MAXC], ph[LP_MAXC];
#pragma unroll
      for (int k = 0; k < LP_MAXC; ++k)
        if (k < lp.n_chunks) {
          pl[k] = *reinterpret_cast<const f32x4*>(q + k * lp.chunk_stride);
          ph[k] = *reinterpret_cast<const f32x4*>(q + k * lp.chunk_stride + 4);
        }
      f32x4 lo = pl[0], hi = ph[0];
#pragma unroll
      for (int k = 1; k < LP_MAXC; ++k)
        if (k < lp.n_chunks)
#pragma unroll
          for (int e = 0; e < 4; ++e) { lo[e] += pl[k][e]; hi[e] += ph[k][e]; }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        out[e] = St<T>::rnd(lp.bias ? lo[e] + bf2f(lp.bias[c + e]) : lo[e]);
        out[4 + e] = St<T>::rnd(lp.bias ? hi[e] + bf2f(lp.bias[c + 4 + e]) : hi[e]);
      }
    } else {
      load8<T>(row + c, out);
    }
  };
  auto lin1 = [&](int c) -> float {
    if (lp.parts) {
      const float* q = lp.parts + (long long)b * a.lin_row_stride + c;
      float pv[LP_MAXC];
#pragma unroll
      for (int k = 0; k < LP_MAXC; ++k)
        if (k < lp.n_chunks) pv[k] = q[k * lp.chunk_stride];
      float v = pv[0];
#pragma unroll
      for (int k = 1; k < LP_MAXC; ++k)
        if (k < lp.n_chunks) v += pv[k];
      return St<T>::rnd(lp.bias ? v + bf2f(lp.bias[c]) : v);
    }
    return St<T>::ld(row + c);
  };
  if (live) {
    lin8(col + 8 * p, x0);
    lin8(col + HALF + 8 * p, x1);
    load8<float>(a.inv_freq + 8 * p, f);
    if (norm) {
      const float* w = kind == 0 ? a.qn_w : a.kn_w;
      load8<float>(w + 8 * p, w0);
      load8<float>(w + HALF + 8 * p, w1);
    }
  }
  // the gate logits (eta of the G query heads, beta of the kv head) are loaded with the rows,
  // not after the stores below: the preparation then waits for one memory round trip, not two
  const bool gate = a.win_beta && tid <= G;
  const float gz = gate ? lin1(tid < G ? gcol + a.HKV + hkv * G + tid : gcol + hkv) : 0.f;
  // the RMS statistic needs all P8 lanes of a unit: the shuffles run on every lane
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x0[e] * x0[e] + x1[e] * x1[e];
#pragma unroll
  for (int o = P8 / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if (norm) {
    const float r = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x0[e] = St<T>::rnd(mul_rn(mul_rn(x0[e], r), w0[e]));
      x1[e] = St<T>::rnd(mul_rn(mul_rn(x1[e], r), w1[e]));
    }
  }
  // |q_raw| after the norm, for the readout
  float qq = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) qq += x0[e] * x0[e] + x1[e] * x1[e];
#pragma unroll
  for (int o = P8 / 2; o >= 1; o >>= 1) qq += __shfl_xor(qq, o, 64);
  if (live) {
    if (kind == 2) {
      Vec8<T> v0, v1;
#pragma unroll
      for (int e = 0; e < 8; ++e) { v0.set(e, x0[e]); v1.set(e, x1[e]); }
      T* vo = reinterpret_cast<T*>(a.win_v) + wbase + (long long)ni * HD;
      v0.store(vo + 8 * p);
      v1.store(vo + HALF + 8 * p);
      if (out.new_v) {
        v0.store(out.new_v + 8 * p);
        v1.store(out.new_v + HALF + 8 * p);
      }
    } else {
      const float pos = (float)sv.pos;
      Vec8<T> r0, r1, u0, u1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float sn, cs;
        sincos_rope(mul_rn(pos, f[e]), &sn, &cs);
        const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
        r0.set(e, add_rn(St<T>::rnd(mul_rn(x0[e], c)), St<T>::rnd(mul_rn(-x1[e], si))));
        r1.set(e, add_rn(St<T>::rnd(mul_rn(x1[e], c)), St<T>::rnd(mul_rn(x0[e], si))));
        u0.set(e, x0[e]);
        u1.set(e, x1[e]);
      }
      if (kind == 0) {
        r0.store(q_rope + u * HD + 8 * p);
        r1.store(q_rope + u * HD + HALF + 8 * p);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          q_raw[u * HD + 8 * p + e] = x0[e];
          q_raw[u * HD + HALF + 8 * p + e] = x1[e];
        }
        if (p == 0) ws_stat[2 * u] = 1.0f / fmaxf(sqrtf(qq), 1e-12f);
      } else {
        T* kp = reinterpret_cast<T*>(a.win_kp) + wbase + (long long)ni * HD;
        if (a.win_kr) {
          T* kr = reinterpret_cast<T*>(a.win_kr) + wbase + (long long)ni * HD;
          u0.store(kr + 8 * p);
          u1.store(kr + HALF + 8 * p);
        }
        r0.store(kp + 8 * p);
        r1.store(kp + HALF + 8 * p);
        if (out.new_k) {
          r0.store(out.new_k + 8 * p);
          r1.store(out.new_k + HALF + 8 * p);
        }
      }
    }
  }
  if (tid < G) ws_stat[2 * tid + 1] = a.win_beta ? St<T>::rnd(tanhf(gz)) : 0.f;
  if (tid == G && a.win_beta) {
    a.win_beta[b * a.wb_sb + hkv * a.wb_sh + ni] = St<T>::rnd(1.0f / (1.0f + expf(-gz)));
    if (bh == 0 && a.win_pos) a.win_pos[ni] = (float)sv.pos;
  }
}

template <typename T, int HD>
__global__ void __launch_bounds__(128) decode_prep_kernel(b3_decode_args a, LinParts lp) {
  const int bh = blockIdx.x;
  const int G = a.H / a.HKV;
  float* ws = a.work + (long long)bh * dec_ws_per_bh(G, HD);
  const PrepOut<T> out{reinterpret_cast<T*>(ws + dec_ws_q(G, HD)), ws + dec_ws_q(G, HD) + G * HD,
                       ws + dec_ws_q(G, HD) - 2 * G, nullptr, nullptr};
  prep_token<T, HD>(a, step_view(a), lp, bh, threadIdx.x, out);
}

// Key-row fragment of a 32-key tile (fp32 storage): lane (key n = lane%32, h = lane/32) holds
// the K sub-index 2*ks + h of its key row.
template <typename T, int HD> struct RowFrag;
template <int HD> struct RowFrag<float, HD> {
  static constexpr int NK = HD / 2;
  float v[NK];
  __device__ __forceinline__ void load(const float* row, int h) {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) v[ks] = row[2 * ks + h];
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) v[ks] = 0.f;
  }
  __device__ __forceinline__ void from_lds(const float* x, int h) {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) v[ks] = x[2 * ks + h];
  }
};

template <typename T, int HD>
__global__ void __launch_bounds__(DNT) decode_split_kernel(b3_decode_args a) {
  static_assert(!St<T>::is_bf16, "bf16 steps run decode_attn_kernel");
  using Sm = SplitSmem<T, HD>;
  __shared__ Sm sm;
  constexpr int NDB = HD / 32;
  const int bh = blockIdx.y, b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 31, h = lane >> 5;
  const long long wbase = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const int ns = a.n_sink_keys, nsl = a.has_slots ? a.S : 0, na = a.a_len, nbk = a.b_len + 1;
  const int nk = ns + nsl + na + nbk;
  const int nsplit = dec_nsplit(nk);
  const int split = blockIdx.x;
  float* ws = a.work + (long long)bh * dec_ws_per_bh(G, HD);
  float* ws_read = ws + NPART * G * (HD + 2);

  if (split >= nsplit) {
    // ---------------- rows [RROWS*r, RROWS*r + RROWS) of the M_res readout
    const int r = split - nsplit;
    constexpr int CG = DNT / HD;            // row groups
    constexpr int RPT = RROWS / CG;         // rows per thread
    const int d = tid % HD, cg = tid / HD;
    float m[RPT];
    const float* M = a.m_res ? a.m_res + (long long)bh * HD * HD : nullptr;
#pragma unroll
    for (int q = 0; q < RPT; ++q) m[q] = M ? M[(long long)(RROWS * r + cg + CG * q) * HD + d] : 0.f;
    const float* q_raw = ws + dec_ws_q(G, HD) + G * HD;
    for (int it = tid; it < G * HD; it += DNT) sm.qr[it / HD][it % HD] = q_raw[it];
    __syncthreads();
    float acc[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) acc[g] = 0.f;
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int c = RROWS * r + cg + CG * q;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) acc[g] += sm.qr[g][c] * m[q];
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      if (g < G) sm.u.part[cg][g][d] = acc[g];
    __syncthreads();
    for (int it = tid; it < G * HD; it += DNT) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < CG; ++q) s += sm.u.part[q][it / HD][it % HD];
      ws_read[r * G * HD + it] = s;
    }
    return;
  }

  // ---------------- attention: wavefront `wave` takes keys kt0 .. kt0+31 of the list
  //   [sinks | attractor slots | window A | window B + new token]
  const int kt0 = split * KWG + 32 * wave;
  const int key = kt0 + n;                     // this lane's key row
  const bool kin = key < nk;
  const T* kp = nullptr;
  const T* vp = nullptr;
  float bias_r = 0.f;
  if (kin) {
    int k = key;
    if (k < ns) {
      const long long o = (long long)b * a.s_sb + (long long)hkv * a.s_sh + (long long)k * HD;
      kp = reinterpret_cast<const T*>(a.sink_k) + o;
      vp = reinterpret_cast<const T*>(a.sink_v) + o;
    } else if ((k -= ns) < nsl) {
      kp = reinterpret_cast<const T*>(a.slot_k) + ((long long)bh * a.S + k) * HD;
      vp = reinterpret_cast<const T*>(a.slot_v) + ((long long)bh * a.S + k) * HD;
      bias_r = a.slot_bias[(long long)bh * a.S + k];
    } else if ((k -= nsl) < na) {
      kp = reinterpret_cast<const T*>(a.win_kp) + wbase + (long long)(a.a_start + k) * HD;
      vp = reinterpret_cast<const T*>(a.win_v) + wbase + (long long)(a.a_start + k) * HD;
    } else {   // window B, the new token (appended by decode_prep_kernel) included
      k -= na;
      kp = reinterpret_cast<const T*>(a.win_kp) + wbase + (long long)(a.b_start + k) * HD;
      vp = reinterpret_cast<const T*>(a.win_v) + wbase + (long long)(a.b_start + k) * HD;
    }
  }
  RowFrag<T, HD> kf, vf;
  if (kp) kf.load(kp, h);
  else kf.zero();
  if (vp) vf.load(vp, h);
  else vf.zero();
  // query rows: G prepared rows from the workspace, rows G..31 zero
  {
    const T* qsrc = reinterpret_cast<const T*>(ws + dec_ws_q(G, HD));
    for (int it = tid; it < 32 * (HD / 8); it += DNT) {
      const int rr = it / (HD / 8), c8 = (it % (HD / 8)) * 8;
      Vec8<T> x;
      if (rr < G) x.load(qsrc + rr * HD + c8);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x.set(e, 0.f);
      }
      x.store(&sm.qt[rr * Sm::QS + c8]);
    }
  }
  if (h == 0) sm.bias[wave][n] = bias_r;
  __syncthreads();

  // ---- S^T[key][head] = K . Q^T (heads as the columns)
  f32x16 sc = zero16();
#pragma unroll 8
  for (int ks = 0; ks < HD / 2; ++ks) mma_f32(sc, kf.v[ks], sm.qt[n * Sm::QS + 2 * ks + h]);
  // V^T of the tile into LDS while the scores are finished
  {
    T* vt = sm.u.vt[wave];
#pragma unroll
    for (int ks = 0; ks < HD / 2; ++ks) vt[(2 * ks + h) * Sm::VS + n] = vf.v[ks];
  }
  const float scale = 1.0f / sqrtf((float)HD);
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kr = d_row(lane, r);
    float x = add_rn(mul_rn(sc[r], scale), sm.bias[wave][kr]);
    x = kt0 + kr < nk ? x : -INFINITY;
    sc[r] = x;
    mx = fmaxf(mx, x);
  }
  mx = fmaxf(mx, xor32(mx));
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float e = mx == -INFINITY ? 0.f : expf(sc[r] - mx);
    sc[r] = e;
    sum += e;
  }
  sum += xor32(sum);
  // ---- O^T[d][head] = V^T . P~^T with p~ = exp(x - max) rounded to the storage dtype
  __syncthreads();   // V^T tiles written
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = zero16();
  const T* vt = sm.u.vt[wave];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d = 32 * db + n;
#pragma unroll
    for (int r = 0; r < 16; ++r) mma_f32(o[db], vt[d * Sm::VS + d_row(lane, r)], sc[r]);
  }
  // ---- merge the four tiles of the workgroup: lane column n = head, rows = features
  if (n < G && h == 0) {
    sm.wm[wave][n] = mx;
    sm.wl[wave][n] = sum;
  }
  __syncthreads();   // every wavefront is done with its V^T tile (the union is reused below)
  if (n < G) {
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < DWAVES; ++w) m = fmaxf(m, sm.wm[w][n]);
    const float f = mx == -INFINITY ? 0.f : expf(mx - m);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<float4*>(&sm.u.part[wave][n][32 * db + 8 * r4 + 4 * h]) =
            make_float4(o[db][4 * r4] * f, o[db][4 * r4 + 1] * f, o[db][4 * r4 + 2] * f, o[db][4 * r4 + 3] * f);
  }
  __syncthreads();
  float* pw = ws + (long long)split * G * (HD + 2);
  for (int it = tid; it < G * (HD / 4); it += DNT) {
    const int g = it / (HD / 4), d4 = (it % (HD / 4)) * 4;
    float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < DWAVES; ++w) {
      const float4 x = *reinterpret_cast<const float4*>(&sm.u.part[w][g][d4]);
      acc4.x += x.x; acc4.y += x.y; acc4.z += x.z; acc4.w += x.w;
    }
    *reinterpret_cast<float4*>(pw + g * (HD + 2) + d4) = acc4;
  }
  if (tid < G) {
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < DWAVES; ++w) m = fmaxf(m, sm.wm[w][tid]);
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < DWAVES; ++w) l += sm.wm[w][tid] == -INFINITY ? 0.f : sm.wl[w][tid] * expf(sm.wm[w][tid] - m);
    pw[tid * (HD + 2) + HD] = m;
    pw[tid * (HD + 2) + HD + 1] = l;
  }
}

// Merge the partial softmaxes of one (batch, kv head), round; finish and add the readout.
template <typename T, int HD>
__global__ void __launch_bounds__(DNT) decode_combine_kernel(b3_decode_args a) {
  static_assert(!St<T>::is_bf16, "bf16 steps run decode_attn_kernel");
  constexpr int NREAD = HD / RROWS;
  constexpr int PER = GMAX * HD / DNT;   // outputs per thread at most
  __shared__ float red[GMAX][DNT / 64];
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x;
  const int nk = a.n_sink_keys + (a.has_slots ? a.S : 0) + a.a_len + a.b_len + 1;
  const int npart = dec_nsplit(nk);
  const float* ws = a.work + (long long)bh * dec_ws_per_bh(G, HD);
  const float* ws_read = ws + NPART * G * (HD + 2);
  const float* ws_stat = ws_read + NREAD * G * HD;
  const float coef = div_rn(1.0f - a.gamma[hkv], sqrtf((float)HD));
  float att[PER], ym[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int it = tid + DNT * q;
    att[q] = 0.f;
    ym[q] = 0.f;
    if (it < G * HD) {
      const int g = it / HD, d = it % HD;
      float m = -INFINITY;
      for (int s = 0; s < npart; ++s) m = fmaxf(m, ws[(s * G + g) * (HD + 2) + HD]);
      float l = 0.f, o = 0.f;
      for (int s = 0; s < npart; ++s) {
        const float ms = ws[(s * G + g) * (HD + 2) + HD];
        const float w = ms == -INFINITY ? 0.f : expf(ms - m);
        l += ws[(s * G + g) * (HD + 2) + HD + 1] * w;
        o += ws[(s * G + g) * (HD + 2) + d] * w;
      }
      att[q] = St<T>::rnd(o / l);
      float r = 0.f;
#pragma unroll
      for (int k = 0; k < NREAD; ++k) r += ws_read[k * G * HD + it];
      ym[q] = mul_rn(r * ws_stat[2 * g], coef);
    }
  }
  // mean square of ym per head: wavefront sums, then across wavefronts
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= G) break;
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int it = tid + DNT * q;
      if (it < G * HD && it / HD == g) ss += ym[q] * ym[q];
    }
    ss = wave_sum(ss);
    if (lane == 0) red[g][wv] = ss;
  }
  __syncthreads();
  T* y = reinterpret_cast<T*>(a.y) + (long long)b * a.H * HD + (long long)hkv * G * HD;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int it = tid + DNT * q;
    if (it < G * HD) {
      const int g = it / HD, d = it % HD;
      float ss = 0.f;
#pragma unroll
      for (int w = 0; w < DNT / 64; ++w) ss += red[g][w];
      const float rs = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
      const float ymn = mul_rn(mul_rn(ym[q], rs), a.res_w[d]);
      const float rd = a.m_res ? St<T>::rnd(mul_rn(ws_stat[2 * g + 1], ymn)) : 0.f;
      y[it] = St<T>::from_f(St<T>::rnd(add_rn(att[q], rd)));
    }
  }
}

// ---------------------------------------------------------------- bf16 attention + readout, one workgroup per bh
//
// decode_attn_kernel, grid (B*HKV), 8 wavefronts, two workgroups per CU: the whole step of
// one (batch, kv head) after the head preparation.  Wavefronts 0-3 take the 32-key tiles of
// the key list [sinks | slots | window A | window B + new token] (tile j to wavefront j % 4),
// with an online softmax per query head over a wavefront's tiles.  Per tile the key rows and
// slot biases go to registers and the value rows to the wavefront's LDS buffer (global->LDS
// loads, the 16-byte pieces of row r permuted by p ^ (r % (HD/8))); S^T = K Q^T with
// v_mfma_f32_16x16x32_bf16 (keys as rows, the G query heads as columns), fp32 scores with the
// slot bias, probabilities rounded to bf16, O^T += V^T P^T with the value rows read
// transposed (ds_read_b64_tr_b16).  Wavefronts 4-7 each multiply a quarter of the rows of
// M_res by the normalised query with fp32 MFMAs (v_mfma_f32_16x16x4f32: rows of M as the A
// operand, the query heads as columns).  The softmax states and readout parts are merged in
// LDS, the attention output rounded, the readout finished
// (eta * RMSNorm(normalize(q_raw) M (1-gamma)/sqrt(HD))) and added, and y written.
constexpr int ADW = 6;             // attention wavefronts
constexpr int ARW = 2;             // readout wavefronts
constexpr int ANT = 64 * (ADW + ARW);

template <int HD>
struct AttnDecSmem {
  static constexpr int TILE = 32 * HD;   // bf16 elements of one value tile
  union {
    alignas(16) uint16_t vrow[ADW][TILE];
    struct {
      float o[ADW][GMAX][HD];            // unnormalised attention outputs of the wavefronts
      float rd[ARW][GMAX][HD];           // readout parts
    } mg;
  } u;
  float wm[ADW][GMAX], wl[ADW][GMAX];
  float wt[GMAX][ADW], lsum[GMAX];       // merge weights exp(m_w - m) and normaliser per head
  float red[GMAX][ANT / 64];
  // the prepared token: roped queries, normalised un-roped queries, (1/|q_raw|, eta) per head,
  // and the new key (roped) and value rows
  alignas(16) uint16_t qrope[GMAX][HD];
  alignas(16) float qhat[GMAX][HD];
  float stat[2 * GMAX];
  alignas(16) uint16_t newk[HD];
  alignas(16) uint16_t newv[HD];
};

template <int HD>
__global__ void __launch_bounds__(ANT, 4) decode_attn_kernel(b3_decode_args a, LinParts lp) {
  using Sm = AttnDecSmem<HD>;
  __shared__ Sm sm;
  constexpr int NP = HD / 8, RPI = 64 / NP, NKS = HD / 32, NDB = HD / 16;
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV;
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long long wbase = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const StepView sv = step_view(a);
  const int ns = sv.n_sink, nsl = sv.has_slots ? a.S : 0, na = sv.a_len, nbk = sv.b_len + 1;
  const int nk = ns + nsl + na + nbk;
  const int ntile = (nk + 31) / 32;
  constexpr int PER = (GMAX * HD + ANT - 1) / ANT;
  float c_rw[PER];   // res_norm weight of this thread's outputs (g, d) = (it / HD, it % HD)
#pragma unroll
  for (int qq = 0; qq < PER; ++qq) {
    const int it = tid + ANT * qq;
    c_rw[qq] = it < G * HD ? a.res_w[it % HD] : 0.f;
  }
  const float gam = a.gamma[hkv];   // used in the merge; no wait here

  const int m = lane & 15, g4 = lane >> 4;
  float mx = -INFINITY, sum = 0.f;   // running softmax state of head column m
  f32x4 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 rdv[HD / 16];   // readout wavefronts: r^T[16dt + 4(l/16) + i][head l%16]

  // key k of the list -> its key and value rows and slot bias (0 outside the slots)
  auto key_rows = [&](int key, const uint16_t*& kp, const uint16_t*& vp, int& slot) {
    int k = min(key, nk - 1);
    slot = -1;
    if (k < ns) {
      const long long off = (long long)b * a.s_sb + (long long)hkv * a.s_sh + (long long)k * HD;
      kp = reinterpret_cast<const uint16_t*>(a.sink_k) + off;
      vp = reinterpret_cast<const uint16_t*>(a.sink_v) + off;
    } else if ((k -= ns) < nsl) {
      kp = reinterpret_cast<const uint16_t*>(a.slot_k) + ((long long)bh * a.S + k) * HD;
      vp = reinterpret_cast<const uint16_t*>(a.slot_v) + ((long long)bh * a.S + k) * HD;
      slot = k;
    } else if ((k -= nsl) < na) {
      kp = reinterpret_cast<const uint16_t*>(a.win_kp) + wbase + (long long)(sv.a_start + k) * HD;
      vp = reinterpret_cast<const uint16_t*>(a.win_v) + wbase + (long long)(sv.a_start + k) * HD;
    } else {
      k -= na;
      kp = reinterpret_cast<const uint16_t*>(a.win_kp) + wbase + (long long)(sv.b_start + k) * HD;
      vp = reinterpret_cast<const uint16_t*>(a.win_v) + wbase + (long long)(sv.b_start + k) * HD;
    }
  };
  // one tile's loads: the value rows to LDS (instruction ch fills rows RPI*ch .. RPI*ch +
  // RPI-1, 1 KB), the key rows to registers (lane (m, g4): features 32ks + 8g4 .. of key
  // kt0 + 16kb + m) and the slot biases of the lane's score rows (keys kt0 + 16kb + 4g4 + i)
  uint16_t* vbuf = sm.u.vrow[wave];
  u16x8 ka[2][NKS];
  float bb[2][4];
  auto load_tile = [&](int j) {
    const int kt0 = 32 * j;
#pragma unroll
    for (int ch = 0; ch < 32 / RPI; ++ch) {
      const int r = RPI * ch + lane / NP, piece = (lane % NP) ^ (r % NP);
      const uint16_t* kp;
      const uint16_t* vp;
      int sl;
      key_rows(kt0 + r, kp, vp, sl);
      dec_dma16(vp + 8 * piece, vbuf + ch * 512);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const uint16_t* kp;
      const uint16_t* vp;
      int sl;
      key_rows(kt0 + 16 * kb + m, kp, vp, sl);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) ka[kb][ks] = *reinterpret_cast<const u16x8*>(kp + 32 * ks + 8 * g4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        key_rows(kt0 + 16 * kb + 4 * g4 + i, kp, vp, sl);
        bb[kb][i] = sl >= 0 ? a.slot_bias[(long long)bh * a.S + sl] : 0.f;
      }
    }
  };
  // attention wavefronts: the first tile goes out before the head preparation is waited for;
  // readout wavefronts: the head preparation of the new token into LDS and the window ring
  if (wave < ADW) {
    if (wave < ntile) load_tile(wave);
  } else {
    const PrepOut<uint16_t> po{&sm.qrope[0][0], &sm.qhat[0][0], sm.stat, sm.newk, sm.newv};
    prep_token<uint16_t, HD>(a, sv, lp, bh, tid - 64 * ADW, po);
  }
  __syncthreads();   // the prepared token is in LDS
  if (wave < ADW) {
    // queries as the B operand: lane (head m, group g4) holds features 32ks + 8g4 .. of head m
    // (read from LDS at every tile rather than held in registers for the whole loop)
    const int qrow = m < G ? m : 0;
    const bool qlive = m < G;
    const float scale = 1.0f / sqrtf((float)HD);
    for (int j = wave; j < ntile; j += ADW) {
      const int kt0 = 32 * j;
      if (j != wave) load_tile(j);
      // the new token (key nk - 1) was read from the ring before it was written there: its
      // key row comes from LDS instead (its value row below)
      const int r_new = nk - 1 - kt0;
      if (r_new < 32) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          if (16 * kb + m == r_new)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) ka[kb][ks] = *reinterpret_cast<const u16x8*>(&sm.newk[32 * ks + 8 * g4]);
      }
      f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        u16x8 qb = *reinterpret_cast<const u16x8*>(&sm.qrope[qrow][32 * ks + 8 * g4]);
        if (!qlive) qb = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) mma16_bf16(sc[kb], ka[kb][ks], qb);
      }
      // fp32 scores (the decoder step does not round q.k), slot bias, keys past nk masked
      float tmx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kt0 + 16 * kb + 4 * g4 + i;
          float x = add_rn(mul_rn(sc[kb][i], scale), bb[kb][i]);
          x = key < nk ? x : -INFINITY;
          sc[kb][i] = x;
          tmx = fmaxf(tmx, x);
        }
      tmx = fmaxf(tmx, __shfl_xor(tmx, 16, 64));
      tmx = fmaxf(tmx, __shfl_xor(tmx, 32, 64));
      const float nmx = fmaxf(mx, tmx);
      const float f = mx == -INFINITY ? 0.f : expf(mx - nmx);
      float ts = 0.f;
      u16x8 pb;   // P^T operand: keys 4g4 + i (i < 4) and 16 + 4g4 + i - 4
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = nmx == -INFINITY ? 0.f : expf(sc[kb][i] - nmx);
          ts += e;
          pb[4 * kb + i] = f2bf(e);
        }
      ts += __shfl_xor(ts, 16, 64);
      ts += __shfl_xor(ts, 32, 64);
      sum = sum * f + ts;
      mx = nmx;
      // every load of the tile (the value rows in LDS included) has landed
      wait_vm<0>();
      // the new token's value row from LDS, in its own row and in every row after it: keys past
      // nk - 1 were clamped to its ring position, read before the token was written there, and
      // their zero probabilities must not meet whatever that memory held (0 * NaN is NaN)
      if (r_new < 32)
        for (int it = lane; it < (32 - r_new) * NP; it += 64) {
          const int rr = r_new + it / NP, pc = it % NP;
          *reinterpret_cast<u16x8*>(vbuf + rr * HD + 8 * (pc ^ (rr % NP))) =
              *reinterpret_cast<const u16x8*>(&sm.newv[8 * pc]);
        }
      const int s = lane & 15;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int r1 = 4 * g4 + (s >> 2), r2 = r1 + 16;
        const int pc = 2 * db + ((s & 3) >> 1), off = 4 * (s & 1);
        u16x4 lo = dec_read_tr(vbuf + r1 * HD + 8 * (pc ^ (r1 % NP)) + off);
        u16x4 hi = dec_read_tr(vbuf + r2 * HD + 8 * (pc ^ (r2 % NP)) + off);
        dec_lds_wait(lo, hi);
        u16x8 av;
#pragma unroll
        for (int e = 0; e < 4; ++e) { av[e] = lo[e]; av[4 + e] = hi[e]; }
#pragma unroll
        for (int e = 0; e < 4; ++e) o[db][e] *= f;
        mma16_bf16(o[db], av, pb);
      }
    }
  }
  if (wave >= ADW && a.m_res) {
    // r^T[d][g] = sum over the wavefront's rows c of M[c][d] q^[g][c]: 16x16x4 fp32 MFMAs,
    // lane (l % 16, l / 16) loads A = M[c0 + l/16][d0 + l%16] and B = q^[l%16][c0 + l/16]
    constexpr int RR = HD / ARW, NDT = HD / 16;
    constexpr int NCS = RR / 4 < 4 ? RR / 4 : 4;   // K steps of 4 rows per pass (register budget)
    constexpr int NPASS = RR / (4 * NCS);
    const int q = wave - ADW;
    const int r16 = lane & 15, k4 = lane >> 4;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) rdv[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int c0 = q * RR + 4 * NCS * ps;
      const float* M = a.m_res + (long long)bh * HD * HD + (long long)(c0 + k4) * HD + r16;
      float ma[NCS][NDT];
#pragma unroll
      for (int cs = 0; cs < NCS; ++cs)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) ma[cs][dt] = M[(long long)(4 * cs) * HD + 16 * dt];
      float qv[NCS];
#pragma unroll
      for (int cs = 0; cs < NCS; ++cs) qv[cs] = r16 < G ? sm.qhat[r16][c0 + 4 * cs + k4] : 0.f;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int cs = 0; cs < NCS; ++cs) rdv[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ma[cs][dt], qv[cs], rdv[dt], 0, 0, 0);
    }
  }
  __syncthreads();   // every wavefront is done with its value tiles (the union is reused below)
  if (wave < ADW) {
    if (m < G) {
      if (g4 == 0) {
        sm.wm[wave][m] = mx;
        sm.wl[wave][m] = sum;
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        *reinterpret_cast<float4*>(&sm.u.mg.o[wave][m][16 * db + 4 * g4]) =
            make_float4(o[db][0], o[db][1], o[db][2], o[db][3]);
    }
  } else {
    const int q = wave - ADW;
    if (m < G)
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.u.mg.rd[q][m][16 * dt + 4 * g4 + i] = a.m_res ? rdv[dt][i] : 0.f;
  }
  __syncthreads();
  // merge weights of the wavefronts' softmax states, once per head
  if (tid < G) {
    const int g = tid;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < ADW; ++w) mm = fmaxf(mm, sm.wm[w][g]);
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < ADW; ++w) {
      const float ms = sm.wm[w][g];
      const float wt = ms == -INFINITY ? 0.f : expf(ms - mm);
      sm.wt[g][w] = wt;
      l += sm.wl[w][g] * wt;
    }
    sm.lsum[g] = l;
  }
  __syncthreads();
  // merge: thread (g, d) for g < G
  const float coef = div_rn(1.0f - gam, sqrtf((float)HD));
  float att[PER], ym[PER];
#pragma unroll
  for (int qq = 0; qq < PER; ++qq) {
    const int it = tid + ANT * qq;
    att[qq] = 0.f;
    ym[qq] = 0.f;
    if (it < G * HD) {
      const int g = it / HD, d = it % HD;
      float ov = 0.f;
#pragma unroll
      for (int w = 0; w < ADW; ++w) ov += sm.u.mg.o[w][g][d] * sm.wt[g][w];
      att[qq] = round_bf(ov / sm.lsum[g]);
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < ARW; ++w) r += sm.u.mg.rd[w][g][d];
      ym[qq] = mul_rn(r * sm.stat[2 * g], coef);
    }
  }
  // mean square of ym per head: wavefront sums, then across wavefronts
  const int wv = tid >> 6;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= G) break;
    float ss = 0.f;
#pragma unroll
    for (int qq = 0; qq < PER; ++qq) {
      const int it = tid + ANT * qq;
      if (it < G * HD && it / HD == g) ss += ym[qq] * ym[qq];
    }
    ss = wave_sum(ss);
    if (lane == 0) sm.red[g][wv] = ss;
  }
  __syncthreads();
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y) + (long long)b * a.H * HD + (long long)hkv * G * HD;
#pragma unroll
  for (int qq = 0; qq < PER; ++qq) {
    const int it = tid + ANT * qq;
    if (it < G * HD) {
      const int g = it / HD;
      float ss = 0.f;
#pragma unroll
      for (int w = 0; w < ANT / 64; ++w) ss += sm.red[g][w];
      const float rs = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
      const float ymn = mul_rn(mul_rn(ym[qq], rs), c_rw[qq]);
      const float rd = a.m_res ? round_bf(mul_rn(sm.stat[2 * g + 1], ymn)) : 0.f;
      y[it] = f2bf(round_bf(add_rn(att[qq], rd)));
    }
  }
}

// ---------------------------------------------------------------- projections of the decode layer
//
// y[m][n] = round(sum_k x[m][k] * W[n][k] + bias[n]) for few rows m (the batch of one-token
// decode steps) and a row-major weight W[N][K] (nn.Linear layout).  The product is bound by
// streaming W once, so every W element is read once and x, which every weight row needs, is
// shared: a workgroup takes 8 tiles of 16 weight rows (one per wavefront) and one chunk of PKC
// columns of K, stages x[64 rows][chunk] in LDS with global->LDS loads, and its wavefronts
// multiply their W rows (loaded straight into MFMA operand registers, all steps of the chunk
// before the first MFMA) by the staged x (v_mfma_f32_16x16x32_bf16: W rows as the A operand,
// x rows as the B columns).  Each workgroup writes the fp32 partial product of its chunk to
// parts[chunk][m][n]; the consumer adds the chunks in order, adds the bias and rounds once
// (the decode prep kernel for the input projection, proj_reduce_kernel for o_proj).  The
// number of tiles per workgroup (NW, 4 to 8) is the smallest that keeps the grid within one
// workgroup per compute unit, so that every compute unit streams its share of W: at B = 64 the
// Qwen3-4B input projection takes 245 workgroups of 8 and o_proj 256 of 5 (160 of 8 would leave
// 96 compute units idle).
constexpr int PKC = 512;               // K columns per chunk
constexpr int PKS = PKC / 32;          // MFMA K steps per chunk
constexpr int PXS = PKC * 2 + 16;      // LDS bytes per staged x row (16-byte pad: conflict-free reads)

__host__ __device__ inline int proj_chunks(int K) { return (K + PKC - 1) / PKC; }
// floats of the fp32 partial products of one projection
__host__ __device__ inline long long proj_parts_floats(int M, int N, int K) {
  return (long long)proj_chunks(K) * M * N;
}

// ds_read_b128 of a staged x row at a compile-time byte offset (inline assembly, as dec_read_tr:
// an ordinary LDS read would make the compiler wait for every outstanding W load first)
template <int OFF>
__device__ __forceinline__ u16x8 rp_read_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  u16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
// lgkmcnt(N), tied to the four x operands of one K step
template <int N>
__device__ __forceinline__ void rp_lds_wait(u16x8 (&x)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]) : "i"(N));
}

struct ProjArgs {
  const uint16_t* x; int64_t x_rs;
  const uint16_t* w;
  float* parts;                        // [chunk][M][N]
  int M, N, K;
};

template <int I>
__device__ __forceinline__ void rp_read_step(u16x8 (&x)[4], uint32_t base) {
  static_assert(48 * PXS + 64 * I < 65536, "ds offset range");
  x[0] = rp_read_at<64 * I>(base);
  x[1] = rp_read_at<16 * PXS + 64 * I>(base);
  x[2] = rp_read_at<32 * PXS + 64 * I>(base);
  x[3] = rp_read_at<48 * PXS + 64 * I>(base);
}
// K step I of the chunk: the x reads of step I + 1 go out before the MFMAs of step I.  The W
// loads were issued in step order and complete in order: quarter q of the steps waits until at
// most the later quarters' loads are outstanding.  Steps past the chunk multiply zeros.
template <int I>
__device__ __forceinline__ void rp_step(f32x4 (&acc)[4], u16x8 (&wa)[PKS], u16x8 (&xb)[2][4], uint32_t base,
                                        int nst) {
  constexpr int C = I & 1;
  __builtin_amdgcn_sched_barrier(0);   // nothing of this step moves above the wait of its quarter
  if constexpr (I + 1 < PKS) rp_read_step<I + 1>(xb[C ^ 1], base);
  if constexpr (I > 0 && I % (PKS / 4) == 0) {
    wait_vm<PKS - PKS / 4 - I>();
    __builtin_amdgcn_sched_barrier(0);
  }
  if (I >= nst) wa[I] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
  if constexpr (I + 1 < PKS) rp_lds_wait<4>(xb[C]);
  else rp_lds_wait<0>(xb[C]);
#pragma unroll
  for (int t = 0; t < 4; ++t) mma16_bf16(acc[t], wa[I], xb[C][t]);
}
template <int... I>
__device__ __forceinline__ void rp_steps(f32x4 (&acc)[4], u16x8 (&wa)[PKS], u16x8 (&xb)[2][4], uint32_t base,
                                         int nst, std::integer_sequence<int, I...>) {
  (rp_step<I>(acc, wa, xb, base, nst), ...);
}

template <int NW>
__global__ void __launch_bounds__(64 * NW, 2) rowproj_kernel(ProjArgs p) {
  constexpr int XR = (64 + NW - 1) / NW;           // staged x rows per wavefront
  __shared__ __attribute__((aligned(16))) unsigned char xs[64 * PXS];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nt = blockIdx.x * NW + wv;             // this wavefront's 16-row tile of W
  const int ch = blockIdx.y, m0 = blockIdx.z * 64;
  const int kc0 = ch * PKC;
  const int nst = min(PKS, (p.K - kc0) >> 5);      // K steps in this chunk
  const int r = lane & 15, kg = lane >> 4;
  const bool live = nt * 16 < p.N;
  // x rows m0 .. m0+63 of the chunk, one 1 KB row per global->LDS load (lane: 8 columns);
  // rows past M repeat row M - 1 and columns past K repeat the last 8 (both multiply zeros
  // or are never stored)
#pragma unroll
  for (int j = 0; j < XR; ++j) {
    const int m = wv * XR + j;
    if (m >= 64) break;   // uniform across the wavefront
    const uint16_t* src = p.x + (long long)min(m0 + m, p.M - 1) * p.x_rs + min(kc0 + 8 * lane, p.K - 8);
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(xs + m * PXS), 16, 0, 0);
  }
  // the W rows: all steps of the chunk, in flight together with the x loads (steps past the
  // chunk re-read its last step and multiply a zero operand, set once their quarter has arrived)
  u16x8 wa[PKS];
  if (live) {
    const uint16_t* wrow = p.w + (long long)(nt * 16 + r) * p.K + kc0 + 8 * kg;
#pragma unroll
    for (int i = 0; i < PKS; ++i) {
      wa[i] = *reinterpret_cast<const u16x8*>(wrow + 32 * min(i, nst - 1));
      __builtin_amdgcn_sched_barrier(0);   // issued in step order: the waits below count on it
    }
  }
  // the x rows and the first quarter of the W steps (in-order completion: at most the other
  // quarters' 3 PKS / 4 loads still outstanding); each quarter multiplies while the later ones
  // arrive.  A wavefront past the last W row issued only its x rows: it waits for all of them.
  static_assert(PKS == 16, "vmcnt below");
  if (live) __builtin_amdgcn_s_waitcnt(12 | (7 << 4) | (15 << 8));   // vmcnt(12)
  else __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));         // vmcnt(0)
  sync_lds();   // every wavefront's x rows are in LDS (a barrier without a drain of the W loads)
  if (!live) return;
  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // x operand of tile t, step i: row 16 t + r, bytes 64 i + 16 kg of it
  const uint32_t xbase = (uint32_t)(size_t)((__attribute__((address_space(3))) unsigned char*)xs) + r * PXS + 16 * kg;
  u16x8 xb[2][4];
  rp_read_step<0>(xb[0], xbase);
  rp_steps(acc, wa, xb, xbase, nst, std::make_integer_sequence<int, PKS>{});
  // D of tile t: column m = 16t + r, rows n = 4 kg + i: four consecutive n per lane
  float* out = p.parts + (long long)ch * p.M * p.N + nt * 16 + 4 * kg;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int m = m0 + 16 * t + r;
    if (m < p.M) *reinterpret_cast<f32x4*>(out + (long long)m * p.N) = acc[t];
  }
}

// y[m][n] = round(sum over chunks of parts + bias), four n per thread
__global__ void __launch_bounds__(256) proj_reduce_kernel(const float* parts, int n_chunks, int M, int N,
                                                          const uint16_t* bias, uint16_t* y, int64_t y_rs) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int m = i / (N / 4), n = 4 * (i % (N / 4));
  if (m >= M) return;
  f32x4 pc[LP_MAXC];
#pragma unroll
  for (int c = 0; c < LP_MAXC; ++c)
    if (c < n_chunks) pc[c] = *reinterpret_cast<const f32x4*>(parts + ((long long)c * M + m) * N + n);
  f32x4 v = pc[0];
#pragma unroll
  for (int c = 1; c < LP_MAXC; ++c)
    if (c < n_chunks) { v[0] += pc[c][0]; v[1] += pc[c][1]; v[2] += pc[c][2]; v[3] += pc[c][3]; }
  u16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = f2bf(bias ? v[e] + bf2f(bias[n + e]) : v[e]);
  *reinterpret_cast<u16x4*>(y + (long long)m * y_rs + n) = o;
}

static int launch_rowproj(const ProjArgs& p, hipStream_t st) {
  const int n_cu = cu_count();
  if (n_cu < 0) return -n_cu;
  const int tiles = p.N / 16, other = proj_chunks(p.K) * ((p.M + 63) / 64);
  int nw = 8;
  for (int w = 4; w <= 8; ++w)
    if ((long long)(tiles + w - 1) / w * other <= n_cu) { nw = w; break; }
  const dim3 grid((tiles + nw - 1) / nw, proj_chunks(p.K), (p.M + 63) / 64);
  switch (nw) {
    case 4: hipLaunchKernelGGL(rowproj_kernel<4>, grid, dim3(256), 0, st, p); break;
    case 5: hipLaunchKernelGGL(rowproj_kernel<5>, grid, dim3(320), 0, st, p); break;
    case 6: hipLaunchKernelGGL(rowproj_kernel<6>, grid, dim3(384), 0, st, p); break;
    case 7: hipLaunchKernelGGL(rowproj_kernel<7>, grid, dim3(448), 0, st, p); break;
    default: hipLaunchKernelGGL(rowproj_kernel<8>, grid, dim3(512), 0, st, p); break;
  }
  return (int)hipGetLastError();
}

template <typename T, int HD>
static int launch_decode(const b3_decode_args& a, hipStream_t st, LinParts lp) {
  const int BH = a.B * a.HKV;
  const int nk = a.n_sink_keys + (a.has_slots ? a.S : 0) + a.a_len + a.b_len + 1;
  if constexpr (St<T>::is_bf16) {
    hipLaunchKernelGGL((decode_attn_kernel<HD>), dim3(BH), dim3(ANT), 0, st, a, lp);
  } else {
    hipLaunchKernelGGL((decode_prep_kernel<T, HD>), dim3(BH), dim3(128), 0, st, a, lp);
    hipError_t e0 = hipGetLastError();
    if (e0 != hipSuccess) return (int)e0;
    hipLaunchKernelGGL((decode_split_kernel<T, HD>), dim3(dec_nsplit(nk) + HD / RROWS, BH), dim3(DNT), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((decode_combine_kernel<T, HD>), dim3(BH), dim3(DNT), 0, st, a);
  }
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int64_t bolt3_decode_workspace_bytes(int32_t B, int32_t H, int32_t HKV, int32_t HD) {
  if (B <= 0 || HKV <= 0 || H % HKV != 0) return 0;
  return (int64_t)B * HKV * b3::dec_ws_per_bh(H / HKV, HD) * 4;
}

// Argument checks shared by bolt3_decode and bolt3_decode_layer (need_lin: the row comes from
// a->lin rather than from the layer's own projection).
static int check_decode(const b3_decode_args* a, bool need_lin, bool fused) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->H % a->HKV != 0) return B3_ERR_ARG;
  if (a->H / a->HKV > b3::GMAX || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  const bool anchor = a->win_beta == nullptr;   // softmax-anchor mode (fused path only)
  if (!fused && (anchor || !a->win_kr || a->step_desc)) return B3_ERR_ARG;
  if (anchor && (a->has_slots || a->n_sink_keys || a->m_res)) return B3_ERR_ARG;
  if (a->step_desc) {
    // fields come from device memory at run time; the kernels clamp them to the ring
    if (a->ring_cap <= 0) return B3_ERR_ARG;
    if (!anchor && (!a->slot_k || !a->slot_v || !a->slot_bias || !a->sink_k || !a->sink_v)) return B3_ERR_ARG;
  } else {
    if (a->n_sink_keys < 0 || a->a_len < 0 || a->b_len < 0 || a->a_start < 0 || a->b_start < 0) return B3_ERR_ARG;
    const int nk = a->n_sink_keys + (a->has_slots ? a->S : 0) + a->a_len + a->b_len + 1;
    if (!fused && nk > b3::NKMAX) return B3_ERR_UNSUPPORTED;   // the split path's partial-state count
    if (a->ring_cap > 0 && (a->a_start + a->a_len > a->ring_cap || a->b_start + a->b_len + 1 > a->ring_cap))
      return B3_ERR_ARG;
    if (a->has_slots && (!a->slot_k || !a->slot_v || !a->slot_bias)) return B3_ERR_ARG;
    if (a->n_sink_keys > 0 && (!a->sink_k || !a->sink_v)) return B3_ERR_ARG;
  }
  if ((need_lin && !a->lin) || !a->win_kp || !a->win_v || !a->inv_freq || !a->gamma || !a->res_w || !a->y ||
      !a->work)
    return B3_ERR_ARG;
  if (a->work_bytes < bolt3_decode_workspace_bytes(a->B, a->H, a->HKV, a->HD)) return B3_ERR_WORKSPACE;
  if (!anchor && (a->S <= 0 || a->S > 128)) return B3_ERR_UNSUPPORTED;   // the slot field's size
  if (a->has_qk_norm && (!a->qn_w || !a->kn_w)) return B3_ERR_ARG;
  // 16-byte rows: the projection row and every key / value row
  const int64_t es = a->dtype == B3_BF16 ? 2 : 4;
  if ((a->lin_row_stride * es) % 16 || (need_lin && reinterpret_cast<uintptr_t>(a->lin) % 16)) return B3_ERR_ARG;
  return 0;
}

extern "C" int bolt3_decode(const b3_decode_args* a, void* stream) {
  const int rc = check_decode(a, true, false);
  if (rc) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const b3::LinParts lp{nullptr, 0, 0, nullptr};
  if (a->dtype == B3_F32)
    return a->HD == 64 ? b3::launch_decode<float, 64>(*a, st, lp) : b3::launch_decode<float, 128>(*a, st, lp);
  if (a->dtype == B3_BF16)
    return a->HD == 64 ? b3::launch_decode<uint16_t, 64>(*a, st, lp) : b3::launch_decode<uint16_t, 128>(*a, st, lp);
  return B3_ERR_UNSUPPORTED;
}

extern "C" int64_t bolt3_decode_layer_workspace_bytes(int32_t B, int32_t d_model, int32_t n_in, int32_t hd_total,
                                                      int32_t n_out) {
  if (B <= 0 || d_model <= 0 || n_in <= 0 || hd_total <= 0 || n_out <= 0) return 0;
  const long long a = b3::proj_parts_floats(B, n_in, d_model), b = b3::proj_parts_floats(B, n_out, hd_total);
  return (int64_t)(a > b ? a : b) * 4;
}

extern "C" int bolt3_decode_layer(const b3_decode_layer_args* a, void* stream) {
  if (!a) return B3_ERR_ARG;
  const b3_decode_args& d = a->dec;
  if (d.dtype != B3_BF16) return B3_ERR_UNSUPPORTED;
  int rc = check_decode(&d, false, true);
  if (rc) return rc;
  const int hd_total = d.H * d.HD;
  if (!a->x || !a->w_in || !a->w_out || !a->out || !a->proj_work) return B3_ERR_ARG;
  const int n_gates = d.win_beta ? d.HKV + d.H : 0;   // anchor mode: q | k | v only
  if (a->d_model < 32 || a->d_model % 32 || a->n_in != d.lin_row_stride || a->n_in % 16 ||
      a->n_in < d.H * d.HD + 2 * d.HKV * d.HD + n_gates || a->n_out <= 0 || a->n_out % 16 ||
      a->x_row_stride < a->d_model || a->x_row_stride % 8 || a->out_row_stride < a->n_out ||
      a->out_row_stride % 4 || reinterpret_cast<uintptr_t>(a->x) % 16 || reinterpret_cast<uintptr_t>(a->out) % 8 ||
      reinterpret_cast<uintptr_t>(a->proj_work) % 16)
    return B3_ERR_ARG;
  if (b3::proj_chunks(a->d_model) > b3::LP_MAXC || b3::proj_chunks(hd_total) > b3::LP_MAXC) return B3_ERR_UNSUPPORTED;
  if (a->proj_work_bytes < bolt3_decode_layer_workspace_bytes(d.B, a->d_model, a->n_in, hd_total, a->n_out))
    return B3_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const b3::ProjArgs pin{reinterpret_cast<const uint16_t*>(a->x), a->x_row_stride,
                         reinterpret_cast<const uint16_t*>(a->w_in), a->proj_work, d.B, a->n_in, a->d_model};
  rc = b3::launch_rowproj(pin, st);
  if (rc) return rc;
  const b3::LinParts lp{a->proj_work, b3::proj_chunks(a->d_model), (long long)d.B * a->n_in,
                        reinterpret_cast<const uint16_t*>(a->b_in)};
  rc = d.HD == 64 ? b3::launch_decode<uint16_t, 64>(d, st, lp) : b3::launch_decode<uint16_t, 128>(d, st, lp);
  if (rc) return rc;
  const b3::ProjArgs pout{reinterpret_cast<const uint16_t*>(d.y), hd_total,
                          reinterpret_cast<const uint16_t*>(a->w_out), a->proj_work, d.B, a->n_out, hd_total};
  rc = b3::launch_rowproj(pout, st);
  if (rc) return rc;
  const int n_thr = d.B * (a->n_out / 4);
  hipLaunchKernelGGL(b3::proj_reduce_kernel, dim3((n_thr + 255) / 256), dim3(256), 0, st, a->proj_work,
                     b3::proj_chunks(hd_total), d.B, a->n_out, reinterpret_cast<const uint16_t*>(a->b_out),
                     reinterpret_cast<uint16_t*>(a->out), a->out_row_stride);
  return (int)hipGetLastError();
}

extern "C" const char* bolt3_version(void) { return "bolt3_amd 0.1 gfx950 (MFMA 32x32, wave64)"; }

namespace b3 {
__global__ void __launch_bounds__(64) step_advance_kernel(int32_t* desc, int32_t d0, int32_t d1, int32_t d2, int32_t d3,
                                                          int32_t d4) {
  const int i = threadIdx.x;
  const int32_t add = i == 0 ? d0 : i == 1 ? d1 : i == 2 ? d2 : i == 3 ? d3 : d4;
  if (i < 5) desc[i] += add;
}
}  // namespace b3

extern "C" int bolt3_step_advance(int32_t* step_desc, int32_t d_pos, int32_t d_a_start, int32_t d_a_len,
                                  int32_t d_b_start, int32_t d_b_len, void* stream) {
  if (!step_desc) return B3_ERR_ARG;
  hipLaunchKernelGGL(b3::step_advance_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), step_desc,
                     d_pos, d_a_start, d_a_len, d_b_start, d_b_len);
  return (int)hipGetLastError();
}


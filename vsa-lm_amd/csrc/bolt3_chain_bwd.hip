// Backward of the consolidation chain (S = 128, HD in {64, 128}, bf16 or fp32 storage, at most
// 128 tokens per step).
//
// The reference differentiates _consolidate_functional (vsa_lm/config/bolt3.py:68-192) with
// autograd; every decision in it (fill picks, merge targets, evictions, delta-rule membership)
// is taken under no_grad (:98-112, :121-135, :165-180), so the gradient is that of a fixed
// sequence of copies, mass-weighted means and delta-rule updates.  The forward chain's decision
// log and its per-step snapshots (slot mass and mean position, M_res) record that sequence; the
// kernels below walk it backwards:
//   tok_stats_kernel  per (step, bh): 1/|k_j|, the Gershgorin row sums r_j = sum_i |khat_i .
//                     khat_j| w_i and bsafe_j = w_j / max(r_j, 1), w_j = beta_j [j goes to M_res]
//                     (:154-158), the forward's own arithmetic;
//   slot_rec_kernel   per (bh, 16 features): the slots' key / value gradients over the steps in
//                     reverse -- the attention's slot gradients (keys through the transpose of
//                     their RoPE), fills and evictions hand a slot's gradient to its token and
//                     clear it (:145-150, :182-191), merges give token j 1/new_mass of its
//                     slot's gradient and scale the slot's by mass/new_mass (:121-136);
//   m_rec_kernel      per (bh, 32 columns of M): G_i = dM_i + (gamma I - Khat^T diag(bsafe)
//                     Khat) G_{i+1} (the columns evolve independently) and each step's share of
//                     dL/dgamma = sum(G_i * M_{i-1}) (:159-162);
//   tok_grad_kernel   per (step, bh): the delta rule's token gradients with R = V - Khat M_{i-1},
//                     E = bsafe R:  dV = bsafe (Khat G), dKhat = E G^T - dV M^T + (dP + dP^T)
//                     Khat with dP through the row sums (|Khat Khat^T| and the clamp at 1), dw,
//                     and the normalisation's backward to the un-roped keys.
// Products run on bf16 MFMA.  fp32 operands (M, G, E, dV, the Gram weights, and the keys when the
// storage is fp32) are split into bf16 hi + lo; a product of two split operands takes hi*hi +
// hi*lo + lo*hi, so every product is fp32-accurate to about 2^-16 (bf16 keys are exact: one
// product fewer).
#include <math.h>

#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {
namespace cbwd {

constexpr int S = 128;
constexpr int LT = 128;          // tokens per step, at most
constexpr int NPT = LT / 8;      // 16-byte pieces of a row of LT bf16
constexpr int NT = 256;          // threads of the per-step kernels and of slot_rec (4 wavefronts)

template <int HD>
struct Dims {
  static constexpr int NP = HD / 8;     // 16-byte pieces of a row of HD bf16
  static constexpr int NSL = HD / 16;   // feature slices of the slot recursion
  static constexpr int NCB = HD / 32;   // 32-column blocks of M (and wavefronts of m_rec)
  static constexpr int KS = HD / 16;    // K steps of 16 over the features
};

__device__ __forceinline__ int step_len(const b3_chain_bwd_args& a, int i) { return i == 0 ? a.len0 : a.step_len; }
__device__ __forceinline__ int step_off(const b3_chain_bwd_args& a, int i) {
  return i == 0 ? a.off0 : i * a.step_stride;
}
// slots filled before step i (the chain starts from the empty state)
__device__ __forceinline__ int filled_before(const b3_chain_bwd_args& a, int i) {
  int nf = 0;
  for (int s = 0; s < i && nf < S; ++s) nf = min(S, nf + step_len(a, s));
  return nf;
}
__device__ __forceinline__ const float* log_rec(const b3_chain_bwd_args& a, int i, int bh) {
  return a.log + ((long long)i * a.B * a.HKV + bh) * B3_LOG_ROWS * B3_LOG_COLS;
}

// Workspace: per (step, bh) four rows of LT floats (1/|k|, row sum, bsafe, w), then per (step,
// bh) G^T as bf16 hi and lo planes of HD x HD (G^T[d][c] = G[c][d], the layout of the bf16
// forward's M_res snapshots).
__host__ __device__ __forceinline__ long long stats_floats(long long n, long long bh) { return n * bh * 4 * LT; }
__host__ __device__ __forceinline__ long long ws_bytes(long long n, long long bh, int hd) {
  return 4 * stats_floats(n, bh) + n * bh * (long long)hd * hd * 4;
}
__device__ __forceinline__ float* stats_of(const b3_chain_bwd_args& a, int i, int bh) {
  return reinterpret_cast<float*>(a.work) + ((long long)i * a.B * a.HKV + bh) * 4 * LT;
}
template <int HD>
__device__ __forceinline__ uint16_t* gt_of(const b3_chain_bwd_args& a, int i, int bh) {
  const long long BH = (long long)a.B * a.HKV;
  return reinterpret_cast<uint16_t*>(reinterpret_cast<float*>(a.work) + stats_floats(a.n_steps, BH)) +
         ((long long)i * BH + bh) * 2 * HD * HD;
}

// Keys of one step in LDS: [LT][HD] bf16 with 16-byte piece p of row r at p ^ (r % NP), rows >= l
// zero; fp32 storage keeps the bf16 remainder of every key in a second plane.
template <int HD, bool F32>
struct KeyTile {
  alignas(16) uint16_t hi[LT * HD];
  alignas(16) uint16_t lo[F32 ? LT * HD : 8];
};

template <int HD, int NTH>
__device__ __forceinline__ void stage_keys_bf16(KeyTile<HD, false>& kt, const uint16_t* kr_rows, int l, int tid);

template <int HD, bool F32, int NTH>
__device__ __forceinline__ void stage_keys(KeyTile<HD, F32>& kt, const void* kr_rows, int l, int tid) {
  if constexpr (!F32) {
    stage_keys_bf16<HD, NTH>(kt, reinterpret_cast<const uint16_t*>(kr_rows), l, tid);
    return;
  }
  constexpr int NP = Dims<HD>::NP;
  for (int it = tid; it < LT * NP; it += NTH) {
    const int r = it / NP, p = it % NP;
    const int o = r * HD + 8 * (p ^ (r % NP));
    if constexpr (F32) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
      if (r < l) {
        const float* src = reinterpret_cast<const float*>(kr_rows) + (long long)r * HD + 8 * p;
        *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(src);
        *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(src + 4);
      }
      u16x8 h, lw;
      split8(v, h, lw);
      *reinterpret_cast<u16x8*>(&kt.hi[o]) = h;
      *reinterpret_cast<u16x8*>(&kt.lo[o]) = lw;
    } else {
      u16x8 v = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (r < l) v = *reinterpret_cast<const u16x8*>(reinterpret_cast<const uint16_t*>(kr_rows) + (long long)r * HD + 8 * p);
      *reinterpret_cast<u16x8*>(&kt.hi[o]) = v;
    }
  }
}
// bf16: the thread's items in batches of 8, every load of a batch before its stores (one
// memory round trip per batch; a load and its store per iteration would wait for each load)
template <int HD, int NTH>
__device__ __forceinline__ void stage_keys_bf16(KeyTile<HD, false>& kt, const uint16_t* kr_rows, int l, int tid) {
  constexpr int NP = Dims<HD>::NP, N = (LT * NP + NTH - 1) / NTH, NB = N < 8 ? N : 8;
  static_assert(N % NB == 0, "batches of the thread's items");
#pragma unroll
  for (int q0 = 0; q0 < N; q0 += NB) {
    u16x8 v[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int it = tid + NTH * (q0 + q), r = it / NP, p = it % NP;
      v[q] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (it < LT * NP && r < l) v[q] = *reinterpret_cast<const u16x8*>(kr_rows + (long long)r * HD + 8 * p);
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int it = tid + NTH * (q0 + q), r = it / NP, p = it % NP;
      if (it < LT * NP) *reinterpret_cast<u16x8*>(&kt.hi[r * HD + 8 * (p ^ (r % NP))]) = v[q];
    }
  }
}

// an M^T hi / lo pair of planes into LDS (rows d, swizzled as the keys): from the bf16 forward's
// snapshot (already M^T hi / lo) or, split here, from an fp32 M[c][d] (the fp32 forward's)
template <int HD, int NTH>
__device__ __forceinline__ void stage_mt(uint16_t* mt, const uint16_t* src, int tid) {
  // the thread's items in batches of 8, every load of a batch before its stores
  constexpr int NP = Dims<HD>::NP, N = (2 * HD * NP + NTH - 1) / NTH, NB = N < 8 ? N : 8;
  static_assert(N % NB == 0, "batches of the thread's items");
#pragma unroll
  for (int q0 = 0; q0 < N; q0 += NB) {
    u16x8 v[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int it = tid + NTH * (q0 + q);
      const int pl = it / (HD * NP), rem = it % (HD * NP), d = rem / NP, p = rem % NP;
      if (it < 2 * HD * NP) v[q] = *reinterpret_cast<const u16x8*>(src + (long long)pl * HD * HD + d * HD + 8 * p);
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int it = tid + NTH * (q0 + q);
      const int pl = it / (HD * NP), rem = it % (HD * NP), d = rem / NP, p = rem % NP;
      if (it < 2 * HD * NP) *reinterpret_cast<u16x8*>(&mt[pl * HD * HD + d * HD + 8 * (p ^ (d % NP))]) = v[q];
    }
  }
}
template <int HD, int NTH>
__device__ __forceinline__ void stage_mt_f32(uint16_t* mt, const float* m, int tid) {
  constexpr int NP = Dims<HD>::NP;
  for (int it = tid; it < HD * NP; it += NTH) {
    const int d = it % HD, p = it / HD;   // consecutive threads: consecutive columns d of one row block
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = m[(long long)(8 * p + e) * HD + d];
    u16x8 h, lw;
    split8(v, h, lw);
    const int o = d * HD + 8 * (p ^ (d % NP));
    *reinterpret_cast<u16x8*>(&mt[o]) = h;
    *reinterpret_cast<u16x8*>(&mt[HD * HD + o]) = lw;
  }
}
template <int HD>
__device__ __forceinline__ u16x8 row_piece(const uint16_t* t, int r, int p) {
  return *reinterpret_cast<const u16x8*>(&t[r * HD + 8 * (p ^ (r % Dims<HD>::NP))]);
}
__device__ __forceinline__ u16x8 neg_bf(u16x8 v) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] ^= 0x8000u;
  return v;
}
// four consecutive features c0.. of key row r of the step (global memory, storage dtype)
template <int HD, bool F32>
__device__ __forceinline__ float4 key_quad(const void* kr_rows, int r, int c0) {
  if constexpr (F32) {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(kr_rows) + (long long)r * HD + c0);
  } else {
    const uint2 k2 = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(kr_rows) + (long long)r * HD + c0);
    return make_float4(bf_lo(k2.x), bf_hi(k2.x), bf_lo(k2.y), bf_hi(k2.y));
  }
}
template <bool F32>
__device__ __forceinline__ const void* rows_at(const void* base, long long row, int hd) {
  return F32 ? (const void*)(reinterpret_cast<const float*>(base) + row * hd)
             : (const void*)(reinterpret_cast<const uint16_t*>(base) + row * hd);
}

// ---------------------------------------------------------------- per-token statistics

template <int HD, bool F32>
__global__ void __launch_bounds__(NT) tok_stats_kernel(b3_chain_bwd_args a) {
  using Dm = Dims<HD>;
  __shared__ KeyTile<HD, F32> kt;
  __shared__ float s_inv[LT], s_w[LT];
  const int i = blockIdx.x, bh = blockIdx.y;
  if (filled_before(a, i) < S) return;   // fill step: no delta rule
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int l = step_len(a, i), t0 = step_off(a, i);
  const void* kr = rows_at<F32>(a.kr, (long long)bh * a.T + t0, HD);
  stage_keys<HD, F32, NT>(kt, kr, l, tid);
  float* st = stats_of(a, i, bh);
  if (tid < LT) {
    float iv = 0.f, wv = 0.f;
    if (tid < l) {
      float ss = 0.f;
      for (int d = 0; d < HD; d += 4) {
        const float4 x = key_quad<HD, F32>(kr, tid, d);
        ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
      }
      iv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      if (log_rec(a, i, bh)[B3_LOG_DELTA * B3_LOG_COLS + tid] > 0.5f) wv = a.beta[(long long)bh * a.T + t0 + tid];
    }
    s_inv[tid] = iv;
    s_w[tid] = wv;
    st[tid] = iv;
    st[3 * LT + tid] = wv;
  }
  __syncthreads();
  // column j = 32 w + n: sum over rows i of |khat_i . khat_j| w_i
  const int j = 32 * w + n;
  const float inj = s_inv[j];
  float colsum = 0.f;
  for (int ti = 0; ti < LT / 32; ++ti) {
    if (32 * ti >= l) break;
    f32x16 acc = zero16();
#pragma unroll
    for (int ks = 0; ks < Dm::KS; ++ks) {
      const u16x8 ai = row_piece<HD>(kt.hi, 32 * ti + n, 2 * ks + h), bj = row_piece<HD>(kt.hi, j, 2 * ks + h);
      mma_bf16(acc, ai, bj);
      if constexpr (F32) {
        mma_bf16(acc, ai, row_piece<HD>(kt.lo, j, 2 * ks + h));
        mma_bf16(acc, row_piece<HD>(kt.lo, 32 * ti + n, 2 * ks + h), bj);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ii = 32 * ti + d_row(lane, r);
      if (ii < l) colsum += fabsf(acc[r] * (s_inv[ii] * inj)) * s_w[ii];
    }
  }
  colsum = pair_sum32(colsum);
  if (h == 0 && j < LT) {
    st[LT + j] = j < l ? colsum : 0.f;
    st[2 * LT + j] = j < l ? s_w[j] / fmaxf(colsum, 1.0f) : 0.f;
  }
}

// ---------------------------------------------------------------- slot recursion

// Features of slice sl: 8 sl .. 8 sl + 7 and HD/2 + 8 sl .. (the RoPE pairs).
template <int HD>
__device__ __forceinline__ void add_row16(float* out, int sl, const float* v) {
  float4* p0 = reinterpret_cast<float4*>(out + 8 * sl);
  float4* p1 = reinterpret_cast<float4*>(out + HD / 2 + 8 * sl);
  float4 x;
  x = p0[0]; x.x += v[0]; x.y += v[1]; x.z += v[2]; x.w += v[3]; p0[0] = x;
  x = p0[1]; x.x += v[4]; x.y += v[5]; x.z += v[6]; x.w += v[7]; p0[1] = x;
  x = p1[0]; x.x += v[8]; x.y += v[9]; x.z += v[10]; x.w += v[11]; p1[0] = x;
  x = p1[1]; x.x += v[12]; x.y += v[13]; x.z += v[14]; x.w += v[15]; p1[1] = x;
}

// What a thread of slot_rec reads for step i that does not depend on the recursion: its slot's
// attention gradient slice, the slot's mean position and previous mass, and the decision-log
// entries its indices select.  Fetched one step ahead, so that a step waits for one round trip
// (its token rows) instead of three.
template <int HD>
struct SlotRecIn {
  float lo[8], hi[8];     // d_slot_{k|v} of (step, slot): features 8 sl .., HD/2 + 8 sl ..
  float p, mb;            // snap_pm of the step, snap_mass of the step before (arr 0)
  int fill;               // fill step: slot s takes a picked token (log TOPTOK at s - nfb)
  float fill_tok;
  float win, bs, tk;      // steady step, tid < min(l, S): log WIN / BOTSLOT / TOPTOK at tid
  float mg, ts;           // tid < l: log MERGE / SLOT at tid
  float mgj, tsj;         // j = tid / 2 < l: log MERGE / SLOT at j
};

template <int HD>
__device__ __forceinline__ SlotRecIn<HD> slot_rec_fetch(const b3_chain_bwd_args& a, int i, int bh, int sl, int s,
                                                        int arr, int tid) {
  SlotRecIn<HD> f;
  const long long BH = (long long)a.B * a.HKV;
  const int l = step_len(a, i), nfb = filled_before(a, i);
  const float* lg = log_rec(a, i, bh);
  const long long base = (((long long)i * BH + bh) * S + s) * HD;
  const float* src = (arr ? a.d_slot_v : a.d_slot_k) + base;
  *reinterpret_cast<float4*>(f.lo) = *reinterpret_cast<const float4*>(src + 8 * sl);
  *reinterpret_cast<float4*>(f.lo + 4) = *reinterpret_cast<const float4*>(src + 8 * sl + 4);
  *reinterpret_cast<float4*>(f.hi) = *reinterpret_cast<const float4*>(src + HD / 2 + 8 * sl);
  *reinterpret_cast<float4*>(f.hi + 4) = *reinterpret_cast<const float4*>(src + HD / 2 + 8 * sl + 4);
  f.p = arr == 0 ? a.snap_pm[((long long)i * BH + bh) * S + s] : 0.f;
  f.mb = 0.f;
  f.fill = 0;
  f.fill_tok = -1.f;
  f.win = f.bs = f.tk = f.mg = f.ts = f.mgj = f.tsj = -1.f;
  if (nfb < S) {
    const int m = min(S - nfb, l);
    if (s >= nfb && s < nfb + m) {
      f.fill = 1;
      f.fill_tok = lg[B3_LOG_TOPTOK * B3_LOG_COLS + (s - nfb)];
    }
  } else {
    if (arr == 0) f.mb = a.snap_mass[((long long)(i - 1) * BH + bh) * S + s];   // steady: i >= 1
    if (tid < min(l, S)) {
      f.win = lg[B3_LOG_WIN * B3_LOG_COLS + tid];
      f.bs = lg[B3_LOG_BOTSLOT * B3_LOG_COLS + tid];
      f.tk = lg[B3_LOG_TOPTOK * B3_LOG_COLS + tid];
    }
    if (tid < l) {
      f.mg = lg[B3_LOG_MERGE * B3_LOG_COLS + tid];
      f.ts = lg[B3_LOG_SLOT * B3_LOG_COLS + tid];
    }
    const int jj = tid >> 1;
    if (jj < l) {
      f.mgj = lg[B3_LOG_MERGE * B3_LOG_COLS + jj];
      f.tsj = lg[B3_LOG_SLOT * B3_LOG_COLS + jj];
    }
  }
  return f;
}

template <int HD>
__global__ void __launch_bounds__(NT) slot_rec_kernel(b3_chain_bwd_args a) {
  // gradients of the slots' un-roped keys (g[0]) and values (g[1]) on this slice
  __shared__ float g[2][S][17];
  __shared__ int map_tok[S], cnt[S];
  __shared__ float massb[S], newm[S];
  const int bh = blockIdx.x, sl = blockIdx.y;
  const int tid = threadIdx.x, s = tid >> 1, arr = tid & 1;
  if (a.started && tid == 0) __hip_atomic_fetch_add(a.started, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float* grow = g[arr][s];
#pragma unroll
  for (int e = 0; e < 16; ++e) grow[e] = 0.f;
  float invf[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) invf[e] = a.inv_freq[8 * sl + e];
  float* const out_all = arr ? a.d_v : a.d_kr;
  if (a.n_steps <= 0) return;
  SlotRecIn<HD> cur = slot_rec_fetch<HD>(a, a.n_steps - 1, bh, sl, s, arr, tid);
  for (int i = a.n_steps - 1; i >= 0; --i) {
    const int l = step_len(a, i), t0 = step_off(a, i), nfb = filled_before(a, i);
    SlotRecIn<HD> nxt;
    if (i > 0) nxt = slot_rec_fetch<HD>(a, i - 1, bh, sl, s, arr, tid);
    float* out = out_all + ((long long)bh * a.T + t0) * HD;
    // the attention's gradients of the slots after step i: keys through the transpose of
    // their RoPE at the slot's mean position
    if (arr == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float sn, cs;
        sincos_rope(cur.p * invf[e], &sn, &cs);   // the forward RoPE's own values
        grow[e] += cur.lo[e] * cs + cur.hi[e] * sn;
        grow[8 + e] += cur.hi[e] * cs - cur.lo[e] * sn;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        grow[e] += cur.lo[e];
        grow[8 + e] += cur.hi[e];
      }
    }
    if (nfb < S) {
      // fill: slots nfb .. nfb + m - 1 are copies of the picked tokens
      if (cur.fill) {
        const int tok = (int)cur.fill_tok;
        if ((unsigned)tok < (unsigned)l) add_row16<HD>(out + (long long)tok * HD, sl, grow);
#pragma unroll
        for (int e = 0; e < 16; ++e) grow[e] = 0.f;
      }
      cur = nxt;
      continue;   // every thread touches only its own row in this step
    }
    // steady step: winners (token -> slot) and merge counts
    if (tid < S) {
      map_tok[tid] = -1;
      cnt[tid] = 0;
    }
    __syncthreads();
    // (indices outside the step's tokens or the slots are ignored)
    if (cur.win > 0.5f) {
      const int bs = (int)cur.bs, tk = (int)cur.tk;
      if ((unsigned)bs < (unsigned)S && (unsigned)tk < (unsigned)l) map_tok[bs] = tk;
    }
    if (cur.mg > 0.5f) {
      const int ts = (int)cur.ts;
      if ((unsigned)ts < (unsigned)S) atomicAdd(&cnt[ts], 1);
    }
    __syncthreads();
    // eviction: the winning token took the slot, so the slot's gradient is the token's
    {
      const int tok = map_tok[s];
      if (tok >= 0) {
        add_row16<HD>(out + (long long)tok * HD, sl, grow);
#pragma unroll
        for (int e = 0; e < 16; ++e) grow[e] = 0.f;
      }
      if (arr == 0) {
        massb[s] = cur.mb;
        newm[s] = cur.mb + (float)cnt[s];
      }
    }
    __syncthreads();
    // merge: slot <- (mass * slot + sum of merged tokens) / new_mass
    {
      const int j = tid >> 1;
      const int ts = (int)cur.tsj;
      if (cur.mgj > 0.5f && (unsigned)ts < (unsigned)S) {
        const float coef = 1.0f / newm[ts];
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = g[arr][ts][e] * coef;
        add_row16<HD>(out + (long long)j * HD, sl, v);
      }
    }
    __syncthreads();
    if (cnt[s] > 0) {
      const float kp = massb[s] / newm[s];
#pragma unroll
      for (int e = 0; e < 16; ++e) grow[e] *= kp;
    }
    __syncthreads();
    cur = nxt;
  }
}

// ---------------------------------------------------------------- M_res recursion

template <int HD, bool F32>
struct MrecSmem {
  KeyTile<HD, F32> kt;                   // the step's keys
  alignas(16) uint16_t ct[2][32 * HD];   // G^T of the column block, hi / lo: row n, columns c
  alignas(16) uint16_t tt[2][32 * LT];   // T^T hi / lo: row n, columns j (tokens)
  float coef[LT];
  float gp[Dims<HD>::NCB];
};

// one wavefront per 32 rows of M: HD / 32 wavefronts
template <int HD, bool F32>
__global__ void __launch_bounds__(HD * 2) m_rec_kernel(b3_chain_bwd_args a) {
  using Dm = Dims<HD>;
  constexpr int NCB = Dm::NCB, NP = Dm::NP, NTH = 64 * NCB;
  __shared__ MrecSmem<HD, F32> sm;
  // XCD-aware order: the NCB column blocks of one bh read the same per-step rows
  const int wg = xcd_grid_pos().x;
  const int bh = wg / NCB, db = wg % NCB;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
  if (a.started && tid == 0) __hip_atomic_fetch_add(a.started, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const long long BH = (long long)a.B * a.HKV;
  const float gam = a.gamma[bh % a.HKV];
  const TrLanes<HD> TL(lane);
  // G of the block: rows c = 32 w + d_row(lane, r), column d = 32 db + n
  f32x16 cur = zero16();
  for (int i = a.n_steps - 1; i >= 0; --i) {
    const float* dm = a.d_m + ((long long)i * BH + bh) * HD * HD;
#pragma unroll
    for (int r = 0; r < 16; ++r) cur[r] += dm[(32 * w + d_row(lane, r)) * HD + 32 * db + n];
    if (filled_before(a, i) < S) {   // fill steps leave M_res as it is
      if (tid == 0) a.d_gamma[((long long)i * BH + bh) * NCB + db] = 0.f;
      continue;
    }
    const int l = step_len(a, i), t0 = step_off(a, i);
    // G_i out (as G^T hi / lo) and this step's share of dL/dgamma: sum(G_i * M_{i-1})
    {
      uint16_t* gt = gt_of<HD>(a, i, bh);
      const float* m0 = a.snap_m + ((long long)(i - 1) * BH + bh) * HD * HD;
      const int d = 32 * db + n;
      float gs = 0.f;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int c0 = 32 * w + 8 * r4 + 4 * h;
        uint16_t hb[4], lb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = cur[4 * r4 + q];
          hb[q] = f2bf(x);
          lb[q] = f2bf(x - bf2f(hb[q]));
        }
        const uint2 ph = make_uint2(hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16));
        const uint2 pl = make_uint2(lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16));
        *reinterpret_cast<uint2*>(gt + d * HD + c0) = ph;
        *reinterpret_cast<uint2*>(gt + HD * HD + d * HD + c0) = pl;
        *reinterpret_cast<uint2*>(&sm.ct[0][n * HD + 8 * ((4 * w + r4) ^ (n % NP)) + 4 * h]) = ph;
        *reinterpret_cast<uint2*>(&sm.ct[1][n * HD + 8 * ((4 * w + r4) ^ (n % NP)) + 4 * h]) = pl;
        if constexpr (F32) {
          // the fp32 forward's snapshot: M[c][d]
#pragma unroll
          for (int q = 0; q < 4; ++q) gs += cur[4 * r4 + q] * m0[(long long)(c0 + q) * HD + d];
        } else {
          // the bf16 forward's snapshot: M^T as bf16 hi, then lo
          const uint16_t* mt = reinterpret_cast<const uint16_t*>(m0);
          const uint2 mh = *reinterpret_cast<const uint2*>(mt + d * HD + c0);
          const uint2 ml = *reinterpret_cast<const uint2*>(mt + HD * HD + d * HD + c0);
          gs += cur[4 * r4] * (bf_lo(mh.x) + bf_lo(ml.x)) + cur[4 * r4 + 1] * (bf_hi(mh.x) + bf_hi(ml.x)) +
                cur[4 * r4 + 2] * (bf_lo(mh.y) + bf_lo(ml.y)) + cur[4 * r4 + 3] * (bf_hi(mh.y) + bf_hi(ml.y));
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) gs += __shfl_xor(gs, o, 64);
      if (lane == 0) sm.gp[w] = gs;
    }
    stage_keys<HD, F32, NTH>(sm.kt, rows_at<F32>(a.kr, (long long)bh * a.T + t0, HD), l, tid);
    for (int j = tid; j < LT; j += NTH) {
      const float* st = stats_of(a, i, bh);
      sm.coef[j] = j < l ? st[j] * st[j] * st[2 * LT + j] : 0.f;   // bsafe / |k|^2
    }
    __syncthreads();
    if (tid == 0) {
      float gsum = 0.f;
#pragma unroll
      for (int q = 0; q < NCB; ++q) gsum += sm.gp[q];
      a.d_gamma[((long long)i * BH + bh) * NCB + db] = gsum;
    }
    // T = K G (token blocks tb = w, w + NCB, ..), then scaled by bsafe / |k|^2 into T^T
    for (int tb = w; tb < LT / 32; tb += NCB) {
      f32x16 t1 = zero16();
      const int jr = 32 * tb + n;
#pragma unroll
      for (int ks = 0; ks < Dm::KS; ++ks) {
        const u16x8 ka = row_piece<HD>(sm.kt.hi, jr, 2 * ks + h);
        const u16x8 bhv = *reinterpret_cast<const u16x8*>(&sm.ct[0][n * HD + 8 * ((2 * ks + h) ^ (n % NP))]);
        const u16x8 blv = *reinterpret_cast<const u16x8*>(&sm.ct[1][n * HD + 8 * ((2 * ks + h) ^ (n % NP))]);
        mma_bf16(t1, ka, bhv);
        mma_bf16(t1, ka, blv);
        if constexpr (F32) mma_bf16(t1, row_piece<HD>(sm.kt.lo, jr, 2 * ks + h), bhv);
      }
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int j0 = 32 * tb + 8 * r4 + 4 * h;
        uint16_t hb[4], lb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = t1[4 * r4 + q] * sm.coef[j0 + q];
          hb[q] = f2bf(x);
          lb[q] = f2bf(x - bf2f(hb[q]));
        }
        const int off = n * LT + 8 * ((4 * tb + r4) ^ (n % NPT)) + 4 * h;
        *reinterpret_cast<uint2*>(&sm.tt[0][off]) = make_uint2(hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16));
        *reinterpret_cast<uint2*>(&sm.tt[1][off]) = make_uint2(lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16));
      }
    }
    __syncthreads();
    // G <- gamma G - K^T T (wavefront w: rows c = 32 w ..); K^T read transposed, T^T in the
    // accumulator's row order
    {
      f32x16 u = zero16();
#pragma unroll
      for (int t4 = 0; t4 < LT / 32; ++t4)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const u16x8 ka = tr_operand<HD>(sm.kt.hi + 32 * t4 * HD, TL, w, kc);
          const int p0 = 4 * t4 + 2 * kc;
          const uint2 h0 = *reinterpret_cast<const uint2*>(&sm.tt[0][n * LT + 8 * (p0 ^ (n % NPT)) + 4 * h]);
          const uint2 h1 = *reinterpret_cast<const uint2*>(&sm.tt[0][n * LT + 8 * ((p0 + 1) ^ (n % NPT)) + 4 * h]);
          const uint2 l0 = *reinterpret_cast<const uint2*>(&sm.tt[1][n * LT + 8 * (p0 ^ (n % NPT)) + 4 * h]);
          const uint2 l1 = *reinterpret_cast<const uint2*>(&sm.tt[1][n * LT + 8 * ((p0 + 1) ^ (n % NPT)) + 4 * h]);
          u16x8 bhv, blv;
          bhv[0] = h0.x & 0xffff; bhv[1] = h0.x >> 16; bhv[2] = h0.y & 0xffff; bhv[3] = h0.y >> 16;
          bhv[4] = h1.x & 0xffff; bhv[5] = h1.x >> 16; bhv[6] = h1.y & 0xffff; bhv[7] = h1.y >> 16;
          blv[0] = l0.x & 0xffff; blv[1] = l0.x >> 16; blv[2] = l0.y & 0xffff; blv[3] = l0.y >> 16;
          blv[4] = l1.x & 0xffff; blv[5] = l1.x >> 16; blv[6] = l1.y & 0xffff; blv[7] = l1.y >> 16;
          mma_bf16(u, ka, bhv);
          mma_bf16(u, ka, blv);
          if constexpr (F32) mma_bf16(u, tr_operand<HD>(sm.kt.lo + 32 * t4 * HD, TL, w, kc), bhv);
        }
#pragma unroll
      for (int r = 0; r < 16; ++r) cur[r] = gam * cur[r] - u[r];
    }
    __syncthreads();   // the tiles are rewritten by the next step
  }
}

// ---------------------------------------------------------------- token gradients

template <int HD, bool F32>
struct TgSmem {
  alignas(16) uint16_t mt[2 * HD * HD];   // M_{i-1}^T or G_i^T, hi then lo (rows d)
  KeyTile<HD, F32> kt;                    // the step's keys
  float inv[LT], raw[LT], bs[LT], wv[LT], drs[LT];
};

template <int HD, bool F32>
__device__ __forceinline__ void stage_m_prev(uint16_t* mt, const b3_chain_bwd_args& a, const float* m0, int tid) {
  if constexpr (F32) stage_mt_f32<HD, NT>(mt, m0, tid);
  else stage_mt<HD, NT>(mt, reinterpret_cast<const uint16_t*>(m0), tid);
}

template <int HD, bool F32>
__global__ void __launch_bounds__(NT) tok_grad_kernel(b3_chain_bwd_args a) {
  using Dm = Dims<HD>;
  constexpr int NCB = Dm::NCB, KS = Dm::KS;
  __shared__ TgSmem<HD, F32> sm;
  const int i = blockIdx.x, bh = blockIdx.y;
  if (filled_before(a, i) < S) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const long long BH = (long long)a.B * a.HKV;
  const int l = step_len(a, i), t0 = step_off(a, i);
  const TrLanes<HD> TL(lane);
  const float* m0 = a.snap_m + ((long long)(i - 1) * BH + bh) * HD * HD;
  const void* krows = rows_at<F32>(a.kr, (long long)bh * a.T + t0, HD);
  stage_m_prev<HD, F32>(sm.mt, a, m0, tid);
  stage_keys<HD, F32, NT>(sm.kt, krows, l, tid);
  if (tid < LT) {
    const float* st = stats_of(a, i, bh);
    const bool ok = tid < l;
    sm.inv[tid] = ok ? st[tid] : 0.f;
    sm.raw[tid] = ok ? st[LT + tid] : 0.f;
    sm.bs[tid] = ok ? st[2 * LT + tid] : 0.f;
    sm.wv[tid] = ok ? st[3 * LT + tid] : 0.f;
    sm.drs[tid] = 0.f;
  }
  __syncthreads();
  const int j = 32 * w + n;   // this lane's token
  const bool live = j < l;
  const float inj = sm.inv[j], bsj = sm.bs[j], wj = sm.wv[j], rawj = sm.raw[j];
  const long long trow = (long long)bh * a.T + t0 + j;
  // R^T[d][j] = v[j][d] - (M^T k_j)[d] / |k_j|
  f32x16 R[NCB];
#pragma unroll
  for (int db = 0; db < NCB; ++db) R[db] = zero16();
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u16x8 kb = row_piece<HD>(sm.kt.hi, j, 2 * ks + h);
#pragma unroll
    for (int db = 0; db < NCB; ++db) {
      const int dr = 32 * db + n;
      const u16x8 mh = row_piece<HD>(sm.mt, dr, 2 * ks + h);
      mma_bf16(R[db], mh, kb);
      mma_bf16(R[db], row_piece<HD>(sm.mt + HD * HD, dr, 2 * ks + h), kb);
      if constexpr (F32) mma_bf16(R[db], mh, row_piece<HD>(sm.kt.lo, j, 2 * ks + h));
    }
  }
  {
#pragma unroll
    for (int db = 0; db < NCB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) v4 = key_quad<HD, F32>(rows_at<F32>(a.v, trow, HD), 0, 32 * db + 8 * r4 + 4 * h);
        R[db][4 * r4] = v4.x - R[db][4 * r4] * inj;
        R[db][4 * r4 + 1] = v4.y - R[db][4 * r4 + 1] * inj;
        R[db][4 * r4 + 2] = v4.z - R[db][4 * r4 + 2] * inj;
        R[db][4 * r4 + 3] = v4.w - R[db][4 * r4 + 3] * inj;
      }
  }
  __syncthreads();   // M_{i-1}^T read
  stage_mt<HD, NT>(sm.mt, gt_of<HD>(a, i, bh), tid);
  __syncthreads();
  // dE^T = (G^T k_j) / |k_j|  (gradient of E's row j through V - Khat M is dE; of R: bsafe dE)
  f32x16 dE[NCB];
#pragma unroll
  for (int db = 0; db < NCB; ++db) dE[db] = zero16();
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u16x8 kb = row_piece<HD>(sm.kt.hi, j, 2 * ks + h);
#pragma unroll
    for (int db = 0; db < NCB; ++db) {
      const int dr = 32 * db + n;
      const u16x8 gh = row_piece<HD>(sm.mt, dr, 2 * ks + h);
      mma_bf16(dE[db], gh, kb);
      mma_bf16(dE[db], row_piece<HD>(sm.mt + HD * HD, dr, 2 * ks + h), kb);
      if constexpr (F32) mma_bf16(dE[db], gh, row_piece<HD>(sm.kt.lo, j, 2 * ks + h));
    }
  }
  float dbs = 0.f;
#pragma unroll
  for (int db = 0; db < NCB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dE[db][r] *= inj;
      dbs += dE[db][r] * R[db][r];
    }
  dbs = pair_sum32(dbs);
  // dKhat^T[c][j] = sum_d G[c][d] E[j][d]: G read transposed out of G^T, E = bsafe R
  f32x16 dkn[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) dkn[cb] = zero16();
#pragma unroll
  for (int db = 0; db < NCB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) R[db][r] *= bsj;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      u16x8 eh, el;
      acc_operand_split(R[db], kc, eh, el);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const u16x8 ah = tr_operand<HD>(sm.mt + 32 * db * HD, TL, cb, kc);
        const u16x8 al = tr_operand<HD>(sm.mt + HD * HD + 32 * db * HD, TL, cb, kc);
        mma_bf16(dkn[cb], ah, eh);
        mma_bf16(dkn[cb], al, eh);
        mma_bf16(dkn[cb], ah, el);
      }
    }
  }
  // dV = bsafe dE (the gradient of R), added to the values' gradient
#pragma unroll
  for (int db = 0; db < NCB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dE[db][r] *= bsj;
  if (live) {
    float* dv = a.d_v + trow * HD;
#pragma unroll
    for (int db = 0; db < NCB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        float4* p = reinterpret_cast<float4*>(dv + 32 * db + 8 * r4 + 4 * h);
        float4 x = *p;
        x.x += dE[db][4 * r4];
        x.y += dE[db][4 * r4 + 1];
        x.z += dE[db][4 * r4 + 2];
        x.w += dE[db][4 * r4 + 3];
        *p = x;
      }
  }
  // the clamp of the row sum at 1 passes its gradient where r_j >= 1
  const float rsj = fmaxf(rawj, 1.0f);
  const float drsj = (live && rawj >= 1.0f) ? -dbs * wj / (rsj * rsj) : 0.f;
  if (h == 0 && live) sm.drs[j] = drsj;
  __syncthreads();   // G^T read; drs complete
  stage_m_prev<HD, F32>(sm.mt, a, m0, tid);
  __syncthreads();
  // dKhat^T -= sum_d M[c][d] dV[j][d]
#pragma unroll
  for (int db = 0; db < NCB; ++db)
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      u16x8 vh, vl;
      acc_operand_split(dE[db], kc, vh, vl);
      vh = neg_bf(vh);
      vl = neg_bf(vl);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const u16x8 ah = tr_operand<HD>(sm.mt + 32 * db * HD, TL, cb, kc);
        const u16x8 al = tr_operand<HD>(sm.mt + HD * HD + 32 * db * HD, TL, cb, kc);
        mma_bf16(dkn[cb], ah, vh);
        mma_bf16(dkn[cb], al, vh);
        mma_bf16(dkn[cb], ah, vl);
      }
    }
  // through the row sums: P = Khat Khat^T, dw_j += sum_i |P_ij| drs_i, and
  // dKhat_j += sum_i sign(P_ij) (drs_j w_i + drs_i w_j) khat_i
  float dwg = 0.f;
#pragma unroll
  for (int ti = 0; ti < LT / 32; ++ti) {
    f32x16 p = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u16x8 ai = row_piece<HD>(sm.kt.hi, 32 * ti + n, 2 * ks + h), bj = row_piece<HD>(sm.kt.hi, j, 2 * ks + h);
      mma_bf16(p, ai, bj);
      if constexpr (F32) {
        mma_bf16(p, ai, row_piece<HD>(sm.kt.lo, j, 2 * ks + h));
        mma_bf16(p, row_piece<HD>(sm.kt.lo, 32 * ti + n, 2 * ks + h), bj);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ii = 32 * ti + d_row(lane, r);
      const float pv = p[r] * (sm.inv[ii] * inj);
      const float sgn = pv > 0.f ? 1.f : (pv < 0.f ? -1.f : 0.f);
      dwg += fabsf(pv) * sm.drs[ii];
      p[r] = sm.inv[ii] * sgn * (drsj * sm.wv[ii] + sm.drs[ii] * wj);
    }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      u16x8 qh, ql;
      acc_operand_split(p, kc, qh, ql);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const u16x8 ka = tr_operand<HD>(sm.kt.hi + 32 * ti * HD, TL, cb, kc);
        mma_bf16(dkn[cb], ka, qh);
        mma_bf16(dkn[cb], ka, ql);
        if constexpr (F32) mma_bf16(dkn[cb], tr_operand<HD>(sm.kt.lo + 32 * ti * HD, TL, cb, kc), qh);
      }
    }
  }
  dwg = pair_sum32(dwg);
  // the normalisation: dk = (dKhat - khat (khat . dKhat)) / |k|
  float kq[NCB][4][4];
  float sdot = 0.f;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      float4 k4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (live) k4 = key_quad<HD, F32>(krows, j, 32 * cb + 8 * r4 + 4 * h);
      kq[cb][r4][0] = k4.x; kq[cb][r4][1] = k4.y; kq[cb][r4][2] = k4.z; kq[cb][r4][3] = k4.w;
      sdot += k4.x * dkn[cb][4 * r4] + k4.y * dkn[cb][4 * r4 + 1] + k4.z * dkn[cb][4 * r4 + 2] +
              k4.w * dkn[cb][4 * r4 + 3];
    }
  sdot = pair_sum32(sdot);
  if (!live) return;
  const float f2 = inj * inj * sdot;
  float* dk = a.d_kr + trow * HD;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      float4* p = reinterpret_cast<float4*>(dk + 32 * cb + 8 * r4 + 4 * h);
      float4 x = *p;
      x.x += (dkn[cb][4 * r4] - kq[cb][r4][0] * f2) * inj;
      x.y += (dkn[cb][4 * r4 + 1] - kq[cb][r4][1] * f2) * inj;
      x.z += (dkn[cb][4 * r4 + 2] - kq[cb][r4][2] * f2) * inj;
      x.w += (dkn[cb][4 * r4 + 3] - kq[cb][r4][3] * f2) * inj;
      *p = x;
    }
  if (h == 0 && log_rec(a, i, bh)[B3_LOG_DELTA * B3_LOG_COLS + j] > 0.5f)
    a.d_beta[trow] += (rsj > 0.f ? dbs / rsj : 0.f) + dwg;
}

template <int HD, bool F32>
static int launch(const b3_chain_bwd_args& a, hipStream_t st) {
  const long long BH = (long long)a.B * a.HKV;
  const int k = a.kernels == 0 ? B3_CBWD_ALL : a.kernels;
  hipError_t e = hipSuccess;
  if (k & B3_CBWD_STATS) {
    hipLaunchKernelGGL((tok_stats_kernel<HD, F32>), dim3(a.n_steps, (unsigned)BH), dim3(NT), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if (k & B3_CBWD_M_REC) {
    hipLaunchKernelGGL((m_rec_kernel<HD, F32>), dim3((unsigned)(BH * Dims<HD>::NCB)), dim3(64 * Dims<HD>::NCB), 0,
                       st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if (k & B3_CBWD_SLOT_REC) {
    hipLaunchKernelGGL((slot_rec_kernel<HD>), dim3((unsigned)BH, Dims<HD>::NSL), dim3(NT), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if (k & B3_CBWD_TOK_GRAD)
    hipLaunchKernelGGL((tok_grad_kernel<HD, F32>), dim3(a.n_steps, (unsigned)BH), dim3(NT), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace cbwd
}  // namespace b3

extern "C" int64_t bolt3_chain_bwd_workspace_bytes(int32_t B, int32_t HKV, int32_t HD, int32_t n_steps) {
  if (B <= 0 || HKV <= 0 || (HD != 64 && HD != 128) || n_steps <= 0) return 0;
  return b3::cbwd::ws_bytes(n_steps, (long long)B * HKV, HD);
}

extern "C" int bolt3_chain_bwd(const b3_chain_bwd_args* a, void* stream) {
  using namespace b3::cbwd;
  if (!a) return B3_ERR_ARG;
  if ((a->dtype != B3_BF16 && a->dtype != B3_F32) || (a->HD != 64 && a->HD != 128) || a->S != S)
    return B3_ERR_UNSUPPORTED;
  if (a->B <= 0 || a->HKV <= 0 || a->T <= 0 || a->n_steps <= 0) return B3_ERR_ARG;
  if (a->len0 <= 0 || a->len0 > LT || a->step_len <= 0 || a->step_len > LT || a->off0 < 0 || a->step_stride <= 0)
    return B3_ERR_UNSUPPORTED;
  if (a->kernels < 0 || a->kernels > B3_CBWD_ALL) return B3_ERR_ARG;
  if ((long long)a->off0 + a->len0 > a->T ||
      (a->n_steps > 1 && (long long)(a->n_steps - 1) * a->step_stride + a->step_len > a->T))
    return B3_ERR_ARG;
  if (!a->kr || !a->v || !a->beta || !a->log || !a->snap_mass || !a->snap_pm || !a->snap_m || !a->gamma ||
      !a->inv_freq || !a->d_slot_k || !a->d_slot_v || !a->d_m || !a->d_kr || !a->d_v || !a->d_beta || !a->d_gamma ||
      !a->work)
    return B3_ERR_ARG;
  const long long BH = (long long)a->B * a->HKV;
  if (a->work_bytes < ws_bytes(a->n_steps, BH, a->HD)) return B3_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_BF16)
    return a->HD == 128 ? launch<128, false>(*a, st) : launch<64, false>(*a, st);
  return a->HD == 128 ? launch<128, true>(*a, st) : launch<64, true>(*a, st);
}

// Consolidation chain: successive attractor consolidations of one (batch,
// kv-head) row per workgroup.
//
// Replaces Bolt3Attn._consolidate_functional (vsa_lm/config/bolt3.py:68-192)
// as driven by the chunk loop (:262-273) and Bolt3Decoder.step (:406-425).
// Per step (l <= 256 tokens of a chunk that left the window):
//   fill   (:165-192) while slots are free: rank tokens by var(normalize(v))
//          (first fill) or rel_err*(1-max cos) (later fills), copy the best
//          min(S - n_filled, l) into the next free slots.
//   steady (:96-163): softmax read of the slots by the roped keys -> rel_err;
//          cosine match to the slots -> merge (cos_k >= .88, cos_v >= .80);
//          redundancy-weighted keep score per slot; the best non-merged tokens
//          replace the least useful slots; the rest go into M_res by the
//          Gershgorin-safe delta rule M <- g*M + K^T diag(b) (V - K M).
//
// Layout: one 256-thread workgroup (4 wavefronts) per bh.  Slot keys/values,
// masses, utilities, positions and activity stay in LDS for all steps; M_res
// stays in the caller's fp32 [bh][HD][HD] array (L2 resident).  Every product
// is a 32x32 MFMA tile: bf16 storage multiplies exact bf16 operands (products
// are exact in fp32) and splits fp32 operands (M_res, delta-rule errors) into
// bf16 hi+lo; fp32 storage uses the fp32 MFMA.  Decisions (argmax, thresholds,
// the two orderings) are made on fp32 values with the reference's tie and NaN
// rules: first index on ties, NaN ranks as the largest value.
#include "bolt3_common.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int S = 128;     // attractor slots
constexpr int LMAX = 256;  // tokens per consolidation step
constexpr int NT = 256;    // threads per workgroup
constexpr int NWAVE = NT / WAVE;
constexpr float SIM_K = 0.88f, SIM_V = 0.80f, UTIL_DECAY = 0.995f;

enum : int { F_MERGE = 1, F_DELTA = 2, F_INS = 4 };

template <typename T, int HD>
struct ChainSmem {
  // bf16 rows padded by 16 bytes (16-byte aligned fragments); fp32 rows by one word.
  static constexpr int KS = sizeof(T) == 2 ? HD + 8 : HD + 1;
  static constexpr bool ERR_LDS = !(sizeof(T) == 4 && HD == 128);
  static constexpr int ES = HD + 4;
  alignas(16) T ak[S * KS];
  alignas(16) T av[S * KS];
  float mass[S], util[S], pm[S], inv_nak[S], keep[S], bias[S], psum[S];
  int act[S], cnt[S], off[S], hits[S];
  float rel[LMAX], score[LMAX], best[LMAX], simv[LMAX], inv_nkr[LMAX], w[LMAX], bsafe[LMAX];
  int slot[LMAX], flags[LMAX], mlist[LMAX];
  float sk_a[LMAX];
  int si_a[LMAX];
  float sk_b[S];
  int si_b[S];
  float err[ERR_LDS ? 32 * ES : 1];
  int nhit;
};

// ----------------------------------------------------------------- fragments

// Token tile fragment: lane (n = lane%32, h = lane/32) holds row tok = t0 + n,
// K sub-index (per K-step ks) 16*ks + 8*h + i (bf16) or 2*ks + h (fp32).
template <typename T, int HD> struct Frag;
template <int HD> struct Frag<uint16_t, HD> {
  static constexpr int NK = HD / 16;
  u16x8 v[NK];
  __device__ __forceinline__ void load(const uint16_t* base, int tok, int l, int lane) {
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      if (tok < l) v[ks] = *reinterpret_cast<const u16x8*>(base + (long long)tok * HD + 16 * ks + 8 * h);
      else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[ks][i] = 0;
      }
    }
  }
  __device__ __forceinline__ float sumsq() const {
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) { const float x = bf2f(v[ks][i]); s += x * x; }
    return s;
  }
};
template <int HD> struct Frag<float, HD> {
  static constexpr int NK = HD / 2;
  float v[NK];
  __device__ __forceinline__ void load(const float* base, int tok, int l, int lane) {
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) v[ks] = tok < l ? base[(long long)tok * HD + 2 * ks + h] : 0.f;
  }
  __device__ __forceinline__ float sumsq() const {
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) s += v[ks] * v[ks];
    return s;
  }
};

// acc (rows = 32 rows of `rows` starting at row0, stride rs) += rows . frag^T over HD.
template <int HD>
__device__ __forceinline__ void mm_rows_frag(f32x16& acc, const uint16_t* rows, int rs, int row0,
                                             const Frag<uint16_t, HD>& f, int lane) {
  const int m = row0 + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int ks = 0; ks < HD / 16; ++ks) {
    const u16x8 a = *reinterpret_cast<const u16x8*>(rows + m * rs + 16 * ks + 8 * h);
    mma_bf16(acc, a, f.v[ks]);
  }
}
template <int HD>
__device__ __forceinline__ void mm_rows_frag(f32x16& acc, const float* rows, int rs, int row0,
                                             const Frag<float, HD>& f, int lane) {
  const int m = row0 + (lane & 31), h = lane >> 5;
#pragma unroll 8
  for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, rows[m * rs + 2 * ks + h], f.v[ks]);
}

// ----------------------------------------------------------------- helpers

template <typename T, int HD>
__device__ void rope_slots_to(T* dst, const ChainSmem<T, HD>& sm, const float* inv_freq, int tid) {
  constexpr int HALF = HD / 2;
  for (int it = tid; it < S * HALF; it += NT) {
    const int s = it / HALF, i = it % HALF;
    const float ang = mul_rn(sm.pm[s], inv_freq[i]);
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
    const float x0 = St<T>::to_f(sm.ak[s * sm.KS + i]), x1 = St<T>::to_f(sm.ak[s * sm.KS + i + HALF]);
    dst[s * HD + i] = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x0, c)), St<T>::rnd(mul_rn(-x1, si))));
    dst[s * HD + i + HALF] = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x1, c)), St<T>::rnd(mul_rn(x0, si))));
  }
}

// 1 / max(||ak_s||, 1e-12) for every slot.
template <typename T, int HD>
__device__ void slot_norms(ChainSmem<T, HD>& sm, int tid) {
  const int s = tid >> 1, half = tid & 1;
  float ss = 0.f;
  for (int d = half * (HD / 2); d < (half + 1) * (HD / 2); ++d) {
    const float x = St<T>::to_f(sm.ak[s * sm.KS + d]);
    ss += x * x;
  }
  ss += __shfl_xor(ss, 1, 64);
  if (half == 0) sm.inv_nak[s] = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
}

// Bitonic sort of NT keys (with indices) in LDS; desc: largest first.
__device__ void bitonic_256(float* key, int* idx, bool desc, int tid) {
  for (int k = 2; k <= NT; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int p = tid ^ j;
      if (p > tid) {
        const bool up = (tid & k) == 0;  // this pair sorted in the requested direction
        const float a = key[tid], b = key[p];
        const int ia = idx[tid], ib = idx[p];
        const bool b_first = desc ? ranks_before_desc(b, ib, a, ia) : ranks_before_asc(b, ib, a, ia);
        const bool swap = up ? b_first : !b_first;
        if (swap) { key[tid] = b; key[p] = a; idx[tid] = ib; idx[p] = ia; }
      }
      __syncthreads();
    }
  }
}

// Same for the first S entries, executed by threads < S (all threads reach the barriers).
__device__ void bitonic_128_asc(float* key, int* idx, int tid) {
  for (int k = 2; k <= S; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int p = tid ^ j;
      if (tid < S && p > tid) {
        const bool up = (tid & k) == 0;
        const float a = key[tid], b = key[p];
        const int ia = idx[tid], ib = idx[p];
        const bool b_first = ranks_before_asc(b, ib, a, ia);
        const bool swap = up ? b_first : !b_first;
        if (swap) { key[tid] = b; key[p] = a; idx[tid] = ib; idx[p] = ia; }
      }
      __syncthreads();
    }
  }
}

// ----------------------------------------------------------------- retrieval (phase A)

// For one 32-token tile: rel_err from the softmax read of the slots, cosine
// match, and (steady) the merge test.  `kread` holds the roped slot keys.
template <typename T, int HD>
__device__ void score_tile(ChainSmem<T, HD>& sm, const T* kread, const T* kr, const T* kp, const T* v,
                           int t0, int l, bool steady, float scale, int lane) {
  const int n = lane & 31, h = lane >> 5;
  const int tok = t0 + n;
  f32x16 acc[4];

  // scores^T[slot][tok] = kread . kp^T
  {
    Frag<T, HD> f;
    f.load(kp, tok, l, lane);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      acc[mb] = zero16();
      mm_rows_frag<HD>(acc[mb], kread, HD, 32 * mb, f, lane);
    }
  }
  // softmax over the slots (column of this lane pair)
  float mx = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int s = 32 * mb + d_row(lane, r);
      float x = add_rn(mul_rn(St<T>::rnd(acc[mb][r]), scale), sm.bias[s]);
      if (!steady && !sm.act[s]) x = -1e9f;
      acc[mb][r] = x;
      mx = fmaxf(mx, x);
    }
  mx = fmaxf(mx, xor32(mx));
  float sum = 0.f;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = expf(acc[mb][r] - mx);
      acc[mb][r] = e;
      sum += e;
    }
  sum += xor32(sum);
  const float rs = 1.0f / sum;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[mb][r] = St<T>::rnd(mul_rn(acc[mb][r], rs));

  // v_hat^T[d][tok] = av^T . P^T
  constexpr int NDB = HD / 32;
  f32x16 vh[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    vh[db] = zero16();
    const int d = 32 * db + n;
    if constexpr (St<T>::is_bf16) {
#pragma unroll
      for (int kc = 0; kc < 8; ++kc) {
        u16x8 a, b;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int s = 16 * kc + 8 * (i >> 2) + 4 * h + (i & 3);
          a[i] = sm.av[s * sm.KS + d];
          b[i] = f2bf(acc[kc >> 1][8 * (kc & 1) + i]);
        }
        mma_bf16(vh[db], a, b);
      }
    } else {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int s = 32 * mb + d_row(lane, r);
          mma_f32(vh[db], sm.av[s * sm.KS + d], acc[mb][r]);
        }
    }
  }
  // rel_err = ||v - v_hat|| / (||v|| + 1e-6)
  float e2 = 0.f, v2 = 0.f;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + d_row(lane, r);
      const float x = tok < l ? St<T>::ld(v + (long long)tok * HD + d) : 0.f;
      const float dv = x - St<T>::rnd(vh[db][r]);
      e2 += dv * dv;
      v2 += x * x;
    }
  e2 += xor32(e2);
  v2 += xor32(v2);
  const float rel = sqrtf(e2) / (sqrtf(v2) + 1e-6f);

  // cos^T[slot][tok] = ak . kr^T / (|ak| |kr|)
  Frag<T, HD> fk;
  fk.load(kr, tok, l, lane);
  float kk = fk.sumsq();
  kk += xor32(kk);
  const float inv_nk = 1.0f / fmaxf(sqrtf(kk), 1e-12f);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    acc[mb] = zero16();
    mm_rows_frag<HD>(acc[mb], sm.ak, sm.KS, 32 * mb, fk, lane);
  }
  float bv = -INFINITY;
  int bs = 0;
  bool first = true;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int s = 32 * mb + d_row(lane, r);
      float c = acc[mb][r] * sm.inv_nak[s] * inv_nk;
      if (!steady && !sm.act[s]) c = 0.f;
      if (first || ranks_before_desc(c, s, bv, bs)) { bv = c; bs = s; first = false; }
    }
  {
    const float ov = xor32(bv);
    const int os = xor32i(bs);
    if (ranks_before_desc(ov, os, bv, bs)) { bv = ov; bs = os; }
  }
  const float score = rel * (1.0f - fminf(fmaxf(bv, 0.0f), 1.0f));

  float simv = 0.f;
  if (steady) {
    // cos(v_tok, av[best]) over this lane's half of the features
    float dvv = 0.f, vv = 0.f, aa = 0.f;
    if (tok < l) {
      for (int d = h * (HD / 2); d < (h + 1) * (HD / 2); ++d) {
        const float x = St<T>::ld(v + (long long)tok * HD + d);
        const float y = St<T>::to_f(sm.av[bs * sm.KS + d]);
        dvv += x * y;
        vv += x * x;
        aa += y * y;
      }
    }
    dvv += xor32(dvv);
    vv += xor32(vv);
    aa += xor32(aa);
    simv = dvv / (fmaxf(sqrtf(vv), 1e-8f) * fmaxf(sqrtf(aa), 1e-8f));
  }
  if (h == 0 && tok < l) {
    sm.rel[tok] = rel;
    sm.score[tok] = score;
    sm.best[tok] = bv;
    sm.simv[tok] = simv;
    sm.slot[tok] = bs;
    sm.inv_nkr[tok] = inv_nk;
    sm.flags[tok] = (steady && bv >= SIM_K && simv >= SIM_V) ? F_MERGE : 0;
  }
}

// ----------------------------------------------------------------- delta rule (phase E)

// gersh_j = max(sum_i |khat_i . khat_j| w_i, 1); bsafe_j = w_j / gersh_j
template <typename T, int HD>
__device__ void gershgorin(ChainSmem<T, HD>& sm, const T* kr, int l, int wave, int lane) {
  const int nT = (l + 31) / 32;
  const int n = lane & 31;
  for (int tj = wave; tj < nT; tj += NWAVE) {
    const int j = 32 * tj + n;
    Frag<T, HD> fj;
    fj.load(kr, j, l, lane);
    float colsum = 0.f;
    for (int ti = 0; ti < nT; ++ti) {
      f32x16 acc = zero16();
      // rows i of tile ti as A operand, read from global memory
      const int m = 32 * ti + (lane & 31), h = lane >> 5;
      if constexpr (St<T>::is_bf16) {
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
          u16x8 a;
          if (m < l) a = *reinterpret_cast<const u16x8*>(kr + (long long)m * HD + 16 * ks + 8 * h);
          else {
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = 0;
          }
          mma_bf16(acc, a, fj.v[ks]);
        }
      } else {
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, m < l ? kr[(long long)m * HD + 2 * ks + h] : 0.f, fj.v[ks]);
      }
      const float inj = j < l ? sm.inv_nkr[j] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * ti + d_row(lane, r);
        if (i < l) colsum += fabsf(acc[r] * sm.inv_nkr[i] * inj) * sm.w[i];
      }
    }
    colsum += xor32(colsum);
    if ((lane >> 5) == 0 && j < l) sm.bsafe[j] = sm.w[j] / fmaxf(colsum, 1.0f);
  }
}

// M <- gamma*M + K^T diag(bsafe) (V - K M) with K = normalized keys.
template <typename T, int HD>
__device__ void delta_update(ChainSmem<T, HD>& sm, float* M, float* errg, const T* kr, const T* v, int l,
                             float gam, int wave, int lane, int tid) {
  constexpr int NB = HD / 32;               // row/col blocks of M
  constexpr int NBLK = NB * NB;
  constexpr int PER_WAVE = (NBLK + NWAVE - 1) / NWAVE;
  float* err = sm.ERR_LDS ? sm.err : errg;  // [32][ES] error tile
  const int ES = sm.ES;
  const int n = lane & 31, h = lane >> 5;
  f32x16 upd[PER_WAVE];
#pragma unroll
  for (int q = 0; q < PER_WAVE; ++q) upd[q] = zero16();
  const int nT = (l + 31) / 32;

  for (int t = 0; t < nT; ++t) {
    const int t0 = 32 * t;
    // v_pred^T[d][j] = sum_c M[c][d] kr[j][c]; wave w takes d-block w
    for (int db = wave; db < NB; db += NWAVE) {
      const int j = t0 + n;
      Frag<T, HD> fj;
      fj.load(kr, j, l, lane);
      f32x16 acc = zero16();
      const int d = 32 * db + n;
      if constexpr (St<T>::is_bf16) {
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
          float mv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) mv[i] = M[(16 * ks + 8 * h + i) * HD + d];
          u16x8 hi, lo;
          split8(mv, hi, lo);
          mma_bf16(acc, hi, fj.v[ks]);
          mma_bf16(acc, lo, fj.v[ks]);
        }
      } else {
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, M[(2 * ks + h) * HD + d], fj.v[ks]);
      }
      const float inj = j < l ? sm.inv_nkr[j] : 0.f;
      const float bj = j < l ? sm.bsafe[j] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dd = 32 * db + d_row(lane, r);
        const float x = j < l ? St<T>::ld(v + (long long)j * HD + dd) : 0.f;
        const float e = (x - acc[r] * inj) * bj;
        err[n * ES + dd] = e * inj;
      }
    }
    __syncthreads();
    // upd[c][d] += sum_j kr[j][c] err[j][d]
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      const int blk = wave + NWAVE * q;
      if (blk < NBLK) {
        const int cb = blk / NB, db = blk % NB;
        const int c = 32 * cb + n, d = 32 * db + n;
        if constexpr (St<T>::is_bf16) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            u16x8 a;
            float ev[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int jj = 16 * kc + 8 * h + i;
              a[i] = (t0 + jj < l) ? kr[(long long)(t0 + jj) * HD + c] : (uint16_t)0;
              ev[i] = err[jj * ES + d];
            }
            u16x8 hi, lo;
            split8(ev, hi, lo);
            mma_bf16(upd[q], a, hi);
            mma_bf16(upd[q], a, lo);
          }
        } else {
#pragma unroll
          for (int kc = 0; kc < 16; ++kc) {
            const int jj = 2 * kc + h;
            const float a = (t0 + jj < l) ? kr[(long long)(t0 + jj) * HD + c] : 0.f;
            mma_f32(upd[q], a, err[jj * ES + d]);
          }
        }
      }
    }
    __syncthreads();
  }
  // M = gamma*M + upd (two rounded ops, as the reference evaluates them)
#pragma unroll
  for (int q = 0; q < PER_WAVE; ++q) {
    const int blk = wave + NWAVE * q;
    if (blk < NBLK) {
      const int cb = blk / NB, db = blk % NB;
      const int d = 32 * db + n;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 32 * cb + d_row(lane, r);
        float* p = M + c * HD + d;
        *p = add_rn(mul_rn(gam, *p), upd[q][r]);
      }
    }
  }
}

// ----------------------------------------------------------------- kernel

template <typename T, int HD>
__global__ void __launch_bounds__(NT) chain_kernel(b3_chain_args a) {
  __shared__ ChainSmem<T, HD> sm;
  const int bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hkv = bh % a.HKV;
  const float kap = a.kappa[hkv], gam = a.gamma[hkv];
  const float scale = 1.0f / sqrtf((float)HD);
  const int KS = sm.KS;

  T* g_ak = reinterpret_cast<T*>(a.ak) + (long long)bh * S * HD;
  T* g_av = reinterpret_cast<T*>(a.av) + (long long)bh * S * HD;
  float* M = a.m_res + (long long)bh * HD * HD;
  const long long kv_blk = (long long)a.B * a.HKV * S * HD;  // elements per step in snapshot arrays
  // scratch: roped slot keys of the current state, and (fp32 HD=128) the error tile
  T* kread_w = reinterpret_cast<T*>(a.work) + (long long)bh * S * HD;
  float* errg = reinterpret_cast<float*>(reinterpret_cast<char*>(a.work) + kv_blk * sizeof(T)) + (long long)bh * 32 * sm.ES;

  // load state
  for (int it = tid; it < S * HD; it += NT) {
    const int s = it / HD, d = it % HD;
    sm.ak[s * KS + d] = g_ak[it];
    sm.av[s * KS + d] = g_av[it];
  }
  if (tid < S) {
    sm.mass[tid] = a.mass[bh * S + tid];
    sm.util[tid] = a.util[bh * S + tid];
    sm.pm[tid] = a.pm[bh * S + tid];
    sm.act[tid] = a.act[bh * S + tid] ? 1 : 0;
  }
  __syncthreads();
  int nf = a.n_filled;
  const T* kread = kread_w;
  if (nf > 0) {
    rope_slots_to<T, HD>(kread_w, sm, a.inv_freq, tid);
    __threadfence_block();
  }
  __syncthreads();

  for (int step = 0; step < a.n_steps; ++step) {
    const int off = step == 0 ? a.off0 : step * a.step_stride;
    const int l = step == 0 ? a.len0 : a.step_len;
    const long long tb = (long long)bh * a.tok_bh_stride + (long long)off * HD;
    const T* kr = reinterpret_cast<const T*>(a.kr) + tb;
    const T* kp = reinterpret_cast<const T*>(a.kp) + tb;
    const T* v = reinterpret_cast<const T*>(a.v) + tb;
    const float* pos = a.pos + off;
    const float* beta = a.beta + (long long)bh * a.beta_bh_stride + off;
    const int nT = (l + 31) / 32;
    const bool steady = nf >= S;
    float* log = a.log ? a.log + ((long long)step * (a.B * a.HKV) + bh) * (B3_LOG_ROWS * B3_LOG_COLS) : nullptr;

    if (tid < S) sm.util[tid] = mul_rn(sm.util[tid], UTIL_DECAY);
    if (tid < S) {
      const float lm = logf(fmaxf(sm.mass[tid], 1.0f));
      sm.bias[tid] = steady ? mul_rn(kap, lm) : lm;
    }
    slot_norms<T, HD>(sm, tid);
    for (int j = tid; j < LMAX; j += NT) { sm.flags[j] = 0; sm.w[j] = 0.f; sm.bsafe[j] = 0.f; }
    __syncthreads();

    if (!steady) {
      // ---------------- fill
      const int m = min(S - nf, l);
      if (nf == 0) {
        // score = unbiased variance of normalize(v)
        const int j = tid;
        if (j < l) {
          const T* vr = v + (long long)j * HD;
          float ss = 0.f;
          for (int d = 0; d < HD; ++d) { const float x = St<T>::ld(vr + d); ss += x * x; }
          const float nrm = fmaxf(sqrtf(ss), 1e-12f);
          float mean = 0.f;
          for (int d = 0; d < HD; ++d) mean += div_rn(St<T>::ld(vr + d), nrm);
          mean /= (float)HD;
          float var = 0.f;
          for (int d = 0; d < HD; ++d) { const float u = div_rn(St<T>::ld(vr + d), nrm) - mean; var += u * u; }
          sm.score[j] = var / (float)(HD - 1);
          sm.rel[j] = 0.15f;
        }
      } else {
        for (int t = wave; t < nT; t += NWAVE) score_tile<T, HD>(sm, kread, kr, kp, v, 32 * t, l, false, scale, lane);
      }
      __syncthreads();
      sm.sk_a[tid] = tid < l ? sm.score[tid] : -INFINITY;
      sm.si_a[tid] = tid;
      __syncthreads();
      bitonic_256(sm.sk_a, sm.si_a, true, tid);
      // slots nf + i <- token si_a[i]
      for (int it = tid; it < m * HD; it += NT) {
        const int i = it / HD, d = it % HD;
        const int j = sm.si_a[i], s = nf + i;
        sm.ak[s * KS + d] = kr[(long long)j * HD + d];
        sm.av[s * KS + d] = v[(long long)j * HD + d];
      }
      if (tid < m) {
        const int j = sm.si_a[tid], s = nf + tid;
        sm.pm[s] = pos[j];
        sm.mass[s] = 1.0f;
        sm.util[s] = sm.rel[j];
        sm.act[s] = 1;
      }
      if (log) {
        for (int j = tid; j < B3_LOG_COLS; j += NT) {
          log[B3_LOG_REL * B3_LOG_COLS + j] = j < l ? sm.rel[j] : 0.f;
          log[B3_LOG_SCORE * B3_LOG_COLS + j] = j < l ? sm.score[j] : 0.f;
          log[B3_LOG_TOPTOK * B3_LOG_COLS + j] = j < m ? (float)sm.si_a[j] : -1.f;
        }
      }
      nf += m;
      __syncthreads();
    } else {
      // ---------------- steady: score
      for (int t = wave; t < nT; t += NWAVE) score_tile<T, HD>(sm, kread, kr, kp, v, 32 * t, l, true, scale, lane);
      __syncthreads();

      // ---------------- merge: per-slot mass-weighted means, tokens in ascending order
      if (tid < S) {
        int c = 0;
        float ps = 0.f;
        for (int j = 0; j < l; ++j)
          if ((sm.flags[j] & F_MERGE) && sm.slot[j] == tid) { ++c; ps += pos[j]; }
        sm.cnt[tid] = c;
        sm.psum[tid] = ps;
      }
      __syncthreads();
      if (tid == 0) {
        int o = 0, nh = 0;
        for (int s = 0; s < S; ++s) {
          sm.off[s] = o;
          o += sm.cnt[s];
          if (sm.cnt[s] > 0) sm.hits[nh++] = s;
        }
        sm.nhit = nh;
      }
      __syncthreads();
      const int nhit = sm.nhit;
      if (nhit > 0) {
        if (tid < l && (sm.flags[tid] & F_MERGE)) {
          const int s = sm.slot[tid];
          int rank = 0;
          for (int j = 0; j < tid; ++j) rank += ((sm.flags[j] & F_MERGE) && sm.slot[j] == s) ? 1 : 0;
          sm.mlist[sm.off[s] + rank] = tid;
        }
        __syncthreads();
        for (int it = tid; it < nhit * HD; it += NT) {
          const int s = sm.hits[it / HD], d = it % HD;
          float ks = 0.f, vs = 0.f;
          for (int q = 0; q < sm.cnt[s]; ++q) {
            const int j = sm.mlist[sm.off[s] + q];
            ks += St<T>::ld(kr + (long long)j * HD + d);
            vs += St<T>::ld(v + (long long)j * HD + d);
          }
          const float m0 = sm.mass[s], nm = add_rn(m0, (float)sm.cnt[s]);
          sm.ak[s * KS + d] = St<T>::from_f(div_rn(add_rn(mul_rn(m0, St<T>::to_f(sm.ak[s * KS + d])), ks), nm));
          sm.av[s * KS + d] = St<T>::from_f(div_rn(add_rn(mul_rn(m0, St<T>::to_f(sm.av[s * KS + d])), vs), nm));
        }
        __syncthreads();
        if (tid < S && sm.cnt[tid] > 0) {
          const float m0 = sm.mass[tid], nm = add_rn(m0, (float)sm.cnt[tid]);
          sm.pm[tid] = div_rn(add_rn(mul_rn(m0, sm.pm[tid]), sm.psum[tid]), nm);
          sm.mass[tid] = nm;
        }
        __syncthreads();
        slot_norms<T, HD>(sm, tid);
        __syncthreads();
      }

      // ---------------- keep score: util * (1 - clamp(max_{s'!=s} cos(ak_s, ak_s'), 0, .98))
      {
        const int n = lane & 31;
        const int col = 32 * wave + n;  // 4 waves x 32 columns = S
        Frag<T, HD> fc;
        {
          const int h = lane >> 5;
          if constexpr (St<T>::is_bf16) {
#pragma unroll
            for (int ks = 0; ks < HD / 16; ++ks) fc.v[ks] = *reinterpret_cast<const u16x8*>(&sm.ak[col * KS + 16 * ks + 8 * h]);
          } else {
#pragma unroll
            for (int ks = 0; ks < HD / 2; ++ks) fc.v[ks] = sm.ak[col * KS + 2 * ks + h];
          }
        }
        float mx = -INFINITY;
        bool has_nan = false;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          f32x16 acc = zero16();
          mm_rows_frag<HD>(acc, sm.ak, KS, 32 * mb, fc, lane);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = 32 * mb + d_row(lane, r);
            // one rounded product of the two inverse norms keeps the matrix bitwise symmetric,
            // so mutual nearest slots (equal utility) get bit-equal keep values as in the reference
            const float c = row == col ? -1.0f : acc[r] * (sm.inv_nak[row] * sm.inv_nak[col]);
            has_nan |= (c != c);
            mx = fmaxf(mx, c);
          }
        }
        mx = fmaxf(mx, xor32(mx));
        has_nan |= __shfl_xor((int)has_nan, 32, 64) != 0;
        if (has_nan) mx = NAN;
        if ((lane >> 5) == 0) sm.keep[col] = mul_rn(sm.util[col], 1.0f - fminf(fmaxf(mx, 0.0f), 0.98f));
      }
      // ---------------- eviction candidates vs least useful slots
      sm.sk_a[tid] = tid < l ? ((sm.flags[tid] & F_MERGE) ? -1e9f : sm.score[tid]) : -INFINITY;
      sm.si_a[tid] = tid;
      __syncthreads();
      if (tid < S) { sm.sk_b[tid] = sm.keep[tid]; sm.si_b[tid] = tid; }
      bitonic_256(sm.sk_a, sm.si_a, true, tid);
      bitonic_128_asc(sm.sk_b, sm.si_b, tid);
      const int kc = min(l, S);
      // win_i = top_i > bot_i and top_i > -1e8 ; token top_i replaces slot bot_i
      if (tid < kc) {
        const float tv = sm.sk_a[tid], bv = sm.sk_b[tid];
        if (tv > bv && tv > -1e8f) sm.flags[sm.si_a[tid]] |= F_INS;
      }
      __syncthreads();
      for (int it = tid; it < kc * HD; it += NT) {
        const int i = it / HD, d = it % HD;
        const float tv = sm.sk_a[i], bv = sm.sk_b[i];
        if (tv > bv && tv > -1e8f) {
          const int j = sm.si_a[i], s = sm.si_b[i];
          sm.ak[s * KS + d] = kr[(long long)j * HD + d];
          sm.av[s * KS + d] = v[(long long)j * HD + d];
        }
      }
      if (tid < kc) {
        const float tv = sm.sk_a[tid], bv = sm.sk_b[tid];
        if (tv > bv && tv > -1e8f) {
          const int j = sm.si_a[tid], s = sm.si_b[tid];
          sm.pm[s] = pos[j];
          sm.mass[s] = 1.0f;
          sm.util[s] = sm.rel[j];
        }
      }
      if (tid < l) {
        const int f = sm.flags[tid];
        const bool dl = !(f & F_MERGE) && !(f & F_INS);
        if (dl) sm.flags[tid] = f | F_DELTA;
        sm.w[tid] = dl ? beta[tid] : 0.f;
      }
      __syncthreads();
      if (log) {
        for (int j = tid; j < B3_LOG_COLS; j += NT) {
          const bool in = j < l;
          log[B3_LOG_REL * B3_LOG_COLS + j] = in ? sm.rel[j] : 0.f;
          log[B3_LOG_SCORE * B3_LOG_COLS + j] = in ? sm.score[j] : 0.f;
          log[B3_LOG_BEST * B3_LOG_COLS + j] = in ? sm.best[j] : 0.f;
          log[B3_LOG_SIMV * B3_LOG_COLS + j] = in ? sm.simv[j] : 0.f;
          log[B3_LOG_SLOT * B3_LOG_COLS + j] = in ? (float)sm.slot[j] : -1.f;
          log[B3_LOG_MERGE * B3_LOG_COLS + j] = in ? (float)((sm.flags[j] & F_MERGE) != 0) : 0.f;
          log[B3_LOG_DELTA * B3_LOG_COLS + j] = in ? (float)((sm.flags[j] & F_DELTA) != 0) : 0.f;
          log[B3_LOG_TOPTOK * B3_LOG_COLS + j] = j < kc ? (float)sm.si_a[j] : -1.f;
          log[B3_LOG_BOTSLOT * B3_LOG_COLS + j] = j < kc ? (float)sm.si_b[j] : -1.f;
          log[B3_LOG_WIN * B3_LOG_COLS + j] =
              j < kc ? (float)(sm.sk_a[j] > sm.sk_b[j] && sm.sk_a[j] > -1e8f) : 0.f;
          log[B3_LOG_KEEP * B3_LOG_COLS + j] = j < S ? sm.keep[j] : 0.f;
          log[B3_LOG_TOPVAL * B3_LOG_COLS + j] = j < kc ? sm.sk_a[j] : 0.f;
          log[B3_LOG_BOTVAL * B3_LOG_COLS + j] = j < kc ? sm.sk_b[j] : 0.f;
        }
      }

      // ---------------- Gershgorin-safe delta rule into M_res
      gershgorin<T, HD>(sm, kr, l, wave, lane);
      __syncthreads();
      delta_update<T, HD>(sm, M, errg, kr, v, l, gam, wave, lane, tid);
      __syncthreads();
    }

    // ---------------- per-step outputs; the roped keys also serve the next step
    T* kdst = a.snap_k ? reinterpret_cast<T*>(a.snap_k) + step * kv_blk + (long long)bh * S * HD : kread_w;
    rope_slots_to<T, HD>(kdst, sm, a.inv_freq, tid);
    kread = kdst;
    if (a.snap_v) {
      T* vd = reinterpret_cast<T*>(a.snap_v) + step * kv_blk + (long long)bh * S * HD;
      for (int it = tid; it < S * HD; it += NT) vd[it] = sm.av[(it / HD) * KS + it % HD];
    }
    if (a.snap_bias && tid < S) {
      a.snap_bias[(long long)step * a.B * a.HKV * S + bh * S + tid] =
          sm.act[tid] ? mul_rn(kap, logf(fmaxf(sm.mass[tid], 1.0f))) : -INFINITY;
    }
    if (a.snap_m) {
      float* md = a.snap_m + (long long)step * a.B * a.HKV * HD * HD + (long long)bh * HD * HD;
      for (int it = tid; it < HD * HD; it += NT) md[it] = M[it];
    }
    __threadfence_block();
    __syncthreads();
  }

  // store state
  for (int it = tid; it < S * HD; it += NT) {
    g_ak[it] = sm.ak[(it / HD) * KS + it % HD];
    g_av[it] = sm.av[(it / HD) * KS + it % HD];
  }
  if (tid < S) {
    a.mass[bh * S + tid] = sm.mass[tid];
    a.util[bh * S + tid] = sm.util[tid];
    a.pm[bh * S + tid] = sm.pm[tid];
    a.act[bh * S + tid] = (uint8_t)sm.act[tid];
  }
}

template <typename T, int HD>
static int launch_chain(const b3_chain_args& a, hipStream_t st) {
  hipLaunchKernelGGL((chain_kernel<T, HD>), dim3(a.B * a.HKV), dim3(NT), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int64_t bolt3_chain_workspace_bytes(int32_t dtype, int32_t B, int32_t HKV, int32_t HD, int32_t S) {
  const int64_t es = dtype == B3_BF16 ? 2 : 4;
  const int64_t bh = (int64_t)B * HKV;
  return bh * S * HD * es + bh * 32 * (HD + 4) * 4;
}

extern "C" int bolt3_chain(const b3_chain_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->n_steps < 0) return B3_ERR_ARG;
  if (a->S != b3::S || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  if (a->n_steps == 0) return B3_OK;
  if (a->len0 < 1 || a->len0 > b3::LMAX || (a->n_steps > 1 && (a->step_len < 1 || a->step_len > b3::LMAX)))
    return B3_ERR_UNSUPPORTED;
  if (a->n_filled < 0 || a->n_filled > b3::S) return B3_ERR_ARG;
  if (!a->kr || !a->kp || !a->v || !a->pos || !a->beta || !a->ak || !a->av || !a->mass || !a->util || !a->pm ||
      !a->act || !a->m_res || !a->kappa || !a->gamma || !a->inv_freq || !a->work)
    return B3_ERR_ARG;
  if (a->work_bytes < bolt3_chain_workspace_bytes(a->dtype, a->B, a->HKV, a->HD, a->S)) return B3_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return a->HD == 64 ? b3::launch_chain<float, 64>(*a, st) : b3::launch_chain<float, 128>(*a, st);
  if (a->dtype == B3_BF16)
    return a->HD == 64 ? b3::launch_chain<uint16_t, 64>(*a, st) : b3::launch_chain<uint16_t, 128>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

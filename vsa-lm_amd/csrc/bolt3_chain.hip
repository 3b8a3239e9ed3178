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
// masses, utilities, positions and activity stay in LDS for all steps.  M_res
// is kept transposed in the workspace, in fp32 and (bf16 storage) split into
// bf16 hi + lo, so every MFMA operand is one 16-byte load; the state array
// [bh][HD][HD] is written after every step.  bf16 storage multiplies exact
// bf16 operands (products are exact in fp32) and splits fp32 operands into
// hi + lo; fp32 storage uses the fp32 MFMA.  Orderings are ranks computed by
// counting on monotone integer keys (one pass, stable): the larger value
// first (NaN first), equal values by lower index.
#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int S = 128;     // attractor slots
constexpr int LMAX = 256;  // tokens per consolidation step
constexpr int NT = 256;    // threads per workgroup
constexpr int NWAVE = NT / WAVE;
constexpr float SIM_K = 0.88f, SIM_V = 0.80f, UTIL_DECAY = 0.995f;

enum : int { F_MERGE = 1, F_DELTA = 2, F_INS = 4 };

// Workspace layout per bh (bytes): roped slot keys of the current state, M^T fp32,
// M^T bf16 hi and lo, and (when they do not fit in LDS) the delta-rule tile buffers.
template <typename T, int HD>
struct Work {
  static constexpr long long KREAD = (long long)S * HD * sizeof(T);
  static constexpr long long MT32 = (long long)HD * HD * 4;
  static constexpr long long MTBF = (long long)HD * HD * 2;
  static constexpr long long TILE = 2LL * HD * 33 * 4;
  static constexpr long long PER_BH = KREAD + MT32 + 2 * MTBF + TILE;
};

template <typename T, int HD>
struct ChainSmem {
  static constexpr int KS = sizeof(T) == 2 ? HD + 8 : HD + 4;   // slot row stride (16-byte aligned rows)
  static constexpr int TS = sizeof(T) == 2 ? 32 + 8 : 32 + 1;   // token-tile row stride (transposed tiles)
  static constexpr bool TILE_LDS = !(sizeof(T) == 4 && HD == 128);
  alignas(16) T ak[S * KS];
  alignas(16) T av[S * KS];
  float mass[S], util[S], pm[S], inv_nak[S], keep[S], bias[S], psum[S];
  int act[S], cnt[S], off[S], hits[S];
  float rel[LMAX], score[LMAX], best[LMAX], simv[LMAX], inv_nkr[LMAX], w[LMAX], bsafe[LMAX], ck[LMAX];
  int slot[LMAX], flags[LMAX], mlist[LMAX];
  float sk_a[LMAX];
  int si_a[LMAX];
  float sk_b[S];
  int si_b[S];
  uint32_t ok_a[LMAX], ok_b[S];   // order keys
  // delta-rule tiles: K^T [HD][32] and the error tile E^T [HD][32] (bf16: hi and lo)
  static constexpr bool KREAD_LDS = sizeof(T) == 2;              // roped slot keys of the current state
  alignas(16) T kread[KREAD_LDS ? S * KS : 1];
  alignas(16) T krt[TILE_LDS ? HD * TS : 1];
  alignas(16) T ert_hi[TILE_LDS ? HD * TS : 1];
  alignas(16) uint16_t ert_lo[(TILE_LDS && sizeof(T) == 2) ? HD * TS : 1];
  int nhit;
};

// ----------------------------------------------------------------- fragments

// Token-tile fragment: lane (n = lane%32, h = lane/32) holds row tok, K sub-index
// 16*ks + 8*h + i (bf16) or 2*ks + h (fp32).
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
  __device__ __forceinline__ void load_lds(const uint16_t* rows, int rs, int r, int lane) {
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) v[ks] = *reinterpret_cast<const u16x8*>(rows + r * rs + 16 * ks + 8 * h);
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
  __device__ __forceinline__ void load_lds(const float* rows, int rs, int r, int lane) {
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) v[ks] = rows[r * rs + 2 * ks + h];
  }
  __device__ __forceinline__ float sumsq() const {
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) s += v[ks] * v[ks];
    return s;
  }
};

// acc += rows[row0 + lane%32][:] . frag over HD  (rows: LDS or global, row stride rs)
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

// 8 consecutive elements as floats (16-byte bf16 or two 16-byte fp32 loads)
__device__ __forceinline__ void ld8(const uint16_t* p, float* o) {
  const u16x8 v = *reinterpret_cast<const u16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = bf2f(v[i]);
}
__device__ __forceinline__ void ld8(const float* p, float* o) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// 8 consecutive elements, 16-byte (bf16) or 2 x 16-byte (fp32) moves; both pointers aligned
__device__ __forceinline__ void copy8(uint16_t* d, const uint16_t* s) {
  *reinterpret_cast<u16x8*>(d) = *reinterpret_cast<const u16x8*>(s);
}
__device__ __forceinline__ void copy8(float* d, const float* s) {
  *reinterpret_cast<float4*>(d) = *reinterpret_cast<const float4*>(s);
  *reinterpret_cast<float4*>(d + 4) = *reinterpret_cast<const float4*>(s + 4);
}

// ----------------------------------------------------------------- helpers

// Slot keys roped at their mean positions -> `dst` (global, may be null) and, for bf16
// storage, the LDS copy the next scoring reads.
template <typename T, int HD>
__device__ void rope_slots_to(T* dst, ChainSmem<T, HD>& sm, const float* inv_freq, int tid) {
  constexpr int HALF = HD / 2;
  for (int it = tid; it < S * HALF; it += NT) {
    const int s = it / HALF, i = it % HALF;
    float sn, cs;
    sincos_rope(mul_rn(sm.pm[s], inv_freq[i]), &sn, &cs);
    const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
    const float x0 = St<T>::to_f(sm.ak[s * sm.KS + i]), x1 = St<T>::to_f(sm.ak[s * sm.KS + i + HALF]);
    const T r0 = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x0, c)), St<T>::rnd(mul_rn(-x1, si))));
    const T r1 = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x1, c)), St<T>::rnd(mul_rn(x0, si))));
    if (dst) {
      dst[s * HD + i] = r0;
      dst[s * HD + i + HALF] = r1;
    }
    if constexpr (ChainSmem<T, HD>::KREAD_LDS) {
      sm.kread[s * sm.KS + i] = r0;
      sm.kread[s * sm.KS + i + HALF] = r1;
    }
  }
}

// 1 / max(||ak_s||, 1e-12) for every slot (two threads per slot).
template <typename T, int HD>
__device__ void slot_norms(ChainSmem<T, HD>& sm, int tid) {
  const int s = tid >> 1, half = tid & 1;
  float ss = 0.f;
#pragma unroll
  for (int d = half * (HD / 2); d < (half + 1) * (HD / 2); d += 8) {
    float x[8];
    ld8(&sm.ak[s * sm.KS + d], x);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
  }
  ss += __shfl_xor(ss, 1, 64);
  if (half == 0) sm.inv_nak[s] = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
}

// Monotone integer image of a float: a < b  <=>  ord(a) < ord(b); NaN maps above +inf, so
// it ranks first in a descending and last in an ascending order (torch.topk's placement).
// -0 and +0 map to adjacent keys.
__device__ __forceinline__ uint32_t ord_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Rank of element `me` among ok[0..n) (order keys), ties by lower index.
__device__ __forceinline__ int rank_desc(const uint32_t* ok, int n, int me) {
  const uint32_t x = ok[me];
  int r = 0;
  for (int i = 0; i < n; ++i) {
    const uint32_t y = ok[i];
    r += (y > x || (y == x && i < me)) ? 1 : 0;
  }
  return r;
}
__device__ __forceinline__ int rank_asc(const uint32_t* ok, int n, int me) {
  const uint32_t x = ok[me];
  int r = 0;
  for (int i = 0; i < n; ++i) {
    const uint32_t y = ok[i];
    r += (y < x || (y == x && i < me)) ? 1 : 0;
  }
  return r;
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
      if constexpr (ChainSmem<T, HD>::KREAD_LDS) mm_rows_frag<HD>(acc[mb], sm.kread, sm.KS, 32 * mb, f, lane);
      else mm_rows_frag<HD>(acc[mb], kread, HD, 32 * mb, f, lane);
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
  if (tok < l) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * h;
        float x[4];
        if constexpr (St<T>::is_bf16) {
          const u16x4 q = *reinterpret_cast<const u16x4*>(v + (long long)tok * HD + d0);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = bf2f(q[i]);
        } else {
          const float4 q = *reinterpret_cast<const float4*>(v + (long long)tok * HD + d0);
          x[0] = q.x; x[1] = q.y; x[2] = q.z; x[3] = q.w;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dv = x[i] - St<T>::rnd(vh[db][4 * g + i]);
          e2 += dv * dv;
          v2 += x[i] * x[i];
        }
      }
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
      float c = acc[mb][r] * (sm.inv_nak[s] * inv_nk);
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
#pragma unroll
      for (int d = h * (HD / 2); d < (h + 1) * (HD / 2); d += 8) {
        float x[8], y[8];
        ld8(v + (long long)tok * HD + d, x);
        ld8(&sm.av[bs * sm.KS + d], y);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dvv += x[i] * y[i];
          vv += x[i] * x[i];
          aa += y[i] * y[i];
        }
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
    const float inj = j < l ? sm.inv_nkr[j] : 0.f;
    float colsum = 0.f;
    for (int ti = 0; ti < nT; ++ti) {
      f32x16 acc = zero16();
      Frag<T, HD> fi;
      fi.load(kr, 32 * ti + (lane & 31), l, lane);
      // rows i of tile ti as the A operand: same fragment layout as a B fragment
      if constexpr (St<T>::is_bf16) {
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) mma_bf16(acc, fi.v[ks], fj.v[ks]);
      } else {
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, fi.v[ks], fj.v[ks]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * ti + d_row(lane, r);
        if (i < l) colsum += fabsf(acc[r] * (sm.inv_nkr[i] * inj)) * sm.w[i];
      }
    }
    colsum += xor32(colsum);
    if ((lane >> 5) == 0 && j < l) sm.bsafe[j] = sm.w[j] / fmaxf(colsum, 1.0f);
  }
}

// M <- gamma*M + K^T diag(bsafe) (V - K M) with K = normalized keys, M kept as M^T.
template <typename T, int HD>
__device__ void delta_update(ChainSmem<T, HD>& sm, char* ws, float* M, float* snap_m, const T* kr, const T* v,
                             int l, float gam, int wave, int lane, int tid) {
  using W = Work<T, HD>;
  constexpr int NB = HD / 32;
  constexpr int NBLK = NB * NB;
  constexpr int PER_WAVE = (NBLK + NWAVE - 1) / NWAVE;
  const int TS = sm.TS;
  float* mt32 = reinterpret_cast<float*>(ws + W::KREAD);
  uint16_t* mthi = reinterpret_cast<uint16_t*>(ws + W::KREAD + W::MT32);
  uint16_t* mtlo = mthi + HD * HD;
  T* krt = sm.TILE_LDS ? sm.krt : reinterpret_cast<T*>(ws + W::KREAD + W::MT32 + 2 * W::MTBF);
  T* ert = sm.TILE_LDS ? sm.ert_hi : krt + HD * 33;
  uint16_t* erl = sm.ert_lo;
  const int n = lane & 31, h = lane >> 5;
  f32x16 upd[PER_WAVE];
#pragma unroll
  for (int q = 0; q < PER_WAVE; ++q) upd[q] = zero16();
  const int nT = (l + 31) / 32;

  for (int t = 0; t < nT; ++t) {
    const int t0 = 32 * t;
    // K^T tile: krt[c][j] = kr[t0 + j][c]
    for (int it = tid; it < 32 * (HD / 8); it += NT) {
      const int j = it / (HD / 8), c8 = (it % (HD / 8)) * 8;
      float x[8];
      if (t0 + j < l) ld8(kr + (long long)(t0 + j) * HD + c8, x);
      else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) krt[(c8 + i) * TS + j] = St<T>::from_f(x[i]);
    }
    // v_pred^T[d][j] = sum_c M^T[d][c] kr[j][c]; error tile E^T[d][j] = (v - v_pred) * bsafe_j / |k_j|
    for (int db = wave; db < NB; db += NWAVE) {
      const int j = t0 + n;
      Frag<T, HD> fj;
      fj.load(kr, j, l, lane);
      f32x16 acc = zero16();
      const int d = 32 * db + n;
      if constexpr (St<T>::is_bf16) {
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
          const u16x8 hi = *reinterpret_cast<const u16x8*>(mthi + d * HD + 16 * ks + 8 * h);
          const u16x8 lo = *reinterpret_cast<const u16x8*>(mtlo + d * HD + 16 * ks + 8 * h);
          mma_bf16(acc, hi, fj.v[ks]);
          mma_bf16(acc, lo, fj.v[ks]);
        }
      } else {
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, mt32[d * HD + 2 * ks + h], fj.v[ks]);
      }
      const float inj = j < l ? sm.inv_nkr[j] : 0.f;
      const float bj = j < l ? sm.bsafe[j] : 0.f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * h;
        float x[4] = {0.f, 0.f, 0.f, 0.f};
        if (j < l) {
          if constexpr (St<T>::is_bf16) {
            const u16x4 q = *reinterpret_cast<const u16x4*>(v + (long long)j * HD + d0);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = bf2f(q[i]);
          } else {
            const float4 q = *reinterpret_cast<const float4*>(v + (long long)j * HD + d0);
            x[0] = q.x; x[1] = q.y; x[2] = q.z; x[3] = q.w;
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = ((x[i] - acc[4 * g + i] * inj) * bj) * inj;
          if constexpr (St<T>::is_bf16) {
            const uint16_t hb = f2bf(e);
            ert[(d0 + i) * TS + n] = hb;
            erl[(d0 + i) * TS + n] = f2bf(e - bf2f(hb));
          } else {
            ert[(d0 + i) * TS + n] = e;
          }
        }
      }
    }
    __syncthreads();
    // upd[c][d] += sum_j K^T[c][j] E^T[d][j]
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      const int blk = wave + NWAVE * q;
      if (blk < NBLK) {
        const int cb = blk / NB, db = blk % NB;
        const int c = 32 * cb + n, d = 32 * db + n;
        if constexpr (St<T>::is_bf16) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            const u16x8 a = *reinterpret_cast<const u16x8*>(krt + c * TS + 16 * kc + 8 * h);
            const u16x8 bh_ = *reinterpret_cast<const u16x8*>(ert + d * TS + 16 * kc + 8 * h);
            const u16x8 bl_ = *reinterpret_cast<const u16x8*>(erl + d * TS + 16 * kc + 8 * h);
            mma_bf16(upd[q], a, bh_);
            mma_bf16(upd[q], a, bl_);
          }
        } else {
#pragma unroll
          for (int kc = 0; kc < 16; ++kc) mma_f32(upd[q], krt[c * TS + 2 * kc + h], ert[d * TS + 2 * kc + h]);
        }
      }
    }
    __syncthreads();
  }
  // M = gamma*M + upd (two rounded ops, as the reference evaluates them); write M^T (fp32 and
  // bf16 hi/lo), the state M[c][d] and the snapshot
#pragma unroll
  for (int q = 0; q < PER_WAVE; ++q) {
    const int blk = wave + NWAVE * q;
    if (blk < NBLK) {
      const int cb = blk / NB, db = blk % NB;
      const int d = 32 * db + n;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = 32 * cb + 8 * g + 4 * h;
        const float4 old = *reinterpret_cast<const float4*>(mt32 + d * HD + c0);
        float nw[4];
        nw[0] = add_rn(mul_rn(gam, old.x), upd[q][4 * g + 0]);
        nw[1] = add_rn(mul_rn(gam, old.y), upd[q][4 * g + 1]);
        nw[2] = add_rn(mul_rn(gam, old.z), upd[q][4 * g + 2]);
        nw[3] = add_rn(mul_rn(gam, old.w), upd[q][4 * g + 3]);
        *reinterpret_cast<float4*>(mt32 + d * HD + c0) = make_float4(nw[0], nw[1], nw[2], nw[3]);
        u16x4 hi4, lo4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hi4[i] = f2bf(nw[i]);
          lo4[i] = f2bf(nw[i] - bf2f(hi4[i]));
          M[(c0 + i) * HD + d] = nw[i];
        }
        *reinterpret_cast<u16x4*>(mthi + d * HD + c0) = hi4;
        *reinterpret_cast<u16x4*>(mtlo + d * HD + c0) = lo4;
        if (snap_m) {
          if constexpr (St<T>::is_bf16) {
            uint16_t* sh = reinterpret_cast<uint16_t*>(snap_m);
            *reinterpret_cast<u16x4*>(sh + d * HD + c0) = hi4;
            *reinterpret_cast<u16x4*>(sh + HD * HD + d * HD + c0) = lo4;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) snap_m[(c0 + i) * HD + d] = nw[i];
          }
        }
      }
    }
  }
}

// ----------------------------------------------------------------- kernel

template <typename T, int HD>
__global__ void __launch_bounds__(NT) chain_kernel(b3_chain_args a) {
  __shared__ ChainSmem<T, HD> sm;
  using W = Work<T, HD>;
  const int bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hkv = bh % a.HKV;
  const float kap = a.kappa[hkv], gam = a.gamma[hkv];
  const float scale = 1.0f / sqrtf((float)HD);
  const int KS = sm.KS;

  T* g_ak = reinterpret_cast<T*>(a.ak) + (long long)bh * S * HD;
  T* g_av = reinterpret_cast<T*>(a.av) + (long long)bh * S * HD;
  float* M = a.m_res + (long long)bh * HD * HD;
  const long long BH = (long long)a.B * a.HKV;
  char* ws = reinterpret_cast<char*>(a.work) + (long long)bh * W::PER_BH;
  T* kread_w = reinterpret_cast<T*>(ws);
  float* mt32 = reinterpret_cast<float*>(ws + W::KREAD);
  uint16_t* mthi = reinterpret_cast<uint16_t*>(ws + W::KREAD + W::MT32);
  uint16_t* mtlo = mthi + HD * HD;

  // load state; M -> M^T (fp32, bf16 hi/lo) in the workspace
  for (int it = tid; it < S * HD; it += NT) {
    const int s = it / HD, d = it % HD;
    sm.ak[s * KS + d] = g_ak[it];
    sm.av[s * KS + d] = g_av[it];
  }
  for (int it = tid; it < HD * HD; it += NT) {
    const int c = it / HD, d = it % HD;
    const float x = M[it];
    mt32[d * HD + c] = x;
    const uint16_t hb = f2bf(x);
    mthi[d * HD + c] = hb;
    mtlo[d * HD + c] = f2bf(x - bf2f(hb));
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
  if (nf > 0) rope_slots_to<T, HD>(sm.KREAD_LDS ? nullptr : kread_w, sm, a.inv_freq, tid);
  __threadfence_block();
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
    float* log = a.log ? a.log + ((long long)step * BH + bh) * (B3_LOG_ROWS * B3_LOG_COLS) : nullptr;
    float* snap_m = a.snap_m ? a.snap_m + (long long)step * BH * HD * HD + (long long)bh * HD * HD : nullptr;

    if (tid < S) {
      sm.util[tid] = mul_rn(sm.util[tid], UTIL_DECAY);
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
          for (int d = 0; d < HD; d += 8) {
            float x[8];
            ld8(vr + d, x);
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
          }
          const float nrm = fmaxf(sqrtf(ss), 1e-12f);
          float mean = 0.f;
          for (int d = 0; d < HD; d += 8) {
            float x[8];
            ld8(vr + d, x);
#pragma unroll
            for (int i = 0; i < 8; ++i) mean += div_rn(x[i], nrm);
          }
          mean /= (float)HD;
          float var = 0.f;
          for (int d = 0; d < HD; d += 8) {
            float x[8];
            ld8(vr + d, x);
#pragma unroll
            for (int i = 0; i < 8; ++i) { const float u = div_rn(x[i], nrm) - mean; var += u * u; }
          }
          sm.score[j] = var / (float)(HD - 1);
          sm.rel[j] = 0.15f;
        }
      } else {
        for (int t = wave; t < nT; t += NWAVE) score_tile<T, HD>(sm, kread, kr, kp, v, 32 * t, l, false, scale, lane);
      }
      __syncthreads();
      if (tid < l) sm.ok_a[tid] = ord_key(sm.score[tid]);
      __syncthreads();
      if (tid < l) {
        const int r = rank_desc(sm.ok_a, l, tid);
        sm.si_a[r] = tid;
        sm.sk_a[r] = sm.score[tid];
      }
      __syncthreads();
      // slots nf + i <- token si_a[i]
      for (int it = tid; it < m * (HD / 8); it += NT) {
        const int i = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
        const int j = sm.si_a[i], s = nf + i;
        copy8(&sm.ak[s * KS + d8], kr + (long long)j * HD + d8);
        copy8(&sm.av[s * KS + d8], v + (long long)j * HD + d8);
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
      // M_res is unchanged by a fill: its snapshot is the current M
      if (snap_m) {
        for (int it = tid; it < HD * HD; it += NT) {
          if constexpr (St<T>::is_bf16) {
            reinterpret_cast<uint16_t*>(snap_m)[it] = mthi[it];
            reinterpret_cast<uint16_t*>(snap_m)[HD * HD + it] = mtlo[it];
          } else {
            snap_m[it] = M[it];
          }
        }
      }
      nf += m;
      __syncthreads();
    } else {
      // ---------------- steady: score
      for (int t = wave; t < nT; t += NWAVE) score_tile<T, HD>(sm, kread, kr, kp, v, 32 * t, l, true, scale, lane);
      const int has = tid < l && (sm.flags[tid] & F_MERGE);
      const int any_merge = __syncthreads_or(has);

      // ---------------- merge: per-slot mass-weighted means, tokens in ascending order
      if (any_merge) {
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
        fc.load_lds(sm.ak, KS, col, lane);
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
      if (tid < l) {
        sm.ck[tid] = (sm.flags[tid] & F_MERGE) ? -1e9f : sm.score[tid];
        sm.ok_a[tid] = ord_key(sm.ck[tid]);
      }
      __syncthreads();
      if (tid < S) sm.ok_b[tid] = ord_key(sm.keep[tid]);
      __syncthreads();
      // ---------------- orderings: best free tokens (desc) against least useful slots (asc)
      if (tid < l) {
        const int r = rank_desc(sm.ok_a, l, tid);
        sm.sk_a[r] = sm.ck[tid];
        sm.si_a[r] = tid;
      }
      if (tid < S) {
        const int r = rank_asc(sm.ok_b, S, tid);
        sm.sk_b[r] = sm.keep[tid];
        sm.si_b[r] = tid;
      }
      __syncthreads();
      const int kc = min(l, S);
      // win_i = top_i > bot_i and top_i > -1e8 ; token top_i replaces slot bot_i
      if (tid < kc) {
        const float tv = sm.sk_a[tid], bv = sm.sk_b[tid];
        if (tv > bv && tv > -1e8f) sm.flags[sm.si_a[tid]] |= F_INS;
      }
      __syncthreads();
      for (int it = tid; it < kc * (HD / 8); it += NT) {
        const int i = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
        const float tv = sm.sk_a[i], bv = sm.sk_b[i];
        if (tv > bv && tv > -1e8f) {
          const int j = sm.si_a[i], s = sm.si_b[i];
          copy8(&sm.ak[s * KS + d8], kr + (long long)j * HD + d8);
          copy8(&sm.av[s * KS + d8], v + (long long)j * HD + d8);
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
      delta_update<T, HD>(sm, ws, M, snap_m, kr, v, l, gam, wave, lane, tid);
      __syncthreads();
    }

    // ---------------- per-step outputs; the roped keys also serve the next step
    T* kdst = a.snap_k ? reinterpret_cast<T*>(a.snap_k) + step * BH * S * HD + (long long)bh * S * HD
                       : (sm.KREAD_LDS ? nullptr : kread_w);
    rope_slots_to<T, HD>(kdst, sm, a.inv_freq, tid);
    if (kdst) kread = kdst;
    if (a.snap_v) {
      T* vd = reinterpret_cast<T*>(a.snap_v) + step * BH * S * HD + (long long)bh * S * HD;
      for (int it = tid; it < S * (HD / 8); it += NT) {
        const int s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
        copy8(vd + s * HD + d8, &sm.av[s * KS + d8]);
      }
    }
    if (a.snap_bias && tid < S) {
      a.snap_bias[(long long)step * BH * S + bh * S + tid] =
          sm.act[tid] ? mul_rn(kap, logf(fmaxf(sm.mass[tid], 1.0f))) : -INFINITY;
    }
    __threadfence_block();
    __syncthreads();
  }

  // store state (M was written after every steady step)
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
  const int64_t bh = (int64_t)B * HKV;
  if (dtype == B3_BF16) return bh * (HD == 64 ? b3::Work<uint16_t, 64>::PER_BH : b3::Work<uint16_t, 128>::PER_BH);
  return bh * (HD == 64 ? b3::Work<float, 64>::PER_BH : b3::Work<float, 128>::PER_BH);
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

// Backward of the Bolt-3 chunk attention and M_res readout (gfx950).
//
// The forward of every chunk c is a joint softmax over four key fields of its (batch, kv head)
// row -- [sinks | attractor slots | previous chunk | own chunk (causal)] -- with the slot field's
// bias kappa*log(mass) (-inf for inactive slots), plus the readout
//     y += eta * RMSNorm(normalize(q_raw) . M * (1 - gamma) / sqrt(HD))
// for chunks c >= 2, which use the slot snapshot and M_res of consolidation step c - 2
// (vsa_lm/config/bolt3.py:219-256).  bolt3_attn_bwd runs three kernels:
//
//   readout_bwd_kernel, grid (B*HKV, chunks): per row D = sum_d dy * (attention output),
//     with the readout's own contribution taken out of y; the readout's gradients with respect
//     to eta, q_raw, M (one dM per chunk), res_norm's weight and gamma.
//   attn_bwd_dq_kernel, grid (query tiles, B*H, chunks): recomputes each row's log-sum-exp over
//     all key fields, then dS = P * (dO . V^T - D) block by block, dQ = scale * dS . K and the
//     slot columns' sums of dS (the gradient of the slot bias).
//   attn_bwd_dkv_kernel, grid (key blocks, B*HKV, chunks): one 32-key block of one field per
//     workgroup, over every query row of the chunk's G heads: dV = P^T . dO, dK = scale * dS^T . Q.
//     Every key row has one writer: the previous chunk's keys go to d_k_next, the chunk's own
//     keys to d_k_own, slots to d_slot_k of step c - 2, sinks to d_sink_k of chunk c.
//
// All arithmetic is fp32 (fp32 FMAs on the vector ALUs); operands of either storage dtype are
// widened while they are staged in LDS.  Scores are rebuilt like the forward's (the q.k
// product rounded to the storage dtype first when score_round is set, then scale, bias, mask).
#include <math.h>

#include "bolt3_common.h"
#include "bolt3_amd.h"

namespace b3 {
namespace bwd {

constexpr int NT = 256;     // threads of every backward workgroup
constexpr int BQ = 64;      // query rows per tile
constexpr int BK = 32;      // keys per block
constexpr int RT = 16;      // query rows per readout tile

// one key field of a chunk: rows of HD elements, `len` of them
struct KField {
  const void* k;
  const void* v;
  const float* bias;   // slots only
  int len;
  int kind;            // 0 sinks, 1 slots, 2 previous chunk, 3 own chunk
};

__device__ __forceinline__ int chunk_len(const b3_attn_bwd_args& a, int c) { return min(a.C, a.T - c * a.C); }

// which fields chunk c has: bit k for kind k (sinks and slots once step c - 2 exists)
__device__ __forceinline__ int field_mask(const b3_attn_bwd_args& a, int c) {
  const bool state = c >= 2 && c - 2 < a.n_steps;
  return (state && a.n_sinks > 0 ? 1 : 0) | (state ? 2 : 0) | (c >= 1 ? 4 : 0) | 8;
}

// the fi-th field of chunk c of row (b, hkv), in the order sinks, slots, previous chunk, own chunk
template <typename T>
__device__ __forceinline__ KField chunk_field(const b3_attn_bwd_args& a, int b, int hkv, int c, int fi) {
  const int mask = field_mask(a, c);
  int kind = 0;
  for (int k = 0, seen = 0; k < 4; ++k)
    if (mask & (1 << k)) {
      if (seen == fi) kind = k;
      ++seen;
    }
  const int HD = a.HD;
  const T* wk = reinterpret_cast<const T*>(a.win_k) + (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const T* wv = reinterpret_cast<const T*>(a.win_v) + (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  if (kind == 0) return KField{wk, wv, nullptr, min(a.n_sinks, a.C), 0};
  if (kind == 1) {
    const long long bh = (long long)b * a.HKV + hkv;
    const long long so = (long long)(c - 2) * a.slot_step + bh * a.S * HD;
    return KField{reinterpret_cast<const T*>(a.slot_k) + so, reinterpret_cast<const T*>(a.slot_v) + so,
                  a.slot_bias + (long long)(c - 2) * (a.slot_step / HD) + bh * a.S, a.S, 1};
  }
  if (kind == 2)
    return KField{wk + (long long)(c - 1) * a.C * HD, wv + (long long)(c - 1) * a.C * HD, nullptr, a.C, 2};
  return KField{wk + (long long)c * a.C * HD, wv + (long long)c * a.C * HD, nullptr, chunk_len(a, c), 3};
}

// rows [0, n_rows) of a [rows][HD] source (row stride `rs` elements) into fp32 LDS rows of
// stride `ls`; rows at or past n_valid are zeros
template <typename T, int HD>
__device__ __forceinline__ void stage_rows(float* lds, int ls, const T* src, long long rs, int n_rows, int n_valid,
                                           int tid) {
  for (int it = tid; it < n_rows * (HD / 4); it += NT) {
    const int r = it / (HD / 4), c4 = (it % (HD / 4)) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < n_valid) {
      const T* p = src + (long long)r * rs + c4;
      if constexpr (St<T>::is_bf16) {
        const u16x4 u = *reinterpret_cast<const u16x4*>(p);
        v = make_float4(bf2f(u[0]), bf2f(u[1]), bf2f(u[2]), bf2f(u[3]));
      } else {
        v = *reinterpret_cast<const float4*>(p);
      }
    }
    *reinterpret_cast<float4*>(lds + r * ls + c4) = v;
  }
}

__device__ __forceinline__ float red16_sum(float x) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}
__device__ __forceinline__ float red16_max(float x) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

// s[i][j] = sum_d A[4 rg + i][d] * B[cg + 16 j][d] (A: BQ rows, B: BK rows, both fp32 in LDS).
// The 16 lanes of a row group read B rows one row stride apart (132 floats = 4 banks): the
// two-pass minimum for 16-byte reads
template <int HD>
__device__ __forceinline__ void tile_dot(float (&s)[4][2], const float* A, const float* B, int ls, int rg, int cg) {
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i][0] = s[i][1] = 0.f;
#pragma unroll 4
  for (int d = 0; d < HD; d += 4) {
    float4 av[4], bv[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const float4*>(A + (4 * rg + i) * ls + d);
#pragma unroll
    for (int j = 0; j < 2; ++j) bv[j] = *reinterpret_cast<const float4*>(B + (cg + 16 * j) * ls + d);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        s[i][j] += av[i].x * bv[j].x + av[i].y * bv[j].y + av[i].z * bv[j].z + av[i].w * bv[j].w;
  }
}

// The forward's score of query row i (index in the chunk) and key `col` of a block starting at
// key j0 of field f: rounding, scale, slot bias, validity (field length, causal own field).
template <typename T>
__device__ __forceinline__ float score_of(const b3_attn_bwd_args& a, float dot, const KField& f, int j0, int col,
                                          int i, float scale) {
  const int j = j0 + col;
  if (j >= f.len) return -INFINITY;
  if (f.kind == 3 && j > i) return -INFINITY;
  float x = a.score_round ? St<T>::rnd(dot) : dot;
  x = mul_rn(x, scale);
  if (f.kind == 1) x = add_rn(x, f.bias[j]);
  return x;
}

template <int HD>
struct DqSmem {
  float q[BQ][HD + 4];
  float dout[BQ][HD + 4];
  float k[BK][HD + 4];
  float v[BK][HD + 4];
  float ds[BQ][BK + 4];
};

template <typename T, int HD>
__global__ void __launch_bounds__(NT) attn_bwd_dq_kernel(b3_attn_bwd_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  DqSmem<HD>& sm = *reinterpret_cast<DqSmem<HD>*>(smem_raw);
  constexpr int LS = HD + 4, DPT = HD / 16;
  const int tid = threadIdx.x, rg = tid >> 4, cg = tid & 15;
  const int qb = blockIdx.x, b = blockIdx.y / a.H, h = blockIdx.y % a.H, c = blockIdx.z;
  const int G = a.H / a.HKV, hkv = h / G;
  const int tc = chunk_len(a, c), q0 = qb * BQ;
  if (q0 >= tc) return;
  const int nq = min(BQ, tc - q0);
  const float scale = 1.0f / sqrtf((float)HD);
  const long long row0 = ((long long)b * a.H + h) * a.T + (long long)c * a.C + q0;   // (b, h, t) row index
  stage_rows<T, HD>(&sm.q[0][0], LS, reinterpret_cast<const T*>(a.q_rope) + (long long)b * a.q_sb +
                                         (long long)h * a.q_sh + ((long long)c * a.C + q0) * HD,
                    HD, BQ, nq, tid);
  stage_rows<float, HD>(&sm.dout[0][0], LS, reinterpret_cast<const float*>(a.dy) + (long long)b * a.dy_sb + ((long long)c * a.C + q0) * a.dy_st +
                                                (long long)h * HD,
                        a.dy_st, BQ, nq, tid);
  float drow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) drow[i] = 4 * rg + i < nq ? a.d_rows[row0 + 4 * rg + i] : 0.f;
  const int n_fields = __popc(field_mask(a, c));

  // pass 1: log-sum-exp of every row over all fields (unless the forward kept it)
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m[i] = -INFINITY; l[i] = 0.f; }
  for (int fi = 0; fi < (a.lse_ready ? 0 : n_fields); ++fi) {
    const KField f = chunk_field<T>(a, b, hkv, c, fi);
    for (int j0 = 0; j0 < f.len; j0 += BK) {
      if (f.kind == 3 && j0 > q0 + nq - 1) break;
      __syncthreads();
      stage_rows<T, HD>(&sm.k[0][0], LS, reinterpret_cast<const T*>(f.k) + (long long)j0 * HD, HD, BK, f.len - j0,
                        tid);
      __syncthreads();
      float s[4][2];
      tile_dot<HD>(s, &sm.q[0][0], &sm.k[0][0], LS, rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x0 = score_of<T>(a, s[i][0], f, j0, cg, q0 + 4 * rg + i, scale);
        const float x1 = score_of<T>(a, s[i][1], f, j0, cg + 16, q0 + 4 * rg + i, scale);
        const float bm = red16_max(fmaxf(x0, x1));
        const float mn = fmaxf(m[i], bm);
        if (mn == -INFINITY) continue;
        const float e = (x0 == -INFINITY ? 0.f : expf(x0 - mn)) + (x1 == -INFINITY ? 0.f : expf(x1 - mn));
        l[i] = l[i] * (m[i] == -INFINITY ? 0.f : expf(m[i] - mn)) + red16_sum(e);
        m[i] = mn;
      }
    }
  }
  float lse[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (a.lse_ready) {
      lse[i] = 4 * rg + i < nq ? a.lse[row0 + 4 * rg + i] : 0.f;
    } else {
      lse[i] = m[i] + logf(l[i]);
      if (cg == 0 && 4 * rg + i < nq) a.lse[row0 + 4 * rg + i] = lse[i];
    }
  }

  // pass 2: dS block by block, dQ += dS . K, slot-bias gradient
  float dq[4][DPT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < DPT; ++e) dq[i][e] = 0.f;
  const long long bias_row = (((long long)(c - 2) * a.B * a.H + (long long)b * a.H + h) * a.n_qtiles + qb) * a.S;
  for (int fi = 0; fi < n_fields; ++fi) {
    const KField f = chunk_field<T>(a, b, hkv, c, fi);
    for (int j0 = 0; j0 < f.len; j0 += BK) {
      if (f.kind == 3 && j0 > q0 + nq - 1) break;
      __syncthreads();
      stage_rows<T, HD>(&sm.k[0][0], LS, reinterpret_cast<const T*>(f.k) + (long long)j0 * HD, HD, BK, f.len - j0,
                        tid);
      stage_rows<T, HD>(&sm.v[0][0], LS, reinterpret_cast<const T*>(f.v) + (long long)j0 * HD, HD, BK, f.len - j0,
                        tid);
      __syncthreads();
      float s[4][2], dp[4][2];
      tile_dot<HD>(s, &sm.q[0][0], &sm.k[0][0], LS, rg, cg);
      tile_dot<HD>(dp, &sm.dout[0][0], &sm.v[0][0], LS, rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float x = score_of<T>(a, s[i][j], f, j0, cg + 16 * j, q0 + 4 * rg + i, scale);
          const bool live = 4 * rg + i < nq && x != -INFINITY;
          const float p = live ? expf(x - lse[i]) : 0.f;
          sm.ds[4 * rg + i][cg + 16 * j] = live ? p * (dp[i][j] - drow[i]) : 0.f;
        }
      __syncthreads();
      if (f.kind == 1 && tid < BK && j0 + tid < f.len) {
        float cs = 0.f;
        for (int r = 0; r < nq; ++r) cs += sm.ds[r][tid];
        a.d_bias[bias_row + j0 + tid] = cs;
      }
      // dq[i][e] += sum_j ds[4 rg + i][j] * k[j][DPT cg + e]
#pragma unroll 2
      for (int j = 0; j < BK; j += 4) {
        float4 dsv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) dsv[i] = *reinterpret_cast<const float4*>(&sm.ds[4 * rg + i][j]);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float kv[DPT];
#pragma unroll
          for (int e = 0; e < DPT; e += 4) {
            const float4 t = *reinterpret_cast<const float4*>(&sm.k[j + jj][DPT * cg + e]);
            kv[e] = t.x; kv[e + 1] = t.y; kv[e + 2] = t.z; kv[e + 3] = t.w;
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float w = jj == 0 ? dsv[i].x : jj == 1 ? dsv[i].y : jj == 2 ? dsv[i].z : dsv[i].w;
#pragma unroll
            for (int e = 0; e < DPT; ++e) dq[i][e] += w * kv[e];
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (4 * rg + i >= nq) continue;
    float* o = static_cast<float*>(a.d_q_rope) + (row0 + 4 * rg + i) * HD + DPT * cg;
#pragma unroll
    for (int e = 0; e < DPT; e += 4)
      *reinterpret_cast<float4*>(o + e) =
          make_float4(dq[i][e] * scale, dq[i][e + 1] * scale, dq[i][e + 2] * scale, dq[i][e + 3] * scale);
  }
}

template <int HD>
struct DkvSmem {
  float q[BQ][HD + 4];
  float dout[BQ][HD + 4];
  float k[BK][HD + 4];
  float v[BK][HD + 4];
  float pt[BK][BQ + 4];    // P transposed: [key][row]
  float dst[BK][BQ + 4];   // dS transposed
  float lse[BQ];
  float drow[BQ];
};

template <typename T, int HD>
__global__ void __launch_bounds__(NT) attn_bwd_dkv_kernel(b3_attn_bwd_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  DkvSmem<HD>& sm = *reinterpret_cast<DkvSmem<HD>*>(smem_raw);
  constexpr int LS = HD + 4, DPT = HD / 16;
  const int tid = threadIdx.x, rg = tid >> 4, cg = tid & 15;
  const int bh = blockIdx.y, b = bh / a.HKV, hkv = bh % a.HKV, c = blockIdx.z;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c);
  const float scale = 1.0f / sqrtf((float)HD);
  // this workgroup's block: the blockIdx.x-th 32-key block of the chunk's fields in order
  const int n_fields = __popc(field_mask(a, c));
  int fi = 0, j0 = blockIdx.x * BK;
  KField f = chunk_field<T>(a, b, hkv, c, 0);
  while (j0 >= f.len) {
    j0 -= (f.len + BK - 1) / BK * BK;
    if (++fi >= n_fields) return;
    f = chunk_field<T>(a, b, hkv, c, fi);
  }
  const int nk = min(BK, f.len - j0);
  stage_rows<T, HD>(&sm.k[0][0], LS, reinterpret_cast<const T*>(f.k) + (long long)j0 * HD, HD, BK, nk, tid);
  stage_rows<T, HD>(&sm.v[0][0], LS, reinterpret_cast<const T*>(f.v) + (long long)j0 * HD, HD, BK, nk, tid);
  // accumulators: keys jg + 16 jj (rows of pt / dst one row stride apart across the lanes),
  // columns DPT dg + e
  const int jg = tid >> 4, dg = tid & 15;
  float dk[2][DPT], dv[2][DPT];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int e = 0; e < DPT; ++e) dk[jj][e] = dv[jj][e] = 0.f;
  for (int g = 0; g < G; ++g) {
    const int h = hkv * G + g;
    for (int q0 = 0; q0 < tc; q0 += BQ) {
      const int nq = min(BQ, tc - q0);
      if (f.kind == 3 && j0 > q0 + nq - 1) continue;   // every row of the tile precedes the keys
      const long long row0 = ((long long)b * a.H + h) * a.T + (long long)c * a.C + q0;
      __syncthreads();
      stage_rows<T, HD>(&sm.q[0][0], LS, reinterpret_cast<const T*>(a.q_rope) + (long long)b * a.q_sb +
                                             (long long)h * a.q_sh + ((long long)c * a.C + q0) * HD,
                        HD, BQ, nq, tid);
      stage_rows<float, HD>(&sm.dout[0][0], LS,
                            reinterpret_cast<const float*>(a.dy) + (long long)b * a.dy_sb + ((long long)c * a.C + q0) * a.dy_st + (long long)h * HD,
                            a.dy_st, BQ, nq, tid);
      if (tid < BQ) {
        sm.lse[tid] = tid < nq ? a.lse[row0 + tid] : INFINITY;
        sm.drow[tid] = tid < nq ? a.d_rows[row0 + tid] : 0.f;
      }
      __syncthreads();
      float s[4][2], dp[4][2];
      tile_dot<HD>(s, &sm.q[0][0], &sm.k[0][0], LS, rg, cg);
      tile_dot<HD>(dp, &sm.dout[0][0], &sm.v[0][0], LS, rg, cg);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int r = 4 * rg + i;
          const float x = score_of<T>(a, s[i][j], f, j0, cg + 16 * j, q0 + r, scale);
          const bool live = r < nq && x != -INFINITY;
          const float p = live ? expf(x - sm.lse[r]) : 0.f;
          sm.pt[cg + 16 * j][r] = p;
          sm.dst[cg + 16 * j][r] = live ? p * (dp[i][j] - sm.drow[r]) : 0.f;
        }
      __syncthreads();
      // dv[jj][e] += sum_r pt[jg + 16 jj][r] * dout[r][DPT dg + e]; dk likewise with dst and q
#pragma unroll 2
      for (int r = 0; r < BQ; r += 4) {
        float4 pv[2], dsv[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          pv[jj] = *reinterpret_cast<const float4*>(&sm.pt[jg + 16 * jj][r]);
          dsv[jj] = *reinterpret_cast<const float4*>(&sm.dst[jg + 16 * jj][r]);
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          float ov[DPT], qv[DPT];
#pragma unroll
          for (int e = 0; e < DPT; e += 4) {
            const float4 to = *reinterpret_cast<const float4*>(&sm.dout[r + rr][DPT * dg + e]);
            const float4 tq = *reinterpret_cast<const float4*>(&sm.q[r + rr][DPT * dg + e]);
            ov[e] = to.x; ov[e + 1] = to.y; ov[e + 2] = to.z; ov[e + 3] = to.w;
            qv[e] = tq.x; qv[e + 1] = tq.y; qv[e + 2] = tq.z; qv[e + 3] = tq.w;
          }
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const float wp = rr == 0 ? pv[jj].x : rr == 1 ? pv[jj].y : rr == 2 ? pv[jj].z : pv[jj].w;
            const float ws = rr == 0 ? dsv[jj].x : rr == 1 ? dsv[jj].y : rr == 2 ? dsv[jj].z : dsv[jj].w;
#pragma unroll
            for (int e = 0; e < DPT; ++e) {
              dv[jj][e] += wp * ov[e];
              dk[jj][e] += ws * qv[e];
            }
          }
        }
      }
    }
  }
  // destination rows of this block's keys
  float *ok = nullptr, *ov = nullptr;
  const long long HDl = HD;
  if (f.kind == 0) {
    const long long o = (((long long)c * a.B * a.HKV + bh) * a.n_sinks + j0) * HDl;
    ok = a.d_sink_k + o;
    ov = a.d_sink_v + o;
  } else if (f.kind == 1) {
    const long long o = (((long long)(c - 2) * a.B * a.HKV + bh) * a.S + j0) * HDl;
    ok = a.d_slot_k + o;
    ov = a.d_slot_v + o;
  } else {
    const long long o = ((long long)bh * a.T + (long long)(f.kind == 2 ? c - 1 : c) * a.C + j0) * HDl;
    ok = static_cast<float*>(f.kind == 2 ? a.d_k_next : a.d_k_own) + o;
    ov = static_cast<float*>(f.kind == 2 ? a.d_v_next : a.d_v_own) + o;
  }
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int j = jg + 16 * jj;
    if (j >= nk) continue;
#pragma unroll
    for (int e = 0; e < DPT; e += 4) {
      *reinterpret_cast<float4*>(ok + j * HDl + DPT * dg + e) =
          make_float4(dk[jj][e] * scale, dk[jj][e + 1] * scale, dk[jj][e + 2] * scale, dk[jj][e + 3] * scale);
      *reinterpret_cast<float4*>(ov + j * HDl + DPT * dg + e) =
          make_float4(dv[jj][e], dv[jj][e + 1], dv[jj][e + 2], dv[jj][e + 3]);
    }
  }
}

// ---------------------------------------------------------------- bf16 storage: MFMA kernels
//
// The same gradients for bf16 storage on v_mfma_f32_32x32x16_bf16 with fp32 accumulation, one
// wavefront per workgroup.  The bf16 operands are the stored q, k, v (exact) and dO, P, dS
// rounded to bf16 where they enter a product, as the reference's autocast backward rounds them.
// Layouts follow the forward: a 32x32 product tile holds, in lane l, column l % 32 and rows
// d_row(l, r); the A operand row l % 32 and the B operand column l % 32 carry the K elements
// 8 * (l / 32) .. + 7.  A product whose K dimension is the rows of an earlier accumulator (dQ^T =
// K^T dS^T, dK^T = Q^T dS, dV^T = dO^T P) takes that accumulator as its B operand in the
// accumulator's own row order and reads the A operand with ds_read_b64_tr_b16 from a row-major
// tile in LDS whose 16-byte pieces p of row r sit at p ^ (r % (HD/8)).
constexpr float L2E = 1.4426950408889634f;

// accumulator values as the B operand of K chunk kc (rows 8 kc .. 8 kc + 7 of the 16), bf16
__device__ __forceinline__ u16x8 acc_operand(const f32x16& v, int kc) {
  u32x4v b;
#pragma unroll
  for (int e = 0; e < 4; ++e) b[e] = pack_bf2(v[8 * kc + 2 * e], v[8 * kc + 2 * e + 1]);
  return __builtin_bit_cast(u16x8, b);
}

// 8 fp32 values as bf16 (the dO rows)
__device__ __forceinline__ u16x8 f32x8_to_bf(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  const u32x4v r = {pack_bf2(a.x, a.y), pack_bf2(a.z, a.w), pack_bf2(b.x, b.y), pack_bf2(b.z, b.w)};
  return __builtin_bit_cast(u16x8, r);
}


// 16-byte piece p of row r of a [32][HD] tile whose pieces sit at p ^ (r % (HD/8))
template <int HD>
__device__ __forceinline__ u16x8 row_piece16(const uint16_t* t, int r, int p) {
  return *reinterpret_cast<const u16x8*>(&t[r * HD + 8 * (p ^ (r % (HD / 8)))]);
}

// Scores of key block j0 of field f against the lane's query qi in log2 units (rows keys j0 +
// d_row(lane, r), the forward's rounding, scale and slot bias), -inf where the key is past the
// field or after the query in the own chunk.  q0: the first query of the tile.
__device__ __forceinline__ void block_scores(const b3_attn_bwd_args& a, f32x16& st, const KField& f, int j0, int qi,
                                             int q0, float sl, int lane) {
  if (a.score_round) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const uint32_t u = pack_bf2(st[r], st[r + 1]);
      st[r] = bf_lo(u);
      st[r + 1] = bf_hi(u);
    }
  }
  if (f.kind == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] = fmaf(st[r], sl, f.bias[min(j0 + d_row(lane, r), f.len - 1)] * L2E);
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] *= sl;
  }
  if (j0 + 32 > f.len || (f.kind == 3 && j0 + 31 > q0)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = j0 + d_row(lane, r);
      if (j >= f.len || (f.kind == 3 && j > qi)) st[r] = -INFINITY;
    }
  }
}

template <int HD>
struct DqMfmaSmem {
  alignas(16) uint16_t k[32 * HD];   // the key block, row-major, swizzled pieces
};

// dQ for one 32-query tile of one query head: lane l owns query l % 32 of the tile.
template <int HD>
__global__ void __launch_bounds__(64) attn_bwd_dq_mfma_kernel(b3_attn_bwd_args a) {
  __shared__ DqMfmaSmem<HD> sm;
  constexpr int KS = HD / 16, NDB = HD / 32, NP = HD / 8;
  const int lane = threadIdx.x, n = lane & 31, h = lane >> 5;
  // XCD-aware order: the query tiles and heads of one (kv head, chunk) read the same key and
  // value blocks
  const GridPos gp = xcd_grid_pos();
  const int qt = gp.x, b = gp.y / a.H, hq = gp.y % a.H, c = gp.z;
  const int G = a.H / a.HKV, hkv = hq / G;
  const int tc = chunk_len(a, c), q0 = qt * 32;
  if (q0 >= tc) return;
  const int nq = min(32, tc - q0);
  const int qi = q0 + n;                      // this lane's query, index in the chunk
  const bool qok = qi < tc;
  const long long t = (long long)c * a.C + qi;
  const long long row = ((long long)b * a.H + hq) * a.T + t;
  const float sl = L2E / sqrtf((float)HD);
  // B operands: the lane's query row and dO row, K elements 16 ks + 8 h ..
  u16x8 qf[KS], of[KS];
  {
    const uint16_t* qr = reinterpret_cast<const uint16_t*>(a.q_rope) + (long long)b * a.q_sb + (long long)hq * a.q_sh +
                         min(t, (long long)c * a.C + tc - 1) * HD;
    const uint16_t* dr = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb +
                         min(t, (long long)c * a.C + tc - 1) * a.dy_st + (long long)hq * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = *reinterpret_cast<const u16x8*>(qr + 16 * ks + 8 * h);
      of[ks] = *reinterpret_cast<const u16x8*>(dr + 16 * ks + 8 * h);
      if (!qok) {
        qf[ks] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        of[ks] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  }
  const float drow = qok ? a.d_rows[row] : 0.f;
  const int n_fields = __popc(field_mask(a, c));
  const TrLanes<HD> TL(lane);
  // A operand of K rows: lane row = key l % 32 of the block (rows past the field repeat its last)
  auto load_rows = [&](const KField& f, int j0, bool v_too, u16x8* ka, u16x8* va) {
    const int kr = min(j0 + n, f.len - 1);
    const uint16_t* kp = reinterpret_cast<const uint16_t*>(f.k) + (long long)kr * HD;
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(f.v) + (long long)kr * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      ka[ks] = *reinterpret_cast<const u16x8*>(kp + 16 * ks + 8 * h);
      if (v_too) va[ks] = *reinterpret_cast<const u16x8*>(vp + 16 * ks + 8 * h);
    }
  };
  // pass 1: log-sum-exp (log2 units) of the lane's query over all fields (unless the forward
  // kept it)
  float m_run = -INFINITY, l_run = 0.f;
  for (int fi = 0; fi < (a.lse_ready ? 0 : n_fields); ++fi) {
    const KField f = chunk_field<uint16_t>(a, b, hkv, c, fi);
    for (int j0 = 0; j0 < f.len; j0 += 32) {
      if (f.kind == 3 && j0 > q0 + nq - 1) break;
      u16x8 ka[KS], va[KS];
      load_rows(f, j0, false, ka, va);
      f32x16 st = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) mma_bf16(st, ka[ks], qf[ks]);
      block_scores(a, st, f, j0, qi, q0, sl, lane);
      float bm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) bm = fmaxf(bm, st[r]);
      bm = pair_max32(bm);
      const float mn = fmaxf(m_run, bm);
      if (mn == -INFINITY) continue;
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) ps += __builtin_amdgcn_exp2f(st[r] - mn);
      ps = pair_sum32(ps);
      l_run = l_run * __builtin_amdgcn_exp2f(m_run - mn) + ps;
      m_run = mn;
    }
  }
  float lse2;
  if (a.lse_ready) {
    lse2 = qok ? a.lse[row] * L2E : 0.f;
  } else {
    lse2 = m_run + log2f(l_run);
    if (qok && h == 0) a.lse[row] = lse2 / L2E;
  }
  // pass 2: dS block by block; dQ^T += K^T dS^T; the slot bias gradient
  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = zero16();
  const long long bias_row = (((long long)(c - 2) * a.B * a.H + (long long)b * a.H + hq) * a.n_qtiles + qt) * a.S;
  for (int fi = 0; fi < n_fields; ++fi) {
    const KField f = chunk_field<uint16_t>(a, b, hkv, c, fi);
    for (int j0 = 0; j0 < f.len; j0 += 32) {
      if (f.kind == 3 && j0 > q0 + nq - 1) break;
      u16x8 ka[KS], va[KS];
      load_rows(f, j0, true, ka, va);
      // the key block into LDS for the transposed reads (piece 2 ks + h of row n)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        *reinterpret_cast<u16x8*>(&sm.k[n * HD + 8 * ((2 * ks + h) ^ (n % NP))]) = ka[ks];
      f32x16 st = zero16(), dpt = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        mma_bf16(st, ka[ks], qf[ks]);
        mma_bf16(dpt, va[ks], of[ks]);
      }
      block_scores(a, st, f, j0, qi, q0, sl, lane);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = qok ? __builtin_amdgcn_exp2f(st[r] - lse2) : 0.f;
        st[r] = p * (dpt[r] - drow);          // dS^T
      }
      if (f.kind == 1) {
        // column sums over the tile's queries: the lanes of each half
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = st[r];
#pragma unroll
          for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
          const int j = j0 + d_row(lane, r);
          if (n == 0 && j < f.len) a.d_bias[bias_row + j] = v;
        }
      }
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u16x8 bs = acc_operand(st, kc);
#pragma unroll
        for (int db = 0; db < NDB; ++db) mma_bf16(dq[db], tr_operand<HD>(sm.k, TL, db, kc), bs);
      }
    }
  }
  if (!qok) return;
  const float scale = 1.0f / sqrtf((float)HD);
  uint16_t* o = static_cast<uint16_t*>(a.d_q_rope) + row * HD;   // bf16, the storage dtype
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<uint2*>(o + 32 * db + 8 * g + 4 * h) =
          make_uint2(pack_bf2(dq[db][4 * g] * scale, dq[db][4 * g + 1] * scale),
                     pack_bf2(dq[db][4 * g + 2] * scale, dq[db][4 * g + 3] * scale));
}

template <int HD>
struct DkvMfmaSmem {
  alignas(16) uint16_t q[32 * HD];    // the query tile, row-major, swizzled pieces
  alignas(16) uint16_t o[32 * HD];    // its dO rows in bf16
  float lse2[32], drow[32];
};

// dK, dV for one 32-key block of one field: lane l owns key l % 32; all query rows of the
// chunk's G heads in 32-row tiles.
template <int HD>
__global__ void __launch_bounds__(64) attn_bwd_dkv_mfma_kernel(b3_attn_bwd_args a) {
  __shared__ DkvMfmaSmem<HD> sm;
  constexpr int KS = HD / 16, NDB = HD / 32, NP = HD / 8;
  const int lane = threadIdx.x, n = lane & 31, h = lane >> 5;
  // XCD-aware order: the key blocks of one (bh, chunk) read the same query and dO rows
  const GridPos gp = xcd_grid_pos();
  const int bh = gp.y, b = bh / a.HKV, hkv = bh % a.HKV, c = gp.z;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c);
  const float sl = L2E / sqrtf((float)HD);
  const int n_fields = __popc(field_mask(a, c));
  int fi = 0, j0 = gp.x * 32;
  KField f = chunk_field<uint16_t>(a, b, hkv, c, 0);
  while (j0 >= f.len) {
    j0 -= (f.len + 31) / 32 * 32;
    if (++fi >= n_fields) return;
    f = chunk_field<uint16_t>(a, b, hkv, c, fi);
  }
  const int nk = min(32, f.len - j0);
  const int j = j0 + n;                       // this lane's key
  const TrLanes<HD> TL(lane);
  const bool kval = j < f.len;
  const float kb2 = f.kind == 1 ? f.bias[min(j, f.len - 1)] * L2E : 0.f;
  // B operands: the lane's key and value rows
  u16x8 kf[KS], vf[KS];
  {
    const int kr = min(j, f.len - 1);
    const uint16_t* kp = reinterpret_cast<const uint16_t*>(f.k) + (long long)kr * HD;
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(f.v) + (long long)kr * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[ks] = *reinterpret_cast<const u16x8*>(kp + 16 * ks + 8 * h);
      vf[ks] = *reinterpret_cast<const u16x8*>(vp + 16 * ks + 8 * h);
    }
  }
  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }
  // the tiles this block needs: all 32-row query tiles of the G heads, for the own chunk's keys
  // only those from the block's first key on (earlier queries precede every key of the block);
  // tile it + 1's rows are loaded into registers while tile it's products run
  const int q_start = f.kind == 3 ? j0 : 0;
  const int nqt = (tc - q_start + 31) / 32, n_it = G * nqt;
  u16x8 nqv[KS], nov[KS];
  float nls = INFINITY, ndr = 0.f;
  auto fetch = [&](int it) {
    const int hq = hkv * G + it / nqt, q0 = q_start + 32 * (it % nqt);
    const bool ok = q0 + n < tc;
    const long long t = (long long)c * a.C + min(q0 + n, tc - 1);
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q_rope) + (long long)b * a.q_sb + (long long)hq * a.q_sh +
                         t * HD;
    const uint16_t* dp = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb + t * a.dy_st +
                         (long long)hq * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      nqv[ks] = ok ? *reinterpret_cast<const u16x8*>(qp + 16 * ks + 8 * h) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      nov[ks] = ok ? *reinterpret_cast<const u16x8*>(dp + 16 * ks + 8 * h) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    if (h == 0) {
      const long long row = ((long long)b * a.H + hq) * a.T + t;
      nls = ok ? a.lse[row] * L2E : INFINITY;
      ndr = ok ? a.d_rows[row] : 0.f;
    }
  };
  auto put = [&]() {   // the fetched tile into LDS (row n, piece 2 ks + h)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int slot = 8 * ((2 * ks + h) ^ (n % NP));
      *reinterpret_cast<u16x8*>(&sm.q[n * HD + slot]) = nqv[ks];
      *reinterpret_cast<u16x8*>(&sm.o[n * HD + slot]) = nov[ks];
    }
    if (h == 0) {
      sm.lse2[n] = nls;
      sm.drow[n] = ndr;
    }
  };
  if (n_it > 0) {
    fetch(0);
    put();
  }
  for (int it = 0; it < n_it; ++it) {
    {
      if (it + 1 < n_it) fetch(it + 1);
      const int q0 = q_start + 32 * (it % nqt);
      // S = Q K^T and dP = dO V^T: rows queries (A operand from the tile rows), columns keys
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int slot = 8 * ((2 * ks + h) ^ (n % NP));
        mma_bf16(s, *reinterpret_cast<const u16x8*>(&sm.q[n * HD + slot]), kf[ks]);
        mma_bf16(dp, *reinterpret_cast<const u16x8*>(&sm.o[n * HD + slot]), vf[ks]);
      }
      if (a.score_round) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const uint32_t u = pack_bf2(s[r], s[r + 1]);
          s[r] = bf_lo(u);
          s[r + 1] = bf_hi(u);
        }
      }
      const bool causal = f.kind == 3 && j0 + 31 > q0;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qr = d_row(lane, r);
        const bool on = kval && !(causal && j > q0 + qr);
        const float p = on ? __builtin_amdgcn_exp2f(fmaf(s[r], sl, kb2) - sm.lse2[qr]) : 0.f;
        s[r] = p;
        dp[r] = p * (dp[r] - sm.drow[qr]);     // dS
      }
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u16x8 bp = acc_operand(s, kc), bs = acc_operand(dp, kc);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          mma_bf16(dv[db], tr_operand<HD>(sm.o, TL, db, kc), bp);
          mma_bf16(dk[db], tr_operand<HD>(sm.q, TL, db, kc), bs);
        }
      }
    }
    if (it + 1 < n_it) put();   // after this tile's LDS reads (one wavefront: LDS in order)
  }
  if (n >= nk) return;
  const float scale = 1.0f / sqrtf((float)HD);
  const long long HDl = HD;
  if (f.kind >= 2) {
    // token rows: bf16, the storage dtype
    const long long o = ((long long)bh * a.T + (long long)(f.kind == 2 ? c - 1 : c) * a.C + j) * HDl;
    uint16_t* ok = static_cast<uint16_t*>(f.kind == 2 ? a.d_k_next : a.d_k_own) + o;
    uint16_t* ov = static_cast<uint16_t*>(f.kind == 2 ? a.d_v_next : a.d_v_own) + o;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * db + 8 * g4 + 4 * h;
        *reinterpret_cast<uint2*>(ok + d0) = make_uint2(pack_bf2(dk[db][4 * g4] * scale, dk[db][4 * g4 + 1] * scale),
                                                        pack_bf2(dk[db][4 * g4 + 2] * scale, dk[db][4 * g4 + 3] * scale));
        *reinterpret_cast<uint2*>(ov + d0) =
            make_uint2(pack_bf2(dv[db][4 * g4], dv[db][4 * g4 + 1]), pack_bf2(dv[db][4 * g4 + 2], dv[db][4 * g4 + 3]));
      }
    return;
  }
  // sinks and slots: fp32 (the chain's backward sums them further)
  float *ok, *ov;
  if (f.kind == 0) {
    const long long o = (((long long)c * a.B * a.HKV + bh) * a.n_sinks + j) * HDl;
    ok = a.d_sink_k + o;
    ov = a.d_sink_v + o;
  } else {
    const long long o = (((long long)(c - 2) * a.B * a.HKV + bh) * a.S + j) * HDl;
    ok = a.d_slot_k + o;
    ov = a.d_slot_v + o;
  }
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = 32 * db + 8 * g4 + 4 * h;
      *reinterpret_cast<float4*>(ok + d0) = make_float4(dk[db][4 * g4] * scale, dk[db][4 * g4 + 1] * scale,
                                                        dk[db][4 * g4 + 2] * scale, dk[db][4 * g4 + 3] * scale);
      *reinterpret_cast<float4*>(ov + d0) =
          make_float4(dv[db][4 * g4], dv[db][4 * g4 + 1], dv[db][4 * g4 + 2], dv[db][4 * g4 + 3]);
    }
}

template <int HD>
struct RdSmem {
  float m[HD][HD + 4];     // M[c][d]
  float qn[RT][HD + 4];    // normalised q_raw rows of the tile
  float du[RT][HD + 4];    // gradient of qn . M
  float part[RT][HD + 4];  // per-row d res_w terms, then reduced
  float inv[RT];           // 1 / max(|q_raw|, 1e-12)
};

// d_rows for every chunk; for chunks with a readout also its gradients.
template <typename T, int HD>
__global__ void __launch_bounds__(NT) readout_bwd_kernel(b3_attn_bwd_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  RdSmem<HD>& sm = *reinterpret_cast<RdSmem<HD>*>(smem_raw);
  constexpr int DPT = HD / 16;
  const int tid = threadIdx.x, r = tid >> 4, dg = tid & 15;   // row of the tile, column group
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV, c = blockIdx.y;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c);
  const int n_rows = G * tc;
  const bool has_m = c >= 2 && c - 2 < a.n_steps && a.m_res != nullptr;
  const float* M = has_m ? a.m_res + (long long)(c - 2) * a.m_step + (long long)bh * HD * HD : nullptr;
  if (has_m) {
    if (a.m_split) {
      // M^T[d][c] stored as bf16 hi then bf16 lo
      const uint16_t* src = reinterpret_cast<const uint16_t*>(M);
      for (int it = tid; it < HD * HD; it += NT) {
        const int d = it / HD, cc = it % HD;
        sm.m[cc][d] = bf2f(src[it]) + bf2f(src[HD * HD + it]);
      }
    } else {
      for (int it = tid; it < HD * HD; it += NT) sm.m[it / HD][it % HD] = M[it];
    }
  }
  const float gam = a.gamma[hkv];
  const float sg = (1.0f - gam) / sqrtf((float)HD);
  float dm[DPT][DPT];   // dM[DPT r' + i][DPT dg + j] with r' = tid >> 4 as the row group of M
#pragma unroll
  for (int i = 0; i < DPT; ++i)
#pragma unroll
    for (int j = 0; j < DPT; ++j) dm[i][j] = 0.f;
  float dres[DPT], dsg = 0.f;
#pragma unroll
  for (int e = 0; e < DPT; ++e) dres[e] = 0.f;
  float wv[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) wv[e] = a.res_w[DPT * dg + e];

  for (int r0 = 0; r0 < n_rows; r0 += RT) {
    const int q = r0 + r;                 // row of the chunk: head g = q / tc, token i = q % tc
    const bool live = q < n_rows;
    const int g = live ? q / tc : 0, i = live ? q % tc : 0;
    const int h = hkv * G + g;
    const long long t = (long long)c * a.C + i;
    const long long row = ((long long)b * a.H + h) * a.T + t;
    // this thread's DPT columns of dy and y
    float dyv[DPT], yv[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) { dyv[e] = 0.f; yv[e] = 0.f; }
    if (live) {
      const float* dyp = reinterpret_cast<const float*>(a.dy) + (long long)b * a.dy_sb + t * a.dy_st + (long long)h * HD + DPT * dg;
      const T* yp = reinterpret_cast<const T*>(a.y) + (long long)b * a.y_sb + t * a.y_st + (long long)h * HD + DPT * dg;
#pragma unroll
      for (int e = 0; e < DPT; ++e) { dyv[e] = dyp[e]; yv[e] = St<T>::ld(yp + e); }
    }
    if (!has_m) {
      float dd = 0.f;
#pragma unroll
      for (int e = 0; e < DPT; ++e) dd += dyv[e] * yv[e];
      dd = red16_sum(dd);
      if (live && dg == 0) a.d_rows[row] = dd;
      continue;
    }
    // q_raw row -> normalised
    float qv[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) qv[e] = 0.f;
    if (live) {
      const T* qp = reinterpret_cast<const T*>(a.q_raw) + (long long)b * a.q_sb + (long long)h * a.q_sh + t * HD +
                    DPT * dg;
#pragma unroll
      for (int e = 0; e < DPT; ++e) qv[e] = St<T>::ld(qp + e);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) ss += qv[e] * qv[e];
    ss = red16_sum(ss);
    const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
    __syncthreads();   // the previous tile's qn / du reads are done
#pragma unroll
    for (int e = 0; e < DPT; ++e) sm.qn[r][DPT * dg + e] = qv[e] * inv;
    if (dg == 0) sm.inv[r] = inv;
    __syncthreads();
    // u = qn . M for this thread's columns
    float u[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) u[e] = 0.f;
    for (int cc = 0; cc < HD; ++cc) {
      const float x = sm.qn[r][cc];
#pragma unroll
      for (int e = 0; e < DPT; e += 4) {
        const float4 mv = *reinterpret_cast<const float4*>(&sm.m[cc][DPT * dg + e]);
        u[e] += x * mv.x; u[e + 1] += x * mv.y; u[e + 2] += x * mv.z; u[e + 3] += x * mv.w;
      }
    }
    float ym[DPT], sq = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) { ym[e] = u[e] * sg; sq += ym[e] * ym[e]; }
    sq = red16_sum(sq);
    const float rr = 1.0f / sqrtf(sq / (float)HD + a.eps);
    const float eta = live ? a.eta[(long long)b * a.e_sb + (long long)h * a.e_sh + t] : 0.f;
    float dd = 0.f, deta = 0.f, gdot = 0.f, gv[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const float yn = ym[e] * rr * wv[e];
      dd += dyv[e] * (yv[e] - eta * yn);
      deta += dyv[e] * yn;
      gv[e] = eta * dyv[e] * wv[e];
      gdot += gv[e] * ym[e];
      dres[e] += eta * dyv[e] * ym[e] * rr;
    }
    dd = red16_sum(dd);
    deta = red16_sum(deta);
    gdot = red16_sum(gdot);
    if (live && dg == 0) {
      a.d_rows[row] = dd;
      a.d_eta[row] = deta;
    }
    float dsg_r = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      const float dym = rr * gv[e] - ym[e] * rr * rr * rr * gdot / (float)HD;
      dsg_r += dym * u[e];
      sm.du[r][DPT * dg + e] = live ? dym * sg : 0.f;
    }
    dsg += red16_sum(dsg_r) * (dg == 0 && live ? 1.f : 0.f);
    __syncthreads();
    // dqn[cc] = sum_d du[d] * M[cc][d] for this thread's columns cc = 16 e + dg (the lanes of a
    // row read M rows one row stride apart: distinct banks)
    float dqn[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) dqn[e] = 0.f;
    for (int d = 0; d < HD; d += 4) {
      const float4 dv4 = *reinterpret_cast<const float4*>(&sm.du[r][d]);
#pragma unroll
      for (int e = 0; e < DPT; ++e) {
        const float4 mv = *reinterpret_cast<const float4*>(&sm.m[16 * e + dg][d]);
        dqn[e] += dv4.x * mv.x + dv4.y * mv.y + dv4.z * mv.z + dv4.w * mv.w;
      }
    }
    float qd = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) qd += sm.qn[r][16 * e + dg] * dqn[e];
    qd = red16_sum(qd);
    if (live) {
      float* o = static_cast<float*>(a.d_q_raw) + row * HD;
#pragma unroll
      for (int e = 0; e < DPT; ++e) o[16 * e + dg] = (dqn[e] - sm.qn[r][16 * e + dg] * qd) * inv;
    }
    // dM[cc][d] += sum over the tile's rows of qn[row][cc] * du[row][d]; this thread: cc in
    // DPT * (tid >> 4) .. and d in DPT * dg ..
    for (int rr2 = 0; rr2 < RT; ++rr2) {
      float qa[DPT], db[DPT];
#pragma unroll
      for (int e = 0; e < DPT; ++e) {
        qa[e] = sm.qn[rr2][DPT * r + e];
        db[e] = sm.du[rr2][DPT * dg + e];
      }
#pragma unroll
      for (int i2 = 0; i2 < DPT; ++i2)
#pragma unroll
        for (int j2 = 0; j2 < DPT; ++j2) dm[i2][j2] += qa[i2] * db[j2];
    }
  }
  if (!has_m) return;
  // rows past n_rows left zeros in qn / du, so they added nothing
  float* dmo = a.d_m + ((long long)(c - 2) * a.B * a.HKV + bh) * HD * HD;
#pragma unroll
  for (int i2 = 0; i2 < DPT; ++i2)
#pragma unroll
    for (int j2 = 0; j2 < DPT; ++j2) dmo[(DPT * r + i2) * HD + DPT * dg + j2] = dm[i2][j2];
  // res_w and gamma partials of this (bh, chunk)
  __syncthreads();
#pragma unroll
  for (int e = 0; e < DPT; ++e) sm.part[r][DPT * dg + e] = dres[e];
  __syncthreads();
  const long long pc = (long long)bh * a.n_chunks + c;
  if (tid < HD) {
    float s = 0.f;
    for (int k = 0; k < RT; ++k) s += sm.part[k][tid];
    a.d_res_w[pc * HD + tid] = s;
  }
  __syncthreads();
  if (dg == 0) sm.inv[r] = dsg;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
    for (int k = 0; k < RT; ++k) s += sm.inv[k];
    a.d_gamma[pc] = -s / sqrtf((float)HD);   // d/dgamma of (1 - gamma) / sqrt(HD)
  }
}

// ---------------------------------------------------------------- readout, bf16 storage: MFMA
//
// The readout's gradients for bf16 storage on MFMA, one workgroup of four wavefronts per (b, kv
// head, chunk), one query row per lane column, 32 rows per wavefront and round:
//   U^T = M^T q_raw^T            (M^T as bf16 hi + lo, q_raw exact: two products, as the forward)
//   u = U / |q_raw|, ym = u (1-gamma)/sqrt(HD), the RMSNorm backward as the fp32 kernel
//   dqn^T = M du^T               (M^T read transposed; hi/lo on both sides: three products)
//   dM += q_raw^T (du / |q_raw|) (bf16 operands from per-wavefront row tiles in LDS; wavefront w
//                                 accumulates its share of the (HD/32)^2 output tiles)
template <int HD>
struct RdMfmaSmem {
  alignas(16) uint16_t mt[2][HD * HD];   // M^T hi, lo: row d, 16-byte piece p at p ^ (d % (HD/8))
  alignas(16) uint16_t qt[4][32 * HD];   // per wavefront: q_raw rows of its tile (same swizzle)
  alignas(16) uint16_t ut[4][32 * HD];   // per wavefront: du / |q_raw| rows, bf16
  float resw[HD];
  float red[4][HD + 1];
};

template <int HD>
__global__ void __launch_bounds__(256) readout_bwd_mfma_kernel(b3_attn_bwd_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  RdMfmaSmem<HD>& sm = *reinterpret_cast<RdMfmaSmem<HD>*>(smem_raw);
  constexpr int KS = HD / 16, NDB = HD / 32, NP = HD / 8, TPW = NDB * NDB / 4;
  static_assert(NDB * NDB % 4 == 0, "dM tiles split over four wavefronts");
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV, c = blockIdx.y;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c);
  const int n_rows = G * tc;
  const bool has_m = c >= 2 && c - 2 < a.n_steps && a.m_res != nullptr;
  if (!has_m) {
    // D = rowsum(dy * y) only: 16 lanes per row, HD / 16 elements each
    constexpr int DPT = HD / 16;
    const int rq = lane >> 4, dg = lane & 15;
    for (int r0 = 4 * w; r0 < n_rows; r0 += 16) {
      const int q = r0 + rq;
      const bool live = q < n_rows;
      const int g = live ? q / tc : 0, i = live ? q % tc : 0;
      const int hq = hkv * G + g;
      const long long t = (long long)c * a.C + i;
      float dd = 0.f;
      if (live) {
        const uint16_t* dyp = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb + t * a.dy_st +
                              (long long)hq * HD + DPT * dg;
        const uint16_t* yp = reinterpret_cast<const uint16_t*>(a.y) + (long long)b * a.y_sb + t * a.y_st +
                             (long long)hq * HD + DPT * dg;
#pragma unroll
        for (int e = 0; e < DPT; ++e) dd += bf2f(dyp[e]) * bf2f(yp[e]);
      }
      dd = red16_sum(dd);
      if (live && dg == 0) a.d_rows[((long long)b * a.H + hq) * a.T + t] = dd;
    }
    return;
  }
  // M^T hi / lo into LDS
  {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(a.m_res + (long long)(c - 2) * a.m_step +
                                                            (long long)bh * HD * HD);
    for (int it = tid; it < 2 * HD * NP; it += 256) {
      const int half = it / (HD * NP), rem = it % (HD * NP), d = rem / NP, pc = rem % NP;
      *reinterpret_cast<u16x8*>(&sm.mt[half][d * HD + 8 * (pc ^ (d % NP))]) =
          *reinterpret_cast<const u16x8*>(src + (long long)half * HD * HD + d * HD + 8 * pc);
    }
    for (int it = tid; it < HD; it += 256) sm.resw[it] = a.res_w[it];
  }
  __syncthreads();
  const float sg = (1.0f - a.gamma[hkv]) / sqrtf((float)HD);
  const TrLanes<HD> TL(lane);
  int dm_off[TPW][4];   // transposed-read offsets of output tile tt: A (rows cf) then B (columns d)
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int id = w * TPW + tt, cb = id / NDB, db = id % NDB;
    dm_off[tt][0] = tr_off<HD>(lane, cb, 0);
    dm_off[tt][1] = tr_off<HD>(lane, cb, 1);
    dm_off[tt][2] = tr_off<HD>(lane, db, 0);
    dm_off[tt][3] = tr_off<HD>(lane, db, 1);
  }
  f32x16 dm[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) dm[tt] = zero16();
  // res_w partials: dres[db] is feature 32 db + d_row(lane, r) with r = 8 (n >> 4 & 1) +
  // 4 (n >> 3 & 1) + 2 (n >> 2 & 1) + (n >> 1 & 1) (the reduce-scatter below leaves it there)
  float dres[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dres[db] = 0.f;
  float dsg = 0.f;
  uint16_t* qt = sm.qt[w];
  uint16_t* ut = sm.ut[w];
  const int n_tiles = (n_rows + 31) / 32;
#pragma unroll 1
  for (int r0 = 0; r0 < n_tiles; r0 += 4) {
    const int q = 32 * (r0 + w) + n;
    const bool live = q < n_rows;
    const int g = live ? q / tc : 0, i = live ? q % tc : 0;
    const int hq = hkv * G + g;
    const long long t = (long long)c * a.C + i;
    const long long row = ((long long)b * a.H + hq) * a.T + t;
    // the lane's q_raw row: B operand (K elements 16 ks + 8 h ..) and row n of the tile
    u16x8 qf[KS];
    {
      const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q_raw) + (long long)b * a.q_sb + (long long)hq * a.q_sh +
                           t * HD;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = live ? *reinterpret_cast<const u16x8*>(qp + 16 * ks + 8 * h) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        *reinterpret_cast<u16x8*>(&qt[n * HD + 8 * ((2 * ks + h) ^ (n % NP))]) = qf[ks];
      }
    }
    const float eta = live ? a.eta[(long long)b * a.e_sb + (long long)hq * a.e_sh + t] : 0.f;
    float qq = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = bf2f(qf[ks][e]);
        qq += x * x;
      }
    qq = pair_sum32(qq);
    const float inv = 1.0f / fmaxf(sqrtf(qq), 1e-12f);
    // U^T: rows d, column = the lane's query
    f32x16 u[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) u[db] = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      // one K step's operands at a time (the scheduler would otherwise hoist every read)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int dr = 32 * db + n, pc = (2 * ks + h) ^ (dr % NP);
        mma_bf16(u[db], *reinterpret_cast<const u16x8*>(&sm.mt[0][dr * HD + 8 * pc]), qf[ks]);
        mma_bf16(u[db], *reinterpret_cast<const u16x8*>(&sm.mt[1][dr * HD + 8 * pc]), qf[ks]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the RMSNorm backward of ym = u * sg at this lane's features d = 32 db + d_row(lane, r)
    const uint16_t* dyp = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb + t * a.dy_st +
                          (long long)hq * HD;
    const uint16_t* yp = reinterpret_cast<const uint16_t*>(a.y) + (long long)b * a.y_sb + t * a.y_st + (long long)hq * HD;
    // u becomes ym = U sg / |q_raw| (sg > 0: gamma <= 0.999)
    const float ks_ = inv * sg;
    float sq = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        u[db][r] *= ks_;
        sq += u[db][r] * u[db][r];
      }
    sq = pair_sum32(sq);
    const float rr = 1.0f / sqrtf(sq / (float)HD + a.eps);
    float dd = 0.f, deta = 0.f, gdot = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      __builtin_amdgcn_sched_barrier(0);   // one block's loads live at a time
      float xr[16];   // res_w terms of the block
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * db + 8 * r4 + 4 * h;
        float4 dy4 = make_float4(0.f, 0.f, 0.f, 0.f);
        uint2 y2 = make_uint2(0u, 0u);
        if (live) {
          const uint2 g2 = *reinterpret_cast<const uint2*>(dyp + d0);
          dy4 = make_float4(bf_lo(g2.x), bf_hi(g2.x), bf_lo(g2.y), bf_hi(g2.y));
          y2 = *reinterpret_cast<const uint2*>(yp + d0);
        }
        const float4 w4 = *reinterpret_cast<const float4*>(&sm.resw[d0]);
        const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
        const float yv[4] = {bf_lo(y2.x), bf_hi(y2.x), bf_lo(y2.y), bf_hi(y2.y)};
        const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * r4 + j;
          const float ym = u[db][r];
          const float yn = ym * rr * wv[j];
          dd += dyv[j] * (yv[j] - eta * yn);
          deta += dyv[j] * yn;
          gdot += eta * dyv[j] * wv[j] * ym;
          xr[r] = eta * dyv[j] * ym * rr;
        }
      }
      // reduce-scatter over the 32 lanes of the half: the step with lane mask m keeps the half
      // of the values selected by (n & m); the last step adds the partner's single value
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int m = 16 >> st, len = 8 >> st;
        const bool up = (n & m) != 0;
#pragma unroll
        for (int j = 0; j < len; ++j) {
          // the empty asm keeps the choice a select of two values (not an indexed array read)
          float lo = xr[j], hi = xr[len + j];
          asm("" : "+v"(lo), "+v"(hi));
          const float keep = up ? hi : lo, send = up ? lo : hi;
          xr[j] = keep + __shfl_xor(send, m, 64);
        }
      }
      dres[db] += xr[0] + __shfl_xor(xr[0], 1, 64);
    }
    dd = pair_sum32(dd);
    deta = pair_sum32(deta);
    gdot = pair_sum32(gdot);
    if (live && h == 0) {
      a.d_rows[row] = dd;
      a.d_eta[row] = deta;
    }
    // du = sg (rr g - ym rr^3 gdot / HD), g = eta dy w (dy read again), in place of u; the gamma
    // partial; du / |q_raw| as bf16 into the wavefront's tile
    float dsg_r = 0.f;
    const float c3 = rr * rr * rr * gdot / (float)HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        if (r4 == 0) __builtin_amdgcn_sched_barrier(0);
        const int d0 = 32 * db + 8 * r4 + 4 * h;
        float4 dy4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) {
          const uint2 g2 = *reinterpret_cast<const uint2*>(dyp + d0);
          dy4 = make_float4(bf_lo(g2.x), bf_hi(g2.x), bf_lo(g2.y), bf_hi(g2.y));
        }
        const float4 w4 = *reinterpret_cast<const float4*>(&sm.resw[d0]);
        const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
        const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * r4 + j;
          const float ym = u[db][r];
          const float dym = rr * (eta * dyv[j] * wv[j]) - ym * c3;
          dsg_r += dym * ym;
          u[db][r] = live ? dym * sg : 0.f;
        }
        const uint2 v = make_uint2(pack_bf2(u[db][4 * r4] * inv, u[db][4 * r4 + 1] * inv),
                                   pack_bf2(u[db][4 * r4 + 2] * inv, u[db][4 * r4 + 3] * inv));
        *reinterpret_cast<uint2*>(&ut[n * HD + 8 * ((4 * db + r4) ^ (n % NP)) + 4 * h]) = v;
      }
    // sum_d dym ym: the gamma partial (times 1/sg) and qn . dqn (qn . M du = u . du)
    const float sdy = pair_sum32(dsg_r);
    if (live && h == 0) dsg += sdy / sg;
    // dqn^T[cf][q] = sum_d M[cf][d] du[q][d]: A = M read transposed out of M^T, K = d in the
    // accumulator's row order, du as bf16 hi + lo; d q_raw = (dqn - qn (qn . dqn)) / |q_raw|,
    // qn = q_raw / |q_raw| (q_raw from the tile), one 32-feature block at a time
    u16x8 bhi[NDB][2], blo[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) acc_operand_split(u[db], kc, bhi[db][kc], blo[db][kc]);
    const float qi2 = sdy * inv;
    uint16_t* o = static_cast<uint16_t*>(a.d_q_raw) + row * HD;   // bf16, the storage dtype
#pragma unroll
    for (int cb = 0; cb < NDB; ++cb) {
      __builtin_amdgcn_sched_barrier(0);
      f32x16 dq = zero16();
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const u16x8 ah = tr_operand<HD>(&sm.mt[0][32 * db * HD], TL, cb, kc);
          const u16x8 al = tr_operand<HD>(&sm.mt[1][32 * db * HD], TL, cb, kc);
          mma_bf16(dq, ah, bhi[db][kc]);
          mma_bf16(dq, al, bhi[db][kc]);
          mma_bf16(dq, ah, blo[db][kc]);
        }
      if (live) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const uint2 q2 = *reinterpret_cast<const uint2*>(&qt[n * HD + 8 * ((4 * cb + r4) ^ (n % NP)) + 4 * h]);
          float4 v;
          v.x = (dq[4 * r4] - bf_lo(q2.x) * qi2) * inv;
          v.y = (dq[4 * r4 + 1] - bf_hi(q2.x) * qi2) * inv;
          v.z = (dq[4 * r4 + 2] - bf_lo(q2.y) * qi2) * inv;
          v.w = (dq[4 * r4 + 3] - bf_hi(q2.y) * qi2) * inv;
          *reinterpret_cast<uint2*>(o + 32 * cb + 8 * r4 + 4 * h) = make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
        }
      }
    }
    __syncthreads();   // every wavefront's q_raw and du tiles are in LDS
    // dM[cf][d] += sum_q q_raw[q][cf] du'[q][d] over the round's tiles; output tile tt of this
    // wavefront is (cb, db) = ((w TPW + tt) / NDB, (w TPW + tt) % NDB)
    for (int ws = 0; ws < 4; ++ws) {
      if (32 * (r0 + ws) >= n_rows) break;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
          const uint16_t* pq = sm.qt[ws] + 16 * kc * HD;
          const uint16_t* pu = sm.ut[ws] + 16 * kc * HD;
          const s16x4 a0 = lds_tr16(pq + dm_off[tt][0]), a1 = lds_tr16(pq + dm_off[tt][1]);
          const s16x4 b0 = lds_tr16(pu + dm_off[tt][2]), b1 = lds_tr16(pu + dm_off[tt][3]);
          u16x8 av, bv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            av[e] = (uint16_t)a0[e];
            av[4 + e] = (uint16_t)a1[e];
            bv[e] = (uint16_t)b0[e];
            bv[4 + e] = (uint16_t)b1[e];
          }
          mma_bf16(dm[tt], av, bv);
        }
    }
    __syncthreads();   // the tiles are read before the next round writes them
  }
  // dM out: tile (cb, db) holds rows cf = 32 cb + d_row(lane, r), column d = 32 db + n
  float* dmo = a.d_m + ((long long)(c - 2) * a.B * a.HKV + bh) * HD * HD;
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int id = w * TPW + tt, cb = id / NDB, db = id % NDB;
#pragma unroll
    for (int r = 0; r < 16; ++r) dmo[(32 * cb + d_row(lane, r)) * HD + 32 * db + n] = dm[tt][r];
  }
  // res_w and gamma partials over the wavefronts (lanes n and n ^ 1 hold the same sums)
  if ((n & 1) == 0) {
    const int r = 8 * ((n >> 4) & 1) + 4 * ((n >> 3) & 1) + 2 * ((n >> 2) & 1) + ((n >> 1) & 1);
#pragma unroll
    for (int db = 0; db < NDB; ++db) sm.red[w][32 * db + d_row(lane, r)] = dres[db];
  }
  {
    float v = dsg;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) sm.red[w][HD] = v;
  }
  __syncthreads();
  const long long pc = (long long)bh * a.n_chunks + c;
  if (tid < HD) a.d_res_w[pc * HD + tid] = sm.red[0][tid] + sm.red[1][tid] + sm.red[2][tid] + sm.red[3][tid];
  if (tid == 0)
    a.d_gamma[pc] = -(sm.red[0][HD] + sm.red[1][HD] + sm.red[2][HD] + sm.red[3][HD]) / sqrtf((float)HD);
}

template <typename T, int HD>
static int launch(const b3_attn_bwd_args& a, hipStream_t st) {
  const int n_chunks = a.n_chunks;
  const int BH = a.B * a.HKV;
  hipError_t e = hipSuccess;
  if (a.part != 2) {
    if constexpr (St<T>::is_bf16)
      hipLaunchKernelGGL((readout_bwd_mfma_kernel<HD>), dim3(BH, n_chunks), dim3(256), sizeof(RdMfmaSmem<HD>), st, a);
    else
      hipLaunchKernelGGL((readout_bwd_kernel<T, HD>), dim3(BH, n_chunks), dim3(NT), sizeof(RdSmem<HD>), st, a);
    e = hipGetLastError();
    if (e != hipSuccess || a.part == 1) return (int)e;
  }
  const int max_blocks = 1 + (a.S + 31) / 32 + 2 * ((a.C + 31) / 32);
  if constexpr (St<T>::is_bf16) {
    hipLaunchKernelGGL((attn_bwd_dq_mfma_kernel<HD>), dim3((a.C + 31) / 32, a.B * a.H, n_chunks), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((attn_bwd_dkv_mfma_kernel<HD>), dim3(max_blocks, BH, n_chunks), dim3(64), 0, st, a);
    return (int)hipGetLastError();
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, HD>), dim3((a.C + BQ - 1) / BQ, a.B * a.H, n_chunks), dim3(NT),
                       sizeof(DqSmem<HD>), st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<T, HD>), dim3(max_blocks, BH, n_chunks), dim3(NT), sizeof(DkvSmem<HD>),
                       st, a);
    return (int)hipGetLastError();
  }
}

template <typename T, int HD>
static int set_smem() {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dq_kernel<T, HD>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(DqSmem<HD>));
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dkv_kernel<T, HD>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(DkvSmem<HD>));
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&readout_bwd_kernel<T, HD>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(RdSmem<HD>));
  if constexpr (St<T>::is_bf16)
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(&readout_bwd_mfma_kernel<HD>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(RdMfmaSmem<HD>));
  return (int)e;
}

}  // namespace bwd
}  // namespace b3

extern "C" int bolt3_attn_bwd(const b3_attn_bwd_args* a, void* stream) {
  if (!a || a->B <= 0 || a->T <= 0 || a->HKV <= 0 || a->H % a->HKV != 0 || a->C <= 0 || a->S <= 0) return B3_ERR_ARG;
  if (a->HD != 64 && a->HD != 128) return B3_ERR_UNSUPPORTED;
  if (a->dtype != B3_F32 && a->dtype != B3_BF16) return B3_ERR_UNSUPPORTED;
  const int n_chunks = (a->T + a->C - 1) / a->C;
  if (a->n_chunks != n_chunks || a->n_qtiles != (a->C + 31) / 32) return B3_ERR_ARG;
  if (a->n_steps < 0 || a->n_steps > (n_chunks > 2 ? n_chunks - 2 : 0) || a->n_sinks < 0 || a->n_sinks > a->C)
    return B3_ERR_ARG;
  if (!a->q_rope || !a->q_raw || !a->win_k || !a->win_v || !a->eta || !a->gamma || !a->res_w || !a->y || !a->dy ||
      !a->d_rows || !a->lse || !a->d_q_rope || !a->d_q_raw || !a->d_eta || !a->d_res_w || !a->d_gamma ||
      !a->d_k_own || !a->d_v_own || !a->d_k_next || !a->d_v_next)
    return B3_ERR_ARG;
  if (a->n_steps > 0 && (!a->slot_k || !a->slot_v || !a->slot_bias || !a->m_res || !a->d_m || !a->d_bias ||
                         !a->d_slot_k || !a->d_slot_v || (a->n_sinks > 0 && (!a->d_sink_k || !a->d_sink_v)) ||
                         a->slot_step < (int64_t)a->B * a->HKV * a->S * a->HD))
    return B3_ERR_ARG;
  if (a->m_split && a->dtype != B3_BF16) return B3_ERR_ARG;
  if (a->part < 0 || a->part > 2 || (a->lse_ready != 0 && a->lse_ready != 1)) return B3_ERR_ARG;
  // 16-byte rows: every (b, h, t) row of the staged operands
  const int64_t es = a->dtype == B3_BF16 ? 2 : 4;
  if ((a->q_sb * es) % 16 || (a->q_sh * es) % 16 || (a->w_sb * es) % 16 || (a->w_sh * es) % 16 ||
      (a->dy_sb * es) % 16 || (a->dy_st * es) % 16)
    return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (a->dtype == B3_F32) {
    rc = a->HD == 64 ? b3::bwd::set_smem<float, 64>() : b3::bwd::set_smem<float, 128>();
    if (rc) return rc;
    return a->HD == 64 ? b3::bwd::launch<float, 64>(*a, st) : b3::bwd::launch<float, 128>(*a, st);
  }
  rc = a->HD == 64 ? b3::bwd::set_smem<uint16_t, 64>() : b3::bwd::set_smem<uint16_t, 128>();
  if (rc) return rc;
  return a->HD == 64 ? b3::bwd::launch<uint16_t, 64>(*a, st) : b3::bwd::launch<uint16_t, 128>(*a, st);
}

// Backward of the Bolt-3 chunk attention and M_res readout (gfx950).
//
// The forward of every chunk c is a joint softmax over four key fields of its (batch, kv head)
// row -- [sinks | attractor slots | previous chunk | own chunk (causal)] -- with the slot field's
// bias kappa*log(mass) (-inf for inactive slots), plus the readout
//     y += eta * RMSNorm(normalize(q_raw) . M * (1 - gamma) / sqrt(HD))
// for chunks c >= 2, which use the slot snapshot and M_res of consolidation step c - 2
// (vsa_lm/config/bolt3.py:219-256).  bolt3_attn_bwd runs three kernels:
//
//   readout: per row D = sum_d dy * (attention output), with the readout's own contribution
//     taken out of y; the readout's gradients with respect to eta, q_raw, M (one dM per
//     chunk), res_norm's weight and gamma.
//   dq: with each row's log-sum-exp as the forward kept it, dS = P * (dO . V^T - D) block by
//     block, dQ = scale * dS . K and the slot columns' sums of dS (the gradient of the slot bias).
//   dkv: every 32-key block of every field over every query row of the chunk's G heads:
//     dV = P^T . dO, dK = scale * dS^T . Q.  Every key row has one writer: the previous chunk's
//     keys go to d_k_next, the chunk's own keys to d_k_own, slots to d_slot_k of step c - 2,
//     sinks to d_sink_k of chunk c.
//
// fp32 storage runs kernels with fp32 arithmetic on the vector ALUs (operands widened while they
// are staged in LDS); bf16 storage runs MFMA kernels (described with them below).  Scores are
// rebuilt like the forward's (the q.k product rounded to the storage dtype first when
// score_round is set, then scale, bias, mask).
#include <math.h>

#include <type_traits>

#include "bolt3_common.h"
#include "bolt3_lds.h"
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

  // every row's log-sum-exp, as the forward kept it
  float lse[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lse[i] = 4 * rg + i < nq ? a.lse[row0 + 4 * rg + i] : 0.f;

  // dS block by block, dQ += dS . K, slot-bias gradient
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
// The same gradients for bf16 storage on v_mfma_f32_32x32x16_bf16 with fp32 accumulation.  The
// bf16 operands are the stored q, k, v (exact) and dO, P, dS rounded to bf16 where they enter a
// product, as the reference's autocast backward rounds them.  Layouts follow the forward: a
// 32x32 product tile holds, in lane l, column l % 32 and rows d_row(l, r); the A operand row
// l % 32 and the B operand column l % 32 carry the K elements 8 * (l / 32) .. + 7.  A product
// whose K dimension is the rows of an earlier accumulator (dQ^T = K^T dS^T, dK^T = Q^T dS,
// dV^T = dO^T P) takes that accumulator as its B operand in the accumulator's own row order and
// reads the A operand transposed (ds_read_b64_tr_b16) out of a staged tile.
//
// Both kernels run four wavefronts per workgroup over a ring of NSB LDS stages that
// global->LDS loads fill NSB - 1 tiles ahead of the one in use (f2 layout, bolt3_lds.h; every
// wavefront issues a quarter of each tile), with one barrier per tile:
//   attn_bwd_dkv_mfma_kernel, grid (key-block quads, B*HKV, chunks): wavefront w owns key block
//     4 x + w of the chunk's block list [sinks | slots | previous chunk | own chunk] (32 keys,
//     its K and V rows in registers, its dK and dV in accumulators); the four share the 32-row
//     query tiles of the chunk's G heads (q_rope and dO rows, lse and D per row).
//   attn_bwd_dq_mfma_kernel, grid (query-tile quads, B*HKV, chunks): wavefront w owns the
//     (query tile, head) pair 4 x + w of the chunk's pairs, tile-major (for G = 4 the four heads
//     of one tile, whose causal extents agree); the four share the key blocks (K and V rows, the
//     slot bias).
constexpr float L2E = 1.4426950408889634f;
constexpr int NSB = 4;   // LDS stages of the ring

// key block kb of chunk c in the list [sinks | slots | previous chunk | own chunk] (32 keys per
// block, a field's last block partial): its field and first key; false past the list
__device__ __forceinline__ bool key_block(const b3_attn_bwd_args& a, int b, int hkv, int c, int kb, KField& f,
                                          int& j0) {
  const int n_fields = __popc(field_mask(a, c));
  for (int fi = 0; fi < n_fields; ++fi) {
    f = chunk_field<uint16_t>(a, b, hkv, c, fi);
    const int nb = (f.len + 31) / 32;
    if (kb < nb) {
      j0 = 32 * kb;
      return true;
    }
    kb -= nb;
  }
  return false;
}

// A walk over a chunk's key blocks in list order (the block's field and first key), one block
// per step
struct BlockCursor {
  KField f;
  int fi, j0;
  __device__ __forceinline__ BlockCursor(const b3_attn_bwd_args& a, int b, int hkv, int c)
      : f(chunk_field<uint16_t>(a, b, hkv, c, 0)), fi(0), j0(0) {}
  __device__ __forceinline__ void next(const b3_attn_bwd_args& a, int b, int hkv, int c) {
    j0 += 32;
    if (j0 >= f.len && fi + 1 < __popc(field_mask(a, c))) {
      j0 = 0;
      f = chunk_field<uint16_t>(a, b, hkv, c, ++fi);
    }
  }
};

// accumulator values as the B operand of K chunk kc (rows 8 kc .. 8 kc + 7 of the 16), bf16
__device__ __forceinline__ u16x8 acc_operand(const f32x16& v, int kc) {
  u32x4v b;
#pragma unroll
  for (int e = 0; e < 4; ++e) b[e] = pack_bf2(v[8 * kc + 2 * e], v[8 * kc + 2 * e + 1]);
  return __builtin_bit_cast(u16x8, b);
}

template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// One 32-row tile of [rows][HD] bf16 in the f2 layout: the global->LDS loads of its 8-row x
// 8-piece blocks blk0 .. blk0 + nblk - 1, row r of the tile from src_row(r) (lane L: row
// 8 (blk % 4) + L % 8, piece 8 (blk / 4) + L / 8)
template <int HD, typename RowPtr>
__device__ __forceinline__ void issue_tile(unsigned char* dst, int blk0, int nblk, int lane, RowPtr src_row) {
  for (int k = 0; k < nblk; ++k) {
    const int blk = blk0 + k;
    const int r = 8 * (blk % (F2_ROWS / 8)) + (lane & 7), pc = 8 * (blk / (F2_ROWS / 8)) + (lane >> 3);
    lds_dma16(src_row(r) + 8 * pc, dst + F2_BLK * blk);
  }
}

// The transposed operand (K chunk kc, feature block db) of a staged f2 tile from the eight
// reads f2_vreads made for that K chunk
__device__ __forceinline__ u16x8 tr_pair(const u16x4 (&tv)[8], int db) {
  u16x8 av;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    av[e] = tv[2 * db][e];
    av[4 + e] = tv[2 * db + 1][e];
  }
  return av;
}

// dkv: eight wavefronts, two per key block of the workgroup's four.  The first of a pair ("P
// wavefront", w < 4) forms S = Q K^T and P for a query tile, adds dO^T P to dV and leaves P in
// LDS; the second ("dS wavefront") takes that P one tile later, forms dP = dO V^T and
// dS = P (dP - D) and adds Q^T dS to dK.  Each holds one of K / V and one of dK / dV, which
// keeps both within the registers of two wavefronts per SIMD.
constexpr int NSK = 4;   // LDS stages of the dkv ring (the dS wavefronts use the stage before)

template <int HD>
struct DkvMfmaSmem {
  static constexpr int TB = (HD / 64) * (F2_ROWS / 8) * F2_BLK;   // bytes of one staged tile
  alignas(16) unsigned char q[NSK][TB];   // the query tile's q_rope rows
  alignas(16) unsigned char o[NSK][TB];   // its dO rows
  alignas(16) float ld[NSK][64];          // its rows' lse (natural log), then D
  alignas(16) float pt[2][4][16 * 64];    // P of each key block, in the accumulator's lane order
};

template <int HD>
__global__ void __launch_bounds__(512, 1) attn_bwd_dkv_mfma_kernel(b3_attn_bwd_args a) {
  using Sm = DkvMfmaSmem<HD>;
  __shared__ Sm sm;
  constexpr int KS = HD / 16, NDB = HD / 32;
  constexpr int IPT = Sm::TB / F2_BLK;    // loads per tile
  constexpr int LPW = 2 * IPT / 8;        // per wavefront per query tile (q_rope and dO)
  static_assert(LPW * 8 == 2 * IPT && IPT % LPW == 0, "tile loads divide over the wavefronts");
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // (wavefront-uniform: scalar branches)
  const int kbw = w & 3;                                     // the wavefront's key block
  const bool ds_wave = w >= 4;
  // XCD-aware order: the key-block quads of one (bh, chunk) read the same query tiles
  const GridPos gp = xcd_grid_pos();
  const int bh = gp.y, b = bh / a.HKV, hkv = bh % a.HKV, c = gp.z;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c);
  const float sl = L2E / sqrtf((float)HD);
  // the workgroup's four blocks (every wavefront derives all four: uniform decisions), the first
  // query row any of them needs, and this wavefront's own
  KField f{};
  int j0 = 0, q_lo = 1 << 30;
  bool mine = false, any = false;
  for (int i = 0; i < 4; ++i) {
    KField fi;
    int ji;
    if (!key_block(a, b, hkv, c, 4 * gp.x + i, fi, ji)) break;
    any = true;
    q_lo = min(q_lo, fi.kind == 3 ? ji : 0);
    if (i == kbw) {
      f = fi;
      j0 = ji;
      mine = true;
    }
  }
  if (!any) return;   // the whole workgroup
  const int qt0 = q_lo / 32, nqt = (tc + 31) / 32 - qt0, n_it = G * nqt;
  const int j = j0 + n;   // this lane's key
  const bool kval = mine && j < f.len;
  const float kb2 = (mine && f.kind == 1) ? f.bias[min(j, f.len - 1)] * L2E : 0.f;
  // B operands: the lane's key row (P wavefronts) or value row (dS wavefronts), 16 ks + 8 h ..
  u16x8 kv[KS];
  if (mine) {
    const int kr = min(j, f.len - 1);
    const uint16_t* p = reinterpret_cast<const uint16_t*>(ds_wave ? f.v : f.k) + (long long)kr * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kv[ks] = *reinterpret_cast<const u16x8*>(p + 16 * ks + 8 * h);
  }
  const uint16_t* qr_base = reinterpret_cast<const uint16_t*>(a.q_rope) + (long long)b * a.q_sb;
  const uint16_t* dy_base = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb;
  // the loads of query tile it into stage it % NSK: wavefront w issues loads w LPW .. of the
  // tile's 2 IPT (q_rope blocks, then dO blocks); wavefront 0 also the 32 rows' lse and D
  auto issue = [&](int it) {
    const int st = it % NSK, hq = hkv * G + it / nqt, q0 = 32 * (qt0 + it % nqt);
    const long long t0 = (long long)c * a.C;
    if (w * LPW < IPT) {
      const uint16_t* qb = qr_base + (long long)hq * a.q_sh;
      issue_tile<HD>(sm.q[st], w * LPW, LPW, lane,
                     [&](int r) { return qb + (t0 + min(q0 + r, tc - 1)) * HD; });
    } else {
      const uint16_t* ob = dy_base + (long long)hq * HD;
      issue_tile<HD>(sm.o[st], w * LPW - IPT, LPW, lane,
                     [&](int r) { return ob + (t0 + min(q0 + r, tc - 1)) * a.dy_st; });
    }
    if (w == 0) {
      const long long row = ((long long)b * a.H + hq) * a.T + t0 + min(q0 + n, tc - 1);
      lds_dma4((h == 0 ? a.lse : a.d_rows) + row, sm.ld[st]);
    }
  };
  const int my_lpt = LPW + (w == 0 ? 1 : 0);
  for (int i = 0; i < min(NSK - 2, n_it); ++i) issue(i);

  // dV (P wavefronts) or dK (dS wavefronts) of the block: rows features, columns keys
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();
  // per-lane LDS bases: row reads (row n, piece 2 ks + h), transposed reads, the P exchange
  const int jv = lane & 15, grp = lane >> 4;
  const uint32_t lane_row = f2_off(n, h);
  const uint32_t lane_tr = f2_off(4 * h + (jv >> 2), 2 * (grp & 1) + ((jv >> 1) & 1)) + 8 * (jv & 1);
  // the P wavefront takes tile it, the dS wavefront tile it - 1 (whose P the barrier at the top
  // of this iteration has published)
  for (int it = 0; it <= n_it; ++it) {
    if (it < n_it) wait_vm_rt(min(NSK - 3, n_it - 1 - it) * my_lpt);
    sync_lds();   // tile it is in LDS; tile it - 2's stage is free
    if (it + NSK - 2 < n_it) issue(it + NSK - 2);
    const int ti = ds_wave ? it - 1 : it;
    if (ti < 0 || ti >= n_it || !mine) continue;
    const int st = ti % NSK, q0 = 32 * (qt0 + ti % nqt);
    if (f.kind == 3 && q0 + 31 < j0) continue;   // every query precedes every key
    const uint32_t qa = lds_addr(sm.q[st]), oa = lds_addr(sm.o[st]);
    const uint32_t pa = lds_addr(sm.pt[ti & 1][kbw]) + 16 * lane;
    const uint32_t la = lds_addr(sm.ld[st]) + 16 * h;
    // S = Q K^T (P wavefront) or dP = dO V^T (dS wavefront): rows queries, columns the keys
    const uint32_t ra = (ds_wave ? oa : qa) + lane_row;
    f32x16 s = zero16();
    static_for<KS / 2>([&](auto ic) {
      constexpr int k2 = decltype(ic)::value;
      u16x8 v0 = lds_read_b128_at<f2_off(0, 4 * k2)>(ra);
      u16x8 v1 = lds_read_b128_at<f2_off(0, 4 * k2 + 2)>(ra);
      lds_wait2(v0, v1);
      mma_bf16(s, v0, kv[2 * k2]);
      mma_bf16(s, v1, kv[2 * k2 + 1]);
    });
    // the first K chunk's transposed operand (dO^T for dV, Q^T for dK) and the rows' lse / D
    // (and P), read while the products finish
    const uint32_t ta = (ds_wave ? qa : oa) + lane_tr;
    u16x4 tv[8];
    f2_vreads<NDB, 0>(tv, ta);
    fx4 rs[4], pv[4];
    if (!ds_wave) {
      rs[0] = lds_read_f4_at<0>(la);
      rs[1] = lds_read_f4_at<32>(la);
      rs[2] = lds_read_f4_at<64>(la);
      rs[3] = lds_read_f4_at<96>(la);
    } else {
      rs[0] = lds_read_f4_at<128>(la);
      rs[1] = lds_read_f4_at<160>(la);
      rs[2] = lds_read_f4_at<192>(la);
      rs[3] = lds_read_f4_at<224>(la);
      pv[0] = lds_read_f4_at<0>(pa);
      pv[1] = lds_read_f4_at<1024>(pa);
      pv[2] = lds_read_f4_at<2048>(pa);
      pv[3] = lds_read_f4_at<3072>(pa);
      lds_wait4(pv[0], pv[1], pv[2], pv[3]);
    }
    lds_wait4(rs[0], rs[1], rs[2], rs[3]);
    lds_wait8(tv);
    if (!ds_wave) {
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
        const bool on = kval && q0 + qr < tc && !(causal && j > q0 + qr);
        s[r] = on ? __builtin_amdgcn_exp2f(fmaf(s[r], sl, kb2) - rs[r >> 2][r & 3] * L2E) : 0.f;
      }
      // P for the dS wavefront
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        fx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = s[4 * r4 + e];
        lds_write_f4(pa + 1024 * r4, v);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = pv[r >> 2][r & 3] * (s[r] - rs[r >> 2][r & 3]);   // dS
    }
    // dV^T += dO^T P or dK^T += Q^T dS (K = the tile's rows)
    {
      const u16x8 bp = acc_operand(s, 0);
#pragma unroll
      for (int db = 0; db < NDB; ++db) mma_bf16(acc[db], tr_pair(tv, db), bp);
    }
    f2_vreads<NDB, 1>(tv, ta);
    lds_wait8(tv);
    {
      const u16x8 bp = acc_operand(s, 1);
#pragma unroll
      for (int db = 0; db < NDB; ++db) mma_bf16(acc[db], tr_pair(tv, db), bp);
    }
  }
  if (!mine || n >= min(32, f.len - j0)) return;
  const float scale = ds_wave ? 1.0f / sqrtf((float)HD) : 1.0f;
  const long long HDl = HD;
  if (f.kind >= 2) {
    // token rows: bf16, the storage dtype
    const long long o = ((long long)bh * a.T + (long long)(f.kind == 2 ? c - 1 : c) * a.C + j) * HDl;
    uint16_t* out = static_cast<uint16_t*>(ds_wave ? (f.kind == 2 ? a.d_k_next : a.d_k_own)
                                                   : (f.kind == 2 ? a.d_v_next : a.d_v_own)) + o;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * db + 8 * g4 + 4 * h;
        *reinterpret_cast<uint2*>(out + d0) =
            make_uint2(pack_bf2(acc[db][4 * g4] * scale, acc[db][4 * g4 + 1] * scale),
                       pack_bf2(acc[db][4 * g4 + 2] * scale, acc[db][4 * g4 + 3] * scale));
      }
    return;
  }
  // sinks and slots: fp32 (the chain's backward sums them further)
  float* out;
  if (f.kind == 0) {
    const long long o = (((long long)c * a.B * a.HKV + bh) * a.n_sinks + j) * HDl;
    out = (ds_wave ? a.d_sink_k : a.d_sink_v) + o;
  } else {
    const long long o = (((long long)(c - 2) * a.B * a.HKV + bh) * a.S + j) * HDl;
    out = (ds_wave ? a.d_slot_k : a.d_slot_v) + o;
  }
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = 32 * db + 8 * g4 + 4 * h;
      *reinterpret_cast<float4*>(out + d0) = make_float4(acc[db][4 * g4] * scale, acc[db][4 * g4 + 1] * scale,
                                                         acc[db][4 * g4 + 2] * scale, acc[db][4 * g4 + 3] * scale);
    }
}

template <int HD>
struct DqMfmaSmem {
  static constexpr int TB = (HD / 64) * (F2_ROWS / 8) * F2_BLK;   // bytes of one staged tile
  alignas(16) unsigned char k[NSB][TB];   // the key block's K rows
  alignas(16) unsigned char v[NSB][TB];   // its V rows
  alignas(16) float bias[NSB][64];        // slot blocks: the 32 keys' bias (twice)
};

template <int HD>
__global__ void __launch_bounds__(256, 2) attn_bwd_dq_mfma_kernel(b3_attn_bwd_args a) {
  using Sm = DqMfmaSmem<HD>;
  __shared__ Sm sm;
  constexpr int KS = HD / 16, NDB = HD / 32;
  constexpr int IPT = Sm::TB / F2_BLK;
  constexpr int LPW = 2 * IPT / 4;
  static_assert(LPW * 4 == 2 * IPT && IPT % LPW == 0, "tile loads divide over the wavefronts");
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // (wavefront-uniform: scalar branches)
  // XCD-aware order: the query-tile quads of one (bh, chunk) read the same key blocks
  const GridPos gp = xcd_grid_pos();
  const int bh = gp.y, b = bh / a.HKV, hkv = bh % a.HKV, c = gp.z;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c), nqt = (tc + 31) / 32;
  const int n_pairs = G * nqt;
  if (4 * gp.x >= n_pairs) return;   // the whole workgroup
  // this wavefront's (query tile, head) pair and the workgroup's last query row
  const int pair = 4 * gp.x + w;
  const bool mine = pair < n_pairs;
  const int qt = mine ? pair / G : 0, g = mine ? pair % G : 0;
  const int q_hi = min(tc - 1, 32 * ((min(n_pairs, 4 * gp.x + 4) - 1) / G) + 31);
  const int hq = hkv * G + g, q0 = 32 * qt;
  const int qi = q0 + n;   // this lane's query
  const bool qok = mine && qi < tc;
  const long long t = (long long)c * a.C + min(qi, tc - 1);
  const long long row = ((long long)b * a.H + hq) * a.T + t;
  const float sl = L2E / sqrtf((float)HD);
  // B operands: the lane's query row and dO row; its lse (log2 units) and D
  u16x8 qf[KS], of[KS];
  {
    const uint16_t* qr = reinterpret_cast<const uint16_t*>(a.q_rope) + (long long)b * a.q_sb + (long long)hq * a.q_sh +
                         t * HD;
    const uint16_t* dr = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb + t * a.dy_st + (long long)hq * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = *reinterpret_cast<const u16x8*>(qr + 16 * ks + 8 * h);
      of[ks] = *reinterpret_cast<const u16x8*>(dr + 16 * ks + 8 * h);
    }
  }
  const float lse2 = a.lse[row] * L2E, drow = a.d_rows[row];
  // key blocks: every block of the fields before the own chunk, the own chunk's up to q_hi
  int n_blk = 0;
  {
    const int n_fields = __popc(field_mask(a, c));
    for (int fi = 0; fi < n_fields; ++fi) {
      const KField f = chunk_field<uint16_t>(a, b, hkv, c, fi);
      n_blk += f.kind == 3 ? q_hi / 32 + 1 : (f.len + 31) / 32;
    }
  }
  // the loads of key block kb into stage kb % NSB: wavefront w issues loads w LPW .. of the
  // block's 2 IPT (K blocks, then V blocks); wavefront 0 also the slot bias (any valid address
  // for the other fields)
  BlockCursor icur(a, b, hkv, c);   // the next block to issue
  auto issue = [&](int kb) {
    const int st = kb % NSB;
    const KField& f = icur.f;
    const int j0 = icur.j0, last = f.len - 1;
    if (w * LPW < IPT) {
      const uint16_t* kp = reinterpret_cast<const uint16_t*>(f.k);
      issue_tile<HD>(sm.k[st], w * LPW, LPW, lane, [&](int r) { return kp + (long long)min(j0 + r, last) * HD; });
    } else {
      const uint16_t* vp = reinterpret_cast<const uint16_t*>(f.v);
      issue_tile<HD>(sm.v[st], w * LPW - IPT, LPW, lane,
                     [&](int r) { return vp + (long long)min(j0 + r, last) * HD; });
    }
    if (w == 0) lds_dma4(f.kind == 1 ? f.bias + min(j0 + n, last) : a.lse, sm.bias[st]);
    icur.next(a, b, hkv, c);
  };
  const int my_lpt = LPW + (w == 0 ? 1 : 0);
  for (int i = 0; i < min(NSB - 1, n_blk); ++i) issue(i);

  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = zero16();
  const int jv = lane & 15, grp = lane >> 4;
  const uint32_t lane_row = f2_off(n, h);
  const uint32_t lane_tr = f2_off(4 * h + (jv >> 2), 2 * (grp & 1) + ((jv >> 1) & 1)) + 8 * (jv & 1);
  const long long bias_row = (((long long)(c - 2) * a.B * a.H + (long long)b * a.H + hq) * a.n_qtiles + qt) * a.S;
  BlockCursor ccur(a, b, hkv, c);   // the block computed
  for (int kb = 0; kb < n_blk; ++kb) {
    wait_vm_rt(min(NSB - 2, n_blk - 1 - kb) * my_lpt);
    sync_lds();   // block kb is in LDS; every wavefront is done with block kb - 1, whose stage is refilled
    if (kb + NSB - 1 < n_blk) issue(kb + NSB - 1);
    if (kb > 0) ccur.next(a, b, hkv, c);
    const KField& f = ccur.f;
    const int j0 = ccur.j0;
    if (!mine || (f.kind == 3 && j0 > q0 + 31)) continue;   // every key follows every query
    const int st = kb % NSB;
    const uint32_t ka = lds_addr(sm.k[st]), va = lds_addr(sm.v[st]);
    // S^T = K Q^T and dP^T = V dO^T: rows the block's keys, columns the wavefront's queries
    f32x16 s = zero16(), dp = zero16();
    static_for<KS / 2>([&](auto ic) {
      constexpr int k2 = decltype(ic)::value;
      u16x8 k0v = lds_read_b128_at<f2_off(0, 4 * k2)>(ka + lane_row);
      u16x8 v0v = lds_read_b128_at<f2_off(0, 4 * k2)>(va + lane_row);
      u16x8 k1v = lds_read_b128_at<f2_off(0, 4 * k2 + 2)>(ka + lane_row);
      u16x8 v1v = lds_read_b128_at<f2_off(0, 4 * k2 + 2)>(va + lane_row);
      lds_wait2(k0v, v0v);
      lds_wait2(k1v, v1v);
      mma_bf16(s, k0v, qf[2 * k2]);
      mma_bf16(dp, v0v, of[2 * k2]);
      mma_bf16(s, k1v, qf[2 * k2 + 1]);
      mma_bf16(dp, v1v, of[2 * k2 + 1]);
    });
    // K^T for the first K chunk and the bias, read while the scores are formed
    u16x4 tk[8];
    f2_vreads<NDB, 0>(tk, ka + lane_tr);
    fx4 bv[4];
    if (f.kind == 1) {
      const uint32_t ba = lds_addr(sm.bias[st]) + 16 * h;
      bv[0] = lds_read_f4_at<0>(ba);
      bv[1] = lds_read_f4_at<32>(ba);
      bv[2] = lds_read_f4_at<64>(ba);
      bv[3] = lds_read_f4_at<96>(ba);
      lds_wait4(bv[0], bv[1], bv[2], bv[3]);
    }
    lds_wait8(tk);
    if (a.score_round) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const uint32_t u = pack_bf2(s[r], s[r + 1]);
        s[r] = bf_lo(u);
        s[r + 1] = bf_hi(u);
      }
    }
    const bool edge = j0 + 32 > f.len || (f.kind == 3 && j0 + 31 > q0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jj = j0 + d_row(lane, r);
      float x = f.kind == 1 ? fmaf(s[r], sl, bv[r >> 2][r & 3] * L2E) : s[r] * sl;
      if (edge && (jj >= f.len || (f.kind == 3 && jj > qi))) x = -INFINITY;
      const float p = qok ? __builtin_amdgcn_exp2f(x - lse2) : 0.f;
      s[r] = p * (dp[r] - drow);   // dS^T
    }
    if (f.kind == 1) {
      // the slot bias gradient: column sums over the wavefront's queries (the lanes of each half)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[r];
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        const int jj = j0 + d_row(lane, r);
        if (n == 0 && jj < f.len) a.d_bias[bias_row + jj] = v;
      }
    }
    // dQ^T += K^T dS^T (K = the block's keys)
    {
      const u16x8 bs = acc_operand(s, 0);
#pragma unroll
      for (int db = 0; db < NDB; ++db) mma_bf16(dq[db], tr_pair(tk, db), bs);
    }
    f2_vreads<NDB, 1>(tk, ka + lane_tr);
    lds_wait8(tk);
    {
      const u16x8 bs = acc_operand(s, 1);
#pragma unroll
      for (int db = 0; db < NDB; ++db) mma_bf16(dq[db], tr_pair(tk, db), bs);
    }
  }
  if (!qok) return;
  const float scale = 1.0f / sqrtf((float)HD);
  uint16_t* o = static_cast<uint16_t*>(a.d_q_rope) + row * HD;   // bf16, the storage dtype
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      *reinterpret_cast<uint2*>(o + 32 * db + 8 * g4 + 4 * h) =
          make_uint2(pack_bf2(dq[db][4 * g4] * scale, dq[db][4 * g4 + 1] * scale),
                     pack_bf2(dq[db][4 * g4 + 2] * scale, dq[db][4 * g4 + 3] * scale));
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
// The readout's gradients for bf16 storage on MFMA in two kernels.  The row kernel: one
// workgroup of RD_W wavefronts per (b, kv head, chunk), one query row per lane column, 32 rows
// per wavefront and round:
//   U^T = M^T q_raw^T            (M^T as bf16 hi + lo, q_raw exact: two products, as the forward)
//   u = U / |q_raw|, ym = u (1-gamma)/sqrt(HD), the RMSNorm backward as the fp32 kernel
//   dqn^T = M du^T               (M^T read transposed; hi/lo on both sides: three products)
//   du / |q_raw| as bf16 rows into rd_rows
// with each round's dy and y rows loaded once, at its start.  The dM kernel, one workgroup of
// four wavefronts per (b, kv head, chunk):
//   dM = q_raw^T (du / |q_raw|)  (32-row tiles of both staged in LDS, read transposed; wavefront
//                                 w accumulates its share of the (HD/32)^2 output tiles, the
//                                 tiles and their two K halves in row order)
constexpr int RD_W = 8;   // wavefronts of the row kernel

template <int HD>
struct RdMfmaSmem {
  alignas(16) uint16_t mt[2][HD * HD];     // M^T hi, lo: row d, 16-byte piece p at p ^ (d % (HD/8))
  alignas(16) uint16_t qt[RD_W][32 * HD];  // per wavefront: q_raw rows of its tile (same swizzle)
  float resw[HD];
  float red[RD_W][HD + 1];
};

template <int HD>
__global__ void __launch_bounds__(64 * RD_W) readout_bwd_mfma_kernel(b3_attn_bwd_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  RdMfmaSmem<HD>& sm = *reinterpret_cast<RdMfmaSmem<HD>*>(smem_raw);
  constexpr int KS = HD / 16, NDB = HD / 32, NP = HD / 8, NT_RD = 64 * RD_W;
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
    for (int r0 = 4 * w; r0 < n_rows; r0 += 4 * RD_W) {
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
    // every load of the thread's items before their stores: one memory round trip
    constexpr int NI = (2 * HD * NP + NT_RD - 1) / NT_RD;
    u16x8 mv[NI];
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int it = tid + NT_RD * q;
      const int half = it / (HD * NP), rem = it % (HD * NP), d = rem / NP, pc = rem % NP;
      if (it < 2 * HD * NP) mv[q] = *reinterpret_cast<const u16x8*>(src + (long long)half * HD * HD + d * HD + 8 * pc);
    }
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int it = tid + NT_RD * q;
      const int half = it / (HD * NP), rem = it % (HD * NP), d = rem / NP, pc = rem % NP;
      if (it < 2 * HD * NP) *reinterpret_cast<u16x8*>(&sm.mt[half][d * HD + 8 * (pc ^ (d % NP))]) = mv[q];
    }
    for (int it = tid; it < HD; it += NT_RD) sm.resw[it] = a.res_w[it];
  }
  __syncthreads();
  const float sg = (1.0f - a.gamma[hkv]) / sqrtf((float)HD);
  const TrLanes<HD> TL(lane);
  // res_w partials: dres[db] is feature 32 db + d_row(lane, r) with r = 8 (n >> 4 & 1) +
  // 4 (n >> 3 & 1) + 2 (n >> 2 & 1) + (n >> 1 & 1) (the reduce-scatter below leaves it there)
  float dres[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dres[db] = 0.f;
  float dsg = 0.f;
  uint16_t* qt = sm.qt[w];
  const int n_tiles = (n_rows + 31) / 32;
#pragma unroll 1
  for (int r0 = 0; r0 < n_tiles; r0 += RD_W) {
    const int q = 32 * (r0 + w) + n;
    const bool live = q < n_rows;
    const int g = live ? q / tc : 0, i = live ? q % tc : 0;
    const int hq = hkv * G + g;
    const long long t = (long long)c * a.C + i;
    const long long row = ((long long)b * a.H + hq) * a.T + t;
    // the lane's q_raw row: B operand (K elements 16 ks + 8 h ..) and row n of the tile
    u16x8 qf[KS];
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q_raw) + (long long)b * a.q_sb + (long long)hq * a.q_sh +
                         t * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[ks] = live ? *reinterpret_cast<const u16x8*>(qp + 16 * ks + 8 * h) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    const float eta = live ? a.eta[(long long)b * a.e_sb + (long long)hq * a.e_sh + t] : 0.f;
    // the round's dy at this lane's accumulator features 32 db + 8 r4 + 4 h .. + 3, loaded once,
    // while the U^T products run (y follows once they are issued)
    const uint16_t* dyp = reinterpret_cast<const uint16_t*>(a.dy) + (long long)b * a.dy_sb + t * a.dy_st +
                          (long long)hq * HD;
    const uint16_t* yp = reinterpret_cast<const uint16_t*>(a.y) + (long long)b * a.y_sb + t * a.y_st + (long long)hq * HD;
    uint2 dyr[NDB][4], yr[NDB][4];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        dyr[db][r4] = live ? *reinterpret_cast<const uint2*>(dyp + 32 * db + 8 * r4 + 4 * h) : make_uint2(0u, 0u);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) *reinterpret_cast<u16x8*>(&qt[n * HD + 8 * ((2 * ks + h) ^ (n % NP))]) = qf[ks];
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
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        yr[db][r4] = live ? *reinterpret_cast<const uint2*>(yp + 32 * db + 8 * r4 + 4 * h) : make_uint2(0u, 0u);
    // the RMSNorm backward of ym = u * sg at this lane's features d = 32 db + d_row(lane, r)
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
      float xr[16];   // res_w terms of the block
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * db + 8 * r4 + 4 * h;
        const uint2 g2 = dyr[db][r4], y2 = yr[db][r4];
        const float4 w4 = *reinterpret_cast<const float4*>(&sm.resw[d0]);
        const float dyv[4] = {bf_lo(g2.x), bf_hi(g2.x), bf_lo(g2.y), bf_hi(g2.y)};
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
    // du = sg (rr g - ym rr^3 gdot / HD), g = eta dy w, in place of u; the gamma partial; du /
    // |q_raw| as bf16 into the row scratch (the dM kernel's operand)
    float dsg_r = 0.f;
    const float c3 = rr * rr * rr * gdot / (float)HD;
    uint16_t* ru = static_cast<uint16_t*>(a.rd_rows) + row * HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * db + 8 * r4 + 4 * h;
        const uint2 g2 = dyr[db][r4];
        const float4 w4 = *reinterpret_cast<const float4*>(&sm.resw[d0]);
        const float dyv[4] = {bf_lo(g2.x), bf_hi(g2.x), bf_lo(g2.y), bf_hi(g2.y)};
        const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * r4 + j;
          const float ym = u[db][r];
          const float dym = rr * (eta * dyv[j] * wv[j]) - ym * c3;
          dsg_r += dym * ym;
          u[db][r] = live ? dym * sg : 0.f;
        }
        if (live)
          *reinterpret_cast<uint2*>(ru + d0) = make_uint2(pack_bf2(u[db][4 * r4] * inv, u[db][4 * r4 + 1] * inv),
                                                          pack_bf2(u[db][4 * r4 + 2] * inv, u[db][4 * r4 + 3] * inv));
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
        // the row's swizzle, opaque here so that the sixteen read addresses are formed at their
        // use (hoisted out of the row loop they were spilled, and every reload waited on vmcnt)
        int sw = n % NP;
        asm volatile("" : "+v"(sw));
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const uint2 q2 = *reinterpret_cast<const uint2*>(&qt[n * HD + 8 * ((4 * cb + r4) ^ sw) + 4 * h]);
          float4 v;
          v.x = (dq[4 * r4] - bf_lo(q2.x) * qi2) * inv;
          v.y = (dq[4 * r4 + 1] - bf_hi(q2.x) * qi2) * inv;
          v.z = (dq[4 * r4 + 2] - bf_lo(q2.y) * qi2) * inv;
          v.w = (dq[4 * r4 + 3] - bf_hi(q2.y) * qi2) * inv;
          *reinterpret_cast<uint2*>(o + 32 * cb + 8 * r4 + 4 * h) = make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
        }
      }
    }
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
  if (tid <= HD) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < RD_W; ++k) s += sm.red[k][tid];
    if (tid < HD) a.d_res_w[pc * HD + tid] = s;
    else a.d_gamma[pc] = -s / sqrtf((float)HD);
  }
}

// dM[cf][d] = sum over the chunk's readout rows q of q_raw[q][cf] (du / |q_raw|)[q][d], chunk c
// >= 2 (blockIdx.y = c - 2).  32-row tiles of both operands go through registers into two LDS
// buffers (the next tile's loads in flight while the current one multiplies), rows past the
// chunk's as zeros; one barrier per tile.
template <int HD>
struct RdDmSmem {
  alignas(16) uint16_t qt[2][32 * HD];   // row n, 16-byte piece p at p ^ (n % (HD/8))
  alignas(16) uint16_t ut[2][32 * HD];
};

template <int HD>
__global__ void __launch_bounds__(256) readout_dm_kernel(b3_attn_bwd_args a) {
  __shared__ RdDmSmem<HD> sm;
  constexpr int NDB = HD / 32, NP = HD / 8, TPW = NDB * NDB / 4, PPT = 32 * NP / 256;
  static_assert(NDB * NDB % 4 == 0 && PPT >= 1 && 32 * NP % 256 == 0, "dM tiles and staging split over 256 threads");
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, n = lane & 31;
  const int bh = blockIdx.x, b = bh / a.HKV, hkv = bh % a.HKV, c = blockIdx.y + 2;
  const int G = a.H / a.HKV;
  const int tc = chunk_len(a, c);
  const int n_rows = G * tc;
  const int n_tiles = (n_rows + 31) / 32;
  int dm_off[TPW][4];   // transposed-read offsets of output tile tt: A (rows cf) then B (columns d)
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int id = w * TPW + tt, cb = id / NDB, db = id % NDB;
    dm_off[tt][0] = tr_off<HD>(lane, cb, 0);
    dm_off[tt][1] = tr_off<HD>(lane, cb, 1);
    dm_off[tt][2] = tr_off<HD>(lane, db, 0);
    dm_off[tt][3] = tr_off<HD>(lane, db, 1);
  }
  // this thread's 16-byte pieces of a tile: piece tid + 256 j is row / NP, piece % NP
  u16x8 rq[PPT], ru[PPT];
  auto load = [&](int k) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pi = tid + 256 * j, rl = pi / NP, p = pi % NP;
      const int q = 32 * k + rl;
      rq[j] = ru[j] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (q < n_rows) {
        const int g = q / tc, i = q % tc, hq = hkv * G + g;
        const long long t = (long long)c * a.C + i;
        rq[j] = *reinterpret_cast<const u16x8*>(reinterpret_cast<const uint16_t*>(a.q_raw) + (long long)b * a.q_sb +
                                                (long long)hq * a.q_sh + t * HD + 8 * p);
        ru[j] = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(a.rd_rows) +
                                                (((long long)b * a.H + hq) * a.T + t) * HD + 8 * p);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pi = tid + 256 * j, rl = pi / NP, p = pi % NP;
      const int o = rl * HD + 8 * (p ^ (rl % NP));
      *reinterpret_cast<u16x8*>(&sm.qt[buf][o]) = rq[j];
      *reinterpret_cast<u16x8*>(&sm.ut[buf][o]) = ru[j];
    }
  };
  f32x16 dm[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) dm[tt] = zero16();
  if (n_tiles > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
#pragma unroll 1
  for (int k = 0; k < n_tiles; ++k) {
    if (k + 1 < n_tiles) load(k + 1);
    const int buf = k & 1;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) {
        const uint16_t* pq = sm.qt[buf] + 16 * kc * HD;
        const uint16_t* pu = sm.ut[buf] + 16 * kc * HD;
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
    // the other buffer was last read in the previous tile, before the barrier that ended it
    if (k + 1 < n_tiles) store(buf ^ 1);
    __syncthreads();
  }
  // dM out: tile (cb, db) holds rows cf = 32 cb + d_row(lane, r), column d = 32 db + n
  float* dmo = a.d_m + ((long long)(c - 2) * a.B * a.HKV + bh) * HD * HD;
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int id = w * TPW + tt, cb = id / NDB, db = id % NDB;
#pragma unroll
    for (int r = 0; r < 16; ++r) dmo[(32 * cb + d_row(lane, r)) * HD + 32 * db + n] = dm[tt][r];
  }
}

template <typename T, int HD>
static int launch(const b3_attn_bwd_args& a, hipStream_t st) {
  const int n_chunks = a.n_chunks;
  const int BH = a.B * a.HKV;
  hipError_t e = hipSuccess;
  if (a.part != 2) {
    if constexpr (St<T>::is_bf16) {
      hipLaunchKernelGGL((readout_bwd_mfma_kernel<HD>), dim3(BH, n_chunks), dim3(64 * RD_W), sizeof(RdMfmaSmem<HD>),
                         st, a);
      // dM of the chunks with a readout: c = 2 .. min(n_chunks, n_steps + 2) - 1
      const int n_m = a.m_res ? min(n_chunks, a.n_steps + 2) - 2 : 0;
      e = hipGetLastError();
      if (e == hipSuccess && n_m > 0) {
        hipLaunchKernelGGL((readout_dm_kernel<HD>), dim3(BH, n_m), dim3(256), 0, st, a);
        e = hipGetLastError();
      }
    } else {
      hipLaunchKernelGGL((readout_bwd_kernel<T, HD>), dim3(BH, n_chunks), dim3(NT), sizeof(RdSmem<HD>), st, a);
      e = hipGetLastError();
    }
    if (e != hipSuccess || a.part == 1) return (int)e;
  }
  // key blocks per chunk at most: sinks, slots, previous and own chunk
  const int max_blocks = (min(a.n_sinks, a.C) + 31) / 32 + (a.S + 31) / 32 + 2 * ((a.C + 31) / 32);
  if constexpr (St<T>::is_bf16) {
    const int n_pairs = (a.H / a.HKV) * ((a.C + 31) / 32);
    hipLaunchKernelGGL((attn_bwd_dq_mfma_kernel<HD>), dim3((n_pairs + 3) / 4, BH, n_chunks), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((attn_bwd_dkv_mfma_kernel<HD>), dim3((max_blocks + 3) / 4, BH, n_chunks), dim3(512), 0, st, a);
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
  if (a->part < 0 || a->part > 2) return B3_ERR_ARG;
  // the bf16 readout's row scratch, 16-byte aligned rows
  if (a->dtype == B3_BF16 && a->part != 2 && a->n_steps > 0 && a->m_res &&
      (!a->rd_rows || reinterpret_cast<uintptr_t>(a->rd_rows) % 16))
    return B3_ERR_ARG;
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

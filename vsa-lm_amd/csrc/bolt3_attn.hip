// Chunk attention over the three Bolt-3 fields plus the M_res readout.
//
// Replaces the body of the chunk loop of Bolt3Attn.forward
// (vsa_lm/config/bolt3.py:219-258) for all chunks at once (mode 0), and the
// attention + readout of Bolt3Decoder.step (:365-402) for a block of queries
// against decoder state (mode 1).  For every query the keys are
//   [sinks (4) | attractor slots (S, roped at their mean positions, bias
//    kappa*log(max(mass,1)), -inf when inactive) | window: previous chunk and
//    the current chunk up to the query (causal)]
// under ONE softmax; probabilities read the matching values.  The readout adds
// eta * RMSNorm(normalize(q_raw) . M_res * (1-gamma)/sqrt(HD)).
//
// Layout: one workgroup per (bh, chunk, query tile) with G*QW wavefronts; a
// wavefront owns 32 queries of one query head, so the G query heads of a kv
// head share every K/V tile staged in LDS.  Scores are computed transposed
// (keys x queries) with 32x32 MFMAs so that each lane owns one query column:
// the online-softmax state is per lane and only one cross-half exchange is
// needed per reduction.
#include "bolt3_common.h"
#include "bolt3_lds.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int KB = 32;  // keys per LDS stage
static_assert(KB == F2_ROWS, "the staged tiles hold one key block");

template <typename T, int HD>
struct AttnSmem {
  static constexpr int KS = sizeof(T) == 2 ? HD + 8 : HD + 1;   // K row stride
  static constexpr int VS = sizeof(T) == 2 ? KB + 8 : KB + 1;   // V^T row stride
  static constexpr int MS = HD + 8;                             // M^T (bf16 hi/lo) row stride
  static constexpr int MF = HD + 1;                             // M (fp32) row stride
  static constexpr int KV_BYTES = KB * KS * sizeof(T) + HD * VS * sizeof(T);
  static constexpr int M_BYTES = sizeof(T) == 2 ? 2 * HD * MS * 2 : HD * MF * 4;
  static constexpr int BYTES = KV_BYTES > M_BYTES ? KV_BYTES : M_BYTES;
  alignas(16) unsigned char raw[BYTES];
  float bias[KB];
  __device__ T* k() { return reinterpret_cast<T*>(raw); }
  __device__ T* vt() { return reinterpret_cast<T*>(raw + KB * KS * sizeof(T)); }
  __device__ uint16_t* mhi() { return reinterpret_cast<uint16_t*>(raw); }
  __device__ uint16_t* mlo() { return reinterpret_cast<uint16_t*>(raw) + HD * MS; }
  __device__ float* mf() { return reinterpret_cast<float*>(raw); }
};

// Query fragments: lane (q = lane%32, h) holds q[q][K sub-index].
template <typename T, int HD> struct QFrag;
template <int HD> struct QFrag<uint16_t, HD> {
  u16x8 v[HD / 16];
  __device__ void load(const uint16_t* row, bool ok, int h) {
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      if (ok) v[ks] = *reinterpret_cast<const u16x8*>(row + 16 * ks + 8 * h);
      else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[ks][i] = 0;
      }
    }
  }
  __device__ float sumsq() const {
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) { const float x = bf2f(v[ks][i]); s += x * x; }
    return s;
  }
};
// The query preparation inside the forward attention (b3_attn_args.q_lin): the lane's fragment
// of row t of query head hq (pieces 2 ks + h, as QFrag) from the q projection output, then the
// optional RMSNorm and RoPE with the arithmetic of bolt3_heads -- the q half of head_qkv
// (vsa_lm/config/bolt3.py:197, the norm of vsa_lm/surgery.py:49-53) and LlamaRoPE
// (vsa_lm/surgery.py:86-93): the fp32 statistic as the same tree of sumsq_pair8 partials
// (within the lane over its pieces, then across the row's two lanes), the weight and one
// rounding; each product and the sum of the rotation rounded.  Fetches are separate from the
// arithmetic so that their latency can overlap other work.
template <int HD> struct QPrep {
  static constexpr int NKH = HD / 32;   // the lane's pieces in the first half of the head
  float4 w[HD / 8];                     // q RMSNorm weight of the lane's elements
  uint32_t cs[NKH][8];                  // (cos, sin) of the lane's first-half elements
  // t: a valid row (rows past the chunk's queries take its last one: each query's scores,
  // softmax and output depend on its own row only, and such rows are never written)
  __device__ static void fetch_row(QFrag<uint16_t, HD>& f, const b3_attn_args& a, int b, int hq, int t, int h) {
    const uint16_t* row = static_cast<const uint16_t*>(a.q_lin) + ((long long)b * a.n_q + t) * a.q_lin_stride + hq * HD;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) f.v[ks] = *reinterpret_cast<const u16x8*>(row + 16 * ks + 8 * h);
  }
  __device__ void fetch_w(const b3_attn_args& a, int h) {
    if (!a.qn_w) return;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      w[2 * ks] = *reinterpret_cast<const float4*>(a.qn_w + 16 * ks + 8 * h);
      w[2 * ks + 1] = *reinterpret_cast<const float4*>(a.qn_w + 16 * ks + 8 * h + 4);
    }
  }
  __device__ void fetch_cs(const b3_attn_args& a, int t, int h) {   // t: a valid row, as fetch_row
    const uint32_t* c = a.rope_cs + (long long)t * (HD / 2);
#pragma unroll
    for (int k = 0; k < NKH; ++k) {
      const uint4 lo = *reinterpret_cast<const uint4*>(c + 16 * k + 8 * h);
      const uint4 hi = *reinterpret_cast<const uint4*>(c + 16 * k + 8 * h + 4);
      cs[k][0] = lo.x; cs[k][1] = lo.y; cs[k][2] = lo.z; cs[k][3] = lo.w;
      cs[k][4] = hi.x; cs[k][5] = hi.y; cs[k][6] = hi.z; cs[k][7] = hi.w;
    }
  }
  // the fragment as fp32 values, x[ks][e] = element 16 ks + 8 h + e
  __device__ static void unpack(const QFrag<uint16_t, HD>& f, float (*x)[8]) {
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[ks][e] = bf2f(f.v[ks][e]);
  }
  // the row's RMS factor 1 / sqrt(mean(x^2) + eps); every lane of the wave takes part (shuffle)
  __device__ static float rms_factor(const float (*x)[8], float eps) {
    float s[NKH];
#pragma unroll
    for (int k = 0; k < NKH; ++k) s[k] = sumsq_pair8(x[k], x[k + NKH]);
    // pieces p = 2k + h: the pairs (p, p ^ HD/32) ... (p, p ^ 2) are in the lane, (p, p ^ 1) across
#pragma unroll
    for (int off = NKH / 2; off >= 1; off >>= 1)
#pragma unroll
      for (int k = 0; k < off; ++k) s[k] = add_rn(s[k], s[k + off]);
    const float ss = add_rn(s[0], __shfl_xor(s[0], 32, 64));
    return 1.0f / sqrtf(div_rn(ss, (float)HD) + eps);
  }
  // x <- round(x * r * qn_w) in place (q_raw), two elements per rounding instruction
  __device__ void scale(float (*x)[8], float r) const {
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      const float wv[8] = {w[2 * ks].x, w[2 * ks].y, w[2 * ks].z, w[2 * ks].w,
                           w[2 * ks + 1].x, w[2 * ks + 1].y, w[2 * ks + 1].z, w[2 * ks + 1].w};
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t pk = pack_bf2(mul_rn(mul_rn(x[ks][e], r), wv[e]), mul_rn(mul_rn(x[ks][e + 1], r), wv[e + 1]));
        x[ks][e] = bf_lo(pk);
        x[ks][e + 1] = bf_hi(pk);
      }
    }
  }
  // the fragment from rounded fp32 values (exact: they are bf16 values)
  __device__ static void pack(QFrag<uint16_t, HD>& f, const float (*x)[8]) {
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) f.v[ks][e] = f2bf(x[ks][e]);
  }
  // f <- RoPE(x): out = x*cos + rotate_half(x)*sin, each product and the sum rounded
  __device__ void rope(QFrag<uint16_t, HD>& f, const float (*x)[8]) const {
#pragma unroll
    for (int k = 0; k < NKH; ++k) {
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float c0 = bf_lo(cs[k][e]), s0 = bf_hi(cs[k][e]), c1 = bf_lo(cs[k][e + 1]), s1 = bf_hi(cs[k][e + 1]);
        const float u0 = x[k][e], u1 = x[k][e + 1], v0 = x[k + NKH][e], v1 = x[k + NKH][e + 1];
        const uint32_t uc = pack_bf2(mul_rn(u0, c0), mul_rn(u1, c1)), vs = pack_bf2(mul_rn(-v0, s0), mul_rn(-v1, s1));
        const uint32_t vc = pack_bf2(mul_rn(v0, c0), mul_rn(v1, c1)), us = pack_bf2(mul_rn(u0, s0), mul_rn(u1, s1));
        lo[e / 2] = pack_bf2(add_rn(bf_lo(uc), bf_lo(vs)), add_rn(bf_hi(uc), bf_hi(vs)));
        hi[e / 2] = pack_bf2(add_rn(bf_lo(vc), bf_lo(us)), add_rn(bf_hi(vc), bf_hi(us)));
      }
      f.v[k] = __builtin_bit_cast(u16x8, u32x4v{lo[0], lo[1], lo[2], lo[3]});
      f.v[k + NKH] = __builtin_bit_cast(u16x8, u32x4v{hi[0], hi[1], hi[2], hi[3]});
    }
  }
};
// eta = tanh(eta_proj x) of query head hq at row t, rounded to bf16 (vsa_lm/config/bolt3.py:199)
__device__ __forceinline__ float eta_from_gates(const b3_attn_args& a, int b, int hq, int t) {
  const uint16_t* g = static_cast<const uint16_t*>(a.gates) + ((long long)b * a.n_q + t) * a.gates_stride + a.gates_col + hq;
  return round_bf(tanhf(bf2f(*g)));
}

template <int HD> struct QFrag<float, HD> {
  float v[HD / 2];
  __device__ void load(const float* row, bool ok, int h) {
#pragma unroll
    for (int ks = 0; ks < HD / 2; ++ks) v[ks] = ok ? row[2 * ks + h] : 0.f;
  }
  __device__ float sumsq() const {
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < HD / 2; ++ks) s += v[ks] * v[ks];
    return s;
  }
};

struct Seg {
  const void* k;
  const void* v;
  long long stride_b, stride_h;  // (b, hkv) strides in elements
  int start, len;
  int kind;                      // 0 sinks, 1 slots, 2 window (older), 3 window (current, causal)
};

template <typename T, int HD>
__global__ void __launch_bounds__(512) attn_kernel(b3_attn_args a, int QW) {
  __shared__ AttnSmem<T, HD> sm;
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int g = wave / QW, qsub = wave % QW;
  const int bh = blockIdx.z, b = bh / a.HKV, hkv = bh % a.HKV;
  const int hq = hkv * G + g;
  const int chunk = blockIdx.y;
  const float scale = 1.0f / sqrtf((float)HD);

  // ---- queries of this wavefront
  int qbase, nq_chunk, qb_off;  // first query index, queries in this chunk, B-segment index of query 0
  Seg seg[4];
  int nseg = 0;
  int step = -1;  // slot / M_res snapshot index
  if (a.mode == 0) {
    qbase = chunk * a.C;
    nq_chunk = min(a.C, a.n_q - qbase);
    qb_off = 0;
    if (chunk >= 2) {
      step = chunk - 2;
      seg[nseg++] = Seg{a.win_k, a.win_v, a.w_sb, a.w_sh, 0, min(a.n_sinks, a.C), 0};
      seg[nseg++] = Seg{nullptr, nullptr, 0, 0, 0, a.S, 1};
    }
    if (chunk >= 1) seg[nseg++] = Seg{a.win_k, a.win_v, a.w_sb, a.w_sh, (chunk - 1) * a.C, a.C, 2};
    seg[nseg++] = Seg{a.win_k, a.win_v, a.w_sb, a.w_sh, qbase, nq_chunk, 3};
  } else {
    qbase = 0;
    nq_chunk = a.n_q;
    qb_off = a.b_len - a.n_q;
    if (a.n_sink_keys > 0) seg[nseg++] = Seg{a.sink_k, a.sink_v, a.s_sb, a.s_sh, 0, a.n_sink_keys, 0};
    if (a.has_slots) { seg[nseg++] = Seg{nullptr, nullptr, 0, 0, 0, a.S, 1}; step = 0; }
    if (a.a_len > 0) seg[nseg++] = Seg{a.win_k, a.win_v, a.w_sb, a.w_sh, a.a_start, a.a_len, 2};
    seg[nseg++] = Seg{a.win_k, a.win_v, a.w_sb, a.w_sh, a.b_start, a.b_len, 3};
  }
  const int qt0 = blockIdx.x * 32 * QW;          // first query of the workgroup within the chunk
  if (qt0 >= nq_chunk) return;                   // uniform across the workgroup
  const int qi = qt0 + 32 * qsub + n;            // this lane's query within the chunk
  const bool qok = qi < nq_chunk;
  const int t = qbase + qi;                      // query index in the q / y arrays
  const int wave_qmax = qt0 + 32 * qsub + 31;    // largest query of this wavefront (for causal skipping)

  const T* qrow = reinterpret_cast<const T*>(a.q_rope) + b * a.q_sb + hq * a.q_sh + (long long)t * HD;
  QFrag<T, HD> qf;
  qf.load(qrow, qok, h);

  constexpr int NDB = HD / 32;
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = zero16();
  float m_run = -INFINITY, l_run = 0.f;

  const T* slot_k = a.slot_k ? reinterpret_cast<const T*>(a.slot_k) + (long long)(step < 0 ? 0 : step) * a.slot_step +
                                   (long long)bh * a.S * HD
                             : nullptr;
  const T* slot_v = a.slot_v ? reinterpret_cast<const T*>(a.slot_v) + (long long)(step < 0 ? 0 : step) * a.slot_step +
                                   (long long)bh * a.S * HD
                             : nullptr;
  const float* slot_b = a.slot_bias ? a.slot_bias + (long long)(step < 0 ? 0 : step) * (a.slot_step / HD) +
                                          (long long)bh * a.S
                                    : nullptr;
  const int nthreads = blockDim.x;

  for (int si = 0; si < nseg; ++si) {
    const Seg sg = seg[si];
    const T* kbase;
    const T* vbase;
    if (sg.kind == 1) {
      kbase = slot_k;
      vbase = slot_v;
    } else {
      kbase = reinterpret_cast<const T*>(sg.k) + b * sg.stride_b + hkv * sg.stride_h + (long long)sg.start * HD;
      vbase = reinterpret_cast<const T*>(sg.v) + b * sg.stride_b + hkv * sg.stride_h + (long long)sg.start * HD;
    }
    for (int k0 = 0; k0 < sg.len; k0 += KB) {
      // causal skip: the whole block lies after every query of the workgroup
      const bool wg_skip = sg.kind == 3 && k0 > qb_off + qt0 + 32 * QW - 1;
      if (wg_skip) break;
      __syncthreads();
      // ---- stage K (rows) and V^T (columns) of keys k0 .. k0+KB-1
      T* sK = sm.k();
      T* sV = sm.vt();
      if constexpr (St<T>::is_bf16) {
        for (int it = tid; it < KB * (HD / 8); it += nthreads) {
          const int r = it / (HD / 8), c8 = (it % (HD / 8)) * 8;
          u16x8 kv, vv;
          if (k0 + r < sg.len) {
            kv = *reinterpret_cast<const u16x8*>(kbase + (long long)(k0 + r) * HD + c8);
            vv = *reinterpret_cast<const u16x8*>(vbase + (long long)(k0 + r) * HD + c8);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) { kv[i] = 0; vv[i] = 0; }
          }
          *reinterpret_cast<u16x8*>(sK + r * sm.KS + c8) = kv;
#pragma unroll
          for (int i = 0; i < 8; ++i) sV[(c8 + i) * sm.VS + r] = vv[i];
        }
      } else {
        for (int it = tid; it < KB * HD; it += nthreads) {
          const int r = it / HD, c = it % HD;
          const bool ok = k0 + r < sg.len;
          sK[r * sm.KS + c] = ok ? kbase[(long long)(k0 + r) * HD + c] : 0.f;
          sV[c * sm.VS + r] = ok ? vbase[(long long)(k0 + r) * HD + c] : 0.f;
        }
      }
      if (tid < KB) sm.bias[tid] = (sg.kind == 1 && k0 + tid < sg.len) ? slot_b[k0 + tid] : 0.f;
      __syncthreads();
      // waves whose queries all precede this block of the current chunk skip it
      if (sg.kind == 3 && k0 > qb_off + wave_qmax) continue;

      // ---- S^T[key][q] = K . Q^T
      f32x16 s = zero16();
      if constexpr (St<T>::is_bf16) {
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
          const u16x8 av = *reinterpret_cast<const u16x8*>(sK + n * sm.KS + 16 * ks + 8 * h);
          mma_bf16(s, av, qf.v[ks]);
        }
      } else {
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(s, sK[n * sm.KS + 2 * ks + h], qf.v[ks]);
      }
      float bm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = d_row(lane, r);
        const int kidx = k0 + kr;
        float x = a.score_round ? St<T>::rnd(s[r]) : s[r];
        x = mul_rn(x, scale);
        if (sg.kind == 1) x = add_rn(x, sm.bias[kr]);
        bool ok = kidx < sg.len;
        if (sg.kind == 3) ok = ok && kidx <= qb_off + qi;
        x = ok ? x : -INFINITY;
        s[r] = x;
        bm = fmaxf(bm, x);
      }
      bm = fmaxf(bm, xor32(bm));
      const float m_new = fmaxf(m_run, bm);
      const float alpha = m_new == -INFINITY ? 1.f : expf(m_run - m_new);
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = m_new == -INFINITY ? 0.f : expf(s[r] - m_new);
        s[r] = p;
        ps += p;
      }
      ps += xor32(ps);
      l_run = l_run * alpha + ps;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      // ---- O^T[d][q] += V^T . P^T
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int d = 32 * db + n;
        if constexpr (St<T>::is_bf16) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            u16x8 av, pv;
            const u16x4 lo = *reinterpret_cast<const u16x4*>(sV + d * sm.VS + 16 * kc + 4 * h);
            const u16x4 hi = *reinterpret_cast<const u16x4*>(sV + d * sm.VS + 16 * kc + 8 + 4 * h);
#pragma unroll
            for (int i = 0; i < 4; ++i) { av[i] = lo[i]; av[4 + i] = hi[i]; }
#pragma unroll
            for (int i = 0; i < 8; ++i) pv[i] = f2bf(s[8 * kc + i]);
            mma_bf16(o[db], av, pv);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) mma_f32(o[db], sV[d * sm.VS + d_row(lane, r)], s[r]);
        }
      }
    }
  }

  // ---- normalise; y = round(O)
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  if (a.mode == 0 && a.lse && qok && h == 0) a.lse[((long long)b * a.H + hq) * a.n_q + t] = m_run + logf(l_run);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = St<T>::rnd(o[db][r] * inv_l);

  // ---- readout: eta * RMSNorm(normalize(q_raw) . M * (1-gamma)/sqrt(HD))
  const float* M = nullptr;
  if (a.m_res && step >= 0) M = a.m_res + (long long)step * a.m_step + (long long)bh * HD * HD;
  if (a.mode == 1 && a.m_res) M = a.m_res + (long long)bh * HD * HD;
  if (M) {
    __syncthreads();
    if constexpr (St<T>::is_bf16) {
      uint16_t* mh = sm.mhi();
      uint16_t* ml = sm.mlo();
      if (a.m_split) {
        // already M^T split into bf16 hi / lo: straight 16-byte copies
        const uint16_t* src = reinterpret_cast<const uint16_t*>(M);
        for (int it = tid; it < 2 * HD * (HD / 8); it += nthreads) {
          const int part = it / (HD * (HD / 8)), rem = it % (HD * (HD / 8));
          const int d = rem / (HD / 8), c8 = (rem % (HD / 8)) * 8;
          *reinterpret_cast<u16x8*>((part ? ml : mh) + d * sm.MS + c8) =
              *reinterpret_cast<const u16x8*>(src + part * HD * HD + d * HD + c8);
        }
      } else {
        for (int it = tid; it < HD * HD; it += nthreads) {
          const int c = it / HD, d = it % HD;  // M[c][d] -> M^T[d][c]
          const float x = M[it];
          const uint16_t hb = f2bf(x);
          mh[d * sm.MS + c] = hb;
          ml[d * sm.MS + c] = f2bf(x - bf2f(hb));
        }
      }
    } else {
      float* mf = sm.mf();
      for (int it = tid; it < HD * HD; it += nthreads) mf[(it / HD) * sm.MF + it % HD] = M[it];
    }
    __syncthreads();
    const T* rrow = reinterpret_cast<const T*>(a.q_raw) + b * a.q_sb + hq * a.q_sh + (long long)t * HD;
    QFrag<T, HD> rf;
    rf.load(rrow, qok, h);
    float qq = rf.sumsq();
    qq += xor32(qq);
    const float inv_q = 1.0f / fmaxf(sqrtf(qq), 1e-12f);
    const float coef = div_rn(1.0f - a.gamma[hkv], sqrtf((float)HD));
    f32x16 rr[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      rr[db] = zero16();
      const int d = 32 * db + n;
      if constexpr (St<T>::is_bf16) {
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
          const u16x8 ah = *reinterpret_cast<const u16x8*>(sm.mhi() + d * sm.MS + 16 * ks + 8 * h);
          const u16x8 al = *reinterpret_cast<const u16x8*>(sm.mlo() + d * sm.MS + 16 * ks + 8 * h);
          mma_bf16(rr[db], ah, rf.v[ks]);
          mma_bf16(rr[db], al, rf.v[ks]);
        }
      } else {
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(rr[db], sm.mf()[(2 * ks + h) * sm.MF + d], rf.v[ks]);
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float y = mul_rn(rr[db][r] * inv_q, coef);
        rr[db][r] = y;
        ss += y * y;
      }
    ss += xor32(ss);
    const float rs = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
    const float eta = qok ? a.eta[b * a.e_sb + hq * a.e_sh + t] : 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * db + d_row(lane, r);
        const float ymn = mul_rn(mul_rn(rr[db][r], rs), a.res_w[d]);
        o[db][r] = St<T>::rnd(add_rn(o[db][r], St<T>::rnd(mul_rn(eta, ymn))));
      }
  }

  // ---- write y[b][t][hq][d]
  if (qok) {
    T* yrow = reinterpret_cast<T*>(a.y) + b * a.y_sb + (long long)t * a.y_st + hq * HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) yrow[32 * db + d_row(lane, r)] = St<T>::from_f(o[db][r]);
  }
}

// ----------------------------------------------------------------- forward, bf16

// Forward (mode 0) with bf16 storage.  Workgroup = (query tile of 32*QW, chunk, bh) with
// G*QW wavefronts as above.  The keys of a chunk are walked as 32-key blocks:
//   [sink block | S/32 slot blocks | C/32 previous-chunk blocks | current-chunk blocks up to
//    the tile's last query]
// with one barrier per block: the next block is loaded into registers while the current one
// is multiplied, then written to the other LDS buffer (K rows and V^T columns).  Softmax is
// online in base 2 (x*log2e folded into one FMA).  The M_res readout stages M^T (bf16 hi/lo)
// in two halves of the feature rows through the same LDS.
template <int HD>
struct FwdSmem {
  static constexpr int KS = HD + 8;              // K row stride
  static constexpr int VS = KB + 8;              // V^T row stride
  static constexpr int MS = HD + 8;              // M^T row stride
  static constexpr int KV = KB * KS + HD * VS;   // elements of one K/V buffer
  static constexpr int MH = (HD / 2) * MS;       // elements of one M^T half (hi or lo)
  static constexpr int RAW = 2 * KV > 2 * MH ? 2 * KV : 2 * MH;
  alignas(16) uint16_t raw[RAW];
  float bias[2][KB];
  __device__ uint16_t* k(int buf) { return raw + buf * KV; }
  __device__ uint16_t* vt(int buf) { return raw + buf * KV + KB * KS; }
};

// Block i of the schedule: key rows, number of valid keys, slot bias row, causal offset.
struct FwdBlock {
  const uint16_t* k;
  const uint16_t* v;
  const float* bias;   // null: no bias
  int nvalid;
  int kpos;            // current-chunk block: index of its first key within the chunk; else -1
};

template <int HD, int IPT>
__global__ void __launch_bounds__(512) attn_fwd_kernel(b3_attn_args a, int QW) {
  using Sm = FwdSmem<HD>;
  __shared__ Sm sm;
  constexpr int NDB = HD / 32;
  constexpr int ITEMS = KB * (HD / 8);
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int nthreads = blockDim.x;
  const int g = wave / QW, qsub = wave % QW;
  const int bh = blockIdx.z, b = bh / a.HKV, hkv = bh % a.HKV;
  const int hq = hkv * G + g;
  const int part = a.part;                       // 0 all fields, 1 sinks + window, 2 slots (chunks >= 2)
  const int chunk = blockIdx.y + a.chunk_begin, C = a.C;   // the launcher sets chunk_begin
  const int qbase = chunk * C;
  const int nq_chunk = min(C, a.n_q - qbase);
  const int qt0 = blockIdx.x * 32 * QW;
  if (qt0 >= nq_chunk) return;                  // uniform across the workgroup
  const int qi = qt0 + 32 * qsub + n;           // this lane's query within the chunk
  const bool qok = qi < nq_chunk;
  const int t = qbase + qi;
  const int wave_q0 = qt0 + 32 * qsub;
  const int wg_qend = min(qt0 + 32 * QW, nq_chunk);
  const int step = chunk - 2;
  const float L2E = 1.4426950408889634f;
  const float scale = 1.0f / sqrtf((float)HD);
  const float sL = scale * L2E;

  // ---- block schedule
  const long long wofs = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const uint16_t* wk = reinterpret_cast<const uint16_t*>(a.win_k) + wofs;
  const uint16_t* wv = reinterpret_cast<const uint16_t*>(a.win_v) + wofs;
  const int n_sink = (chunk >= 2 && part != 2) ? 1 : 0;
  const int n_slot = (chunk >= 2 && part != 1) ? (a.S + KB - 1) / KB : 0;
  const int n_pre = n_sink + n_slot;
  const int n_prev = (chunk >= 1 && part != 2) ? (C + KB - 1) / KB : 0;
  const int n_cur = part != 2 ? (wg_qend + KB - 1) / KB : 0;
  const int nb = n_pre + n_prev + n_cur;
  const bool keep_partial = part == 1 && chunk >= 2;   // the slot field follows in part 2
  float* pq = a.partial ? a.partial + (((long long)b * a.H + hq) * a.n_q + t) * (HD + 4) : nullptr;
  auto block = [&](int i) -> FwdBlock {
    FwdBlock f;
    f.bias = nullptr;
    f.kpos = -1;
    if (i < n_pre) {
      if (i < n_sink) {
        f.k = wk;
        f.v = wv;
        f.nvalid = min(a.n_sinks, C);
      } else {
        const int j = i - n_sink;
        const long long so = (long long)step * a.slot_step + (long long)bh * a.S * HD + (long long)j * KB * HD;
        f.k = reinterpret_cast<const uint16_t*>(a.slot_k) + so;
        f.v = reinterpret_cast<const uint16_t*>(a.slot_v) + so;
        f.bias = a.slot_bias + (long long)step * (a.slot_step / HD) + (long long)bh * a.S + j * KB;
        f.nvalid = min(KB, a.S - j * KB);
      }
    } else if (i < n_pre + n_prev) {
      const int j = i - n_pre;
      const long long o = ((long long)(chunk - 1) * C + j * KB) * HD;
      f.k = wk + o;
      f.v = wv + o;
      f.nvalid = min(KB, C - j * KB);
    } else {
      const int j = i - n_pre - n_prev;
      const long long o = ((long long)qbase + j * KB) * HD;
      f.k = wk + o;
      f.v = wv + o;
      f.nvalid = min(KB, nq_chunk - j * KB);
      f.kpos = j * KB;
    }
    return f;
  };

  // ---- staging registers: IPT 16-byte K pieces per thread (rows in order); V^T is staged by
  // key pairs (keys 2p, 2p+1 at 8 features: 8 dword writes of two bf16 each; the lanes of a
  // wavefront take consecutive pairs, so the writes fall into distinct banks); plus one bias
  // value in log2 units
  constexpr int VITEMS = (KB / 2) * (HD / 8);
  u16x8 rk[IPT], rv0[IPT], rv1[IPT];
  float rb = 0.f;
  auto load = [&](int i) {
    const FwdBlock f = block(i);
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
      const int it = tid + q * nthreads;
      const int r = it / (HD / 8), c8 = (it % (HD / 8)) * 8;
      if (it < ITEMS && r < f.nvalid) rk[q] = *reinterpret_cast<const u16x8*>(f.k + (long long)r * HD + c8);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) rk[q][e] = 0;
      }
      const int pr = it % (KB / 2), vc8 = (it / (KB / 2)) * 8;
      if (it < VITEMS && 2 * pr < f.nvalid) rv0[q] = *reinterpret_cast<const u16x8*>(f.v + (long long)(2 * pr) * HD + vc8);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) rv0[q][e] = 0;
      }
      if (it < VITEMS && 2 * pr + 1 < f.nvalid)
        rv1[q] = *reinterpret_cast<const u16x8*>(f.v + (long long)(2 * pr + 1) * HD + vc8);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) rv1[q][e] = 0;
      }
    }
    rb = (tid < KB && f.bias && tid < f.nvalid) ? f.bias[tid] * L2E : 0.f;
  };
  auto store = [&](int buf) {
    uint16_t* sK = sm.k(buf);
    uint16_t* sV = sm.vt(buf);
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
      const int it = tid + q * nthreads;
      if (it < ITEMS) {
        const int r = it / (HD / 8), c8 = (it % (HD / 8)) * 8;
        *reinterpret_cast<u16x8*>(sK + r * Sm::KS + c8) = rk[q];
      }
      if (it < VITEMS) {
        const int pr = it % (KB / 2), vc8 = (it / (KB / 2)) * 8;
        // key k sits at column (k & ~15) + 4*[0,2,1,3][(k >> 2) & 3] + (k & 3): the 8 keys
        // 16kc + {4h..4h+3, 8+4h..8+4h+3} of MFMA lane group h are then 8 contiguous columns
        const int k0 = 2 * pr, qd = (k0 >> 2) & 3;
        const int col = (k0 & ~15) + 4 * ((qd == 1) ? 2 : (qd == 2) ? 1 : qd) + (k0 & 3);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<uint32_t*>(sV + (vc8 + e) * Sm::VS + col) = (uint32_t)rv0[q][e] | ((uint32_t)rv1[q][e] << 16);
      }
    }
    if (tid < KB) sm.bias[buf][tid] = rb;
  };

  const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q_rope) + b * a.q_sb + hq * a.q_sh + (long long)t * HD;
  QFrag<uint16_t, HD> qf;
  qf.load(qrow, qok, h);
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  if (part == 2 && qok) {
    // online-softmax state left by part 1: lane half h holds features 64h.. in (db, r) order
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float4 q4 = *reinterpret_cast<const float4*>(pq + h * (HD / 2) + 16 * db + 4 * r4);
        o[db][4 * r4 + 0] = q4.x;
        o[db][4 * r4 + 1] = q4.y;
        o[db][4 * r4 + 2] = q4.z;
        o[db][4 * r4 + 3] = q4.w;
      }
    m_run = pq[HD];
    l_run = pq[HD + 1];
  }

  load(0);
  store(0);
  sync_lds();
  for (int i = 0; i < nb; ++i) {
    const int buf = i & 1;
    if (i + 1 < nb) load(i + 1);
    const FwdBlock f = block(i);
    // a wave whose queries all precede the block's first key skips it
    if (!(f.kpos >= 0 && f.kpos > wave_q0 + 31)) {
      const uint16_t* sK = sm.k(buf);
      const uint16_t* sV = sm.vt(buf);
      f32x16 s = zero16();
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) {
        const u16x8 av = *reinterpret_cast<const u16x8*>(sK + n * Sm::KS + 16 * ks + 8 * h);
        mma_bf16(s, av, qf.v[ks]);
      }
      // scores in log2 units: round_bf(q.k) * scale*log2(e) (+ slot bias * log2(e)), one FMA
      float bm = -INFINITY;
      if (f.bias) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const float4 b4 = *reinterpret_cast<const float4*>(&sm.bias[buf][8 * r4 + 4 * h]);
          const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) s[4 * r4 + q] = fmaf(round_bf(s[4 * r4 + q]), sL, bb[q]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = round_bf(s[r]) * sL;
      }
      if (f.kpos >= 0 || f.nvalid < KB) {
        // valid keys of this lane's query: kr <= lim
        const int lim = min(f.nvalid - 1, f.kpos >= 0 ? qi - f.kpos : KB - 1);
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = d_row(lane, r) <= lim ? s[r] : -INFINITY;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) bm = fmaxf(bm, s[r]);
      bm = fmaxf(bm, xor32(bm));
      // the running max moves only when it grows by more than 2^8 (probabilities up to 2^8
      // before the final normalisation are exact enough in fp32 and rescale-free)
      const bool grow = bm > m_run + 8.0f;
      const float m_use = grow ? bm : m_run;
      {
        // a lane whose keys so far are all masked keeps m = -inf: p = 0 and alpha = 0 for it
        const float mu = m_use == -INFINITY ? 0.f : m_use;
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[r] - mu);
          s[r] = p;
          ps += p;
        }
        ps += xor32(ps);
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float alpha = __builtin_amdgcn_exp2f(m_run - mu);   // m_run = -inf: alpha = 0
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
          l_run *= alpha;
        }
        l_run += ps;
        m_run = m_use;
        u16x8 pv[2];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int e = 0; e < 8; ++e) pv[kc][e] = f2bf(s[8 * kc + e]);
        // ---- O^T[d][q] += V^T . P^T
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const int d = 32 * db + n;
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            mma_bf16(o[db], *reinterpret_cast<const u16x8*>(sV + d * Sm::VS + 16 * kc + 8 * h), pv[kc]);
        }
      }
    }
    if (i + 1 < nb) store(buf ^ 1);
    sync_lds();
  }

  if (keep_partial) {
    if (qok) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(pq + h * (HD / 2) + 16 * db + 4 * r4) =
              make_float4(o[db][4 * r4], o[db][4 * r4 + 1], o[db][4 * r4 + 2], o[db][4 * r4 + 3]);
      if (h == 0) {
        pq[HD] = m_run;
        pq[HD + 1] = l_run;
      }
    }
    return;
  }

  // ---- normalise; y = round(O)
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  if (a.lse && qok && h == 0) a.lse[((long long)b * a.H + hq) * a.n_q + t] = (m_run + log2f(l_run)) / L2E;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = round_bf(o[db][r] * inv_l);

  // ---- readout: eta * RMSNorm(normalize(q_raw) . M * (1-gamma)/sqrt(HD)), M^T staged by halves
  if (a.m_res && step >= 0) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(a.m_res + (long long)step * a.m_step) +
                          (long long)bh * 2 * HD * HD;   // bf16 M^T hi, then lo (HD*HD floats of room)
    const uint16_t* rrow = reinterpret_cast<const uint16_t*>(a.q_raw) + b * a.q_sb + hq * a.q_sh + (long long)t * HD;
    QFrag<uint16_t, HD> rf;
    rf.load(rrow, qok, h);
    float qq = rf.sumsq();
    qq += xor32(qq);
    const float inv_q = 1.0f / fmaxf(sqrtf(qq), 1e-12f);
    const float coef = div_rn(1.0f - a.gamma[hkv], sqrtf((float)HD));
    f32x16 rr[NDB];
    uint16_t* mh = sm.raw;
    uint16_t* ml = sm.raw + Sm::MH;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (p > 0) sync_lds();
      for (int it = tid; it < 2 * (HD / 2) * (HD / 8); it += nthreads) {
        const int part = it / ((HD / 2) * (HD / 8)), rem = it % ((HD / 2) * (HD / 8));
        const int dr = rem / (HD / 8), c8 = (rem % (HD / 8)) * 8;
        *reinterpret_cast<u16x8*>((part ? ml : mh) + dr * Sm::MS + c8) =
            *reinterpret_cast<const u16x8*>(src + part * HD * HD + (long long)((HD / 2) * p + dr) * HD + c8);
      }
      sync_lds();
#pragma unroll
      for (int dh = 0; dh < NDB / 2; ++dh) {
        const int db = (NDB / 2) * p + dh;
        rr[db] = zero16();
        const int dr = 32 * dh + n;
#pragma unroll
        for (int ks = 0; ks < HD / 16; ++ks) {
          const u16x8 ah = *reinterpret_cast<const u16x8*>(mh + dr * Sm::MS + 16 * ks + 8 * h);
          const u16x8 al = *reinterpret_cast<const u16x8*>(ml + dr * Sm::MS + 16 * ks + 8 * h);
          mma_bf16(rr[db], ah, rf.v[ks]);
          mma_bf16(rr[db], al, rf.v[ks]);
        }
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float y = mul_rn(rr[db][r] * inv_q, coef);
        rr[db][r] = y;
        ss += y * y;
      }
    ss += xor32(ss);
    const float rs = 1.0f / sqrtf(div_rn(ss, (float)HD) + a.eps);
    const float eta = qok ? a.eta[b * a.e_sb + hq * a.e_sh + t] : 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * db + d_row(lane, r);
        const float ymn = mul_rn(mul_rn(rr[db][r], rs), a.res_w[d]);
        o[db][r] = round_bf(add_rn(o[db][r], round_bf(mul_rn(eta, ymn))));
      }
  }

  // ---- write y[b][t][hq][d], 4 consecutive features per store
  if (qok) {
    uint16_t* yrow = reinterpret_cast<uint16_t*>(a.y) + b * a.y_sb + (long long)t * a.y_st + hq * HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        u16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = f2bf(o[db][4 * r4 + e]);
        *reinterpret_cast<u16x4*>(yrow + 32 * db + 8 * r4 + 4 * h) = w;
      }
  }
}

// ---------------------------------------------------------------- bf16 forward, DMA staging
//
// The same attention for the forward (mode 0, all key fields, bf16), with the K and V tiles
// brought into LDS by global->LDS loads (global_load_lds_dwordx4), so that no staging goes
// through registers.  Blocks go in pairs: one barrier per pair, and the QK products of a
// pair's second block are issued before the softmax of its first, so that the softmax runs
// beside MFMA work.  The ring has NPS pair slots.  Three (one eight-wavefront workgroup per
// CU): while pair p is computed, pair p + 1 is in flight and pair p + 2 is issued into the
// slot pair p - 1 has left.  Two (74 KB of LDS, two four-wavefront workgroups per CU, each
// covering the other's load waits, start and readout): pair p + 1 is issued at pair p's
// barrier into the slot pair p - 1 has left.  A
// tile is stored as blocks of 8 rows x 8 sixteen-byte pieces (one global->LDS instruction each:
// 8 whole 128-byte row segments), piece-major inside a block and 128 bytes of padding between
// blocks (f2_off below).  Every operand read of the loop is then a per-lane base plus a
// compile-time offset (no address arithmetic per read), the K reads (ds_read_b128) are
// conflict-free and the transposed V reads take the minimum two LDS cycles.  The V operand of
// O^T = V^T P^T is read with ds_read_b64_tr_b16, which transposes 16-bit elements across lanes,
// so V needs no transpose when staged.  The M_res snapshot (M^T bf16 hi / lo) comes by the same
// loads into pair slots the last pair leaves free.  Three slots: hi at the barrier before the
// last pair, lo at the last barrier.  Two: hi at the last barrier, lo once every wavefront is
// done with the last pair.
template <int HD, int NPS>
struct Fwd2Smem {
  static constexpr int TILEB = (HD / 64) * (KB / 8) * F2_BLK;   // bytes of one K or V tile
  static_assert(4 * TILEB >= 2 * HD * HD, "an M^T half fits in one pair slot");
  alignas(16) unsigned char ring[2 * NPS][2][TILEB];
  alignas(16) float sbias[128];          // slot bias row of the step (log2 units)
  alignas(16) float resw[128];           // res_norm weight
};


template <int HD, int NW, int NPS, bool SR>
__global__ void __launch_bounds__(64 * NW, NPS == 2 ? 2 : 1) attn_fwd2_kernel(b3_attn_args a, int QW) {
  static_assert(NPS == 2 || NPS == 3, "two or three pair slots");
  using Sm = Fwd2Smem<HD, NPS>;
  __shared__ Sm sm;
  constexpr int NDB = HD / 32, NP = HD / 8;
  constexpr int RPI = 1024 / (2 * HD);              // tile rows per 1 KB load instruction
  constexpr int IPT = KB / RPI;                     // load instructions per tile
  constexpr int LPB = 2 * IPT / NW;                 // per wave per block (K and V)
  static_assert(LPB * NW == 2 * IPT, "tile loads must divide over the waves");
  constexpr int MIPT = HD / RPI;                    // instructions per M^T half (hi or lo)
  constexpr int LPMH = MIPT / NW;                   // per wave per M^T half
  static_assert(LPMH * NW == MIPT, "M^T loads must divide over the waves");
  const int G = a.H / a.HKV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int g = wave / QW, qsub = wave % QW;
  // XCD-aware order: the query tiles and neighbouring chunks of one bh, which read the same
  // key/value tiles and snapshots, share one XCD's L2
  const GridPos gp = xcd_grid_pos();
  const int bx = gp.x, by = gp.y, bh = gp.z, b = bh / a.HKV, hkv = bh % a.HKV;
  const int hq = hkv * G + g;
  const int chunk = by + a.chunk_begin, C = a.C;
  const int qbase = chunk * C;
  const int nq_chunk = min(C, a.n_q - qbase);
  const int qt0 = bx * 32 * QW;
  if (qt0 >= nq_chunk) return;                  // uniform across the workgroup
  const int qi = qt0 + 32 * qsub + n;
  const bool qok = qi < nq_chunk;
  const int t = qbase + qi;
  const int wave_q0 = qt0 + 32 * qsub;
  const int wg_qend = min(qt0 + 32 * QW, nq_chunk);
  const int step = chunk - 2;
  const float L2E = 1.4426950408889634f;
  const float sL = (1.0f / sqrtf((float)HD)) * L2E;

  // ---- block schedule: [sinks | slots (step c-2) | previous chunk | current chunk (causal)]
  const long long wofs = (long long)b * a.w_sb + (long long)hkv * a.w_sh;
  const uint16_t* wk = reinterpret_cast<const uint16_t*>(a.win_k) + wofs;
  const uint16_t* wv = reinterpret_cast<const uint16_t*>(a.win_v) + wofs;
  const bool has_slots = chunk >= 2;
  const int n_sink = has_slots ? 1 : 0;
  const int n_slot = has_slots ? (a.S + KB - 1) / KB : 0;
  const int n_pre = n_sink + n_slot;
  const int n_prev = chunk >= 1 ? (C + KB - 1) / KB : 0;
  const int n_cur = (wg_qend + KB - 1) / KB;
  const int nb = n_pre + n_prev + n_cur;
  auto block = [&](int i) -> FwdBlock {
    FwdBlock f;
    f.bias = nullptr;
    f.kpos = -1;
    if (i < n_pre) {
      if (i < n_sink) {
        f.k = wk;
        f.v = wv;
        f.nvalid = min(a.n_sinks, C);
      } else {
        const int j = i - n_sink;
        const long long so = (long long)step * a.slot_step + (long long)bh * a.S * HD + (long long)j * KB * HD;
        f.k = reinterpret_cast<const uint16_t*>(a.slot_k) + so;
        f.v = reinterpret_cast<const uint16_t*>(a.slot_v) + so;
        f.bias = sm.sbias + j * KB;
        f.nvalid = min(KB, a.S - j * KB);
      }
    } else if (i < n_pre + n_prev) {
      const int j = i - n_pre;
      const long long o = ((long long)(chunk - 1) * C + j * KB) * HD;
      f.k = wk + o;
      f.v = wv + o;
      f.nvalid = min(KB, C - j * KB);
    } else {
      const int j = i - n_pre - n_prev;
      const long long o = ((long long)qbase + j * KB) * HD;
      f.k = wk + o;
      f.v = wv + o;
      f.nvalid = min(KB, nq_chunk - j * KB);
      f.kpos = j * KB;
    }
    return f;
  };
  // this wave's share of the tile loads of block i into stage st; rows past the valid ones
  // repeat the last valid row (their scores are masked)
  auto issue = [&](int i, int st) {
    const FwdBlock f = block(i);
    const int last = max(f.nvalid - 1, 0);
#pragma unroll
    for (int q = 0; q < LPB; ++q) {
      const int ins = wave * LPB + q;
      const int tile = ins / IPT, ch = ins % IPT;     // block ch = (piece group, row group)
      const int r = 8 * (ch % (KB / 8)) + (lane & 7), p = 8 * (ch / (KB / 8)) + (lane >> 3);
      lds_dma16((tile ? f.v : f.k) + (long long)min(r, last) * HD + 8 * p, sm.ring[st][tile] + ch * F2_BLK);
    }
  };
  const bool readout = a.m_res && step >= 0;
  // M^T half (0: hi, 1: lo) into pair slot ps
  auto issue_mhalf = [&](int half, int ps) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(a.m_res + (long long)step * a.m_step) +
                          (long long)bh * 2 * HD * HD + (long long)half * HD * HD;   // bf16 M^T hi, then lo
    uint16_t* dst = reinterpret_cast<uint16_t*>(sm.ring[2 * ps][0]);   // 2 HD^2 bytes, row-major
#pragma unroll
    for (int q = 0; q < LPMH; ++q) {
      const int ch = wave * LPMH + q;
      const int r = ch * RPI + lane / NP, p = (lane % NP) ^ (r % NP);
      lds_dma16(src + (long long)r * HD + 8 * p, dst + ch * 512);
    }
  };
  const int npair = (nb + 1) / 2, P = npair - 1;
  // this wave's loads of pair q, and the stages of its blocks (pair slot q % NPS)
  auto issue_pair = [&](int q) {
    issue(2 * q, 2 * (q % NPS));
    if (2 * q + 1 < nb) issue(2 * q + 1, 2 * (q % NPS) + 1);
  };

  // ---- prologue: the slot bias row, the res_norm weight and the query fragment into
  // registers, pairs 0 and 1 into LDS; the bias and weight go to LDS after the tile loads are
  // issued (in-order completion makes every later wait cover the loads issued before it)
  const float sb = (has_slots && tid < 128)
                       ? a.slot_bias[(long long)step * (a.slot_step / HD) + (long long)bh * a.S + tid] : 0.f;
  const float rw = tid < HD ? a.res_w[tid] : 0.f;
  const bool fuse_q = a.q_lin != nullptr;   // the q head preparation done here
  QFrag<uint16_t, HD> qf;
  QPrep<HD> qp;
  const int t_valid = qok ? t : qbase + nq_chunk - 1;
  if (fuse_q) {
    QPrep<HD>::fetch_row(qf, a, b, hq, t_valid, h);
    qp.fetch_w(a, h);
    qp.fetch_cs(a, t_valid, h);
  } else {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q_rope) + b * a.q_sb + hq * a.q_sh + (long long)t * HD;
    qf.load(qrow, qok, h);
  }
  issue_pair(0);
  if constexpr (NPS == 3) {
    if (P >= 1) issue_pair(1);
    if (P == 0 && readout) issue_mhalf(0, 1);
  }
  if (tid < 128) lds_write_f32(&sm.sbias[tid], sb * L2E);   // bias in log2 units
  if (tid < HD) lds_write_f32(&sm.resw[tid], rw);
  float q_r = 1.f;   // the rows' RMS factor, kept for the readout's q_raw
  if (fuse_q) {
    float x[HD / 16][8];
    QPrep<HD>::unpack(qf, x);
    if (a.qn_w) {
      q_r = QPrep<HD>::rms_factor(x, a.qn_eps);
      qp.scale(x, q_r);
    }
    qp.rope(qf, x);
  }

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = zero16();
  float m_run = -INFINITY, l_run = 0.f;

  // S^T = K Q^T of the block in stage st
  // (row n, piece 2 ks + h) of a staged tile is at f2_off(n, h) + f2_off(0, 2 ks)
  const int lane_k = f2_off(n, h);
  auto qk = [&](int st) -> f32x16 {
    const unsigned char* sK = sm.ring[st][0] + lane_k;
    f32x16 sc = zero16();
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks)
      mma_bf16(sc, *reinterpret_cast<const u16x8*>(sK + f2_off(0, 2 * ks)), qf.v[ks]);
    return sc;
  };
  // the lane's V^T operand base: row r1 = 4h + jv/4 (+8, +16, +24 at compile-time offsets),
  // elements 32 db + 16 (grp & 1) + 4 (jv & 3) .. +3 of the row (piece 4 db + c, half jv & 1)
  const int jv = lane & 15, grp = lane >> 4;
  const uint32_t lane_v = f2_off(4 * h + (jv >> 2), 2 * (grp & 1) + ((jv >> 1) & 1)) + 8 * (jv & 1);
  // softmax step and O^T += V^T P^T for block f in stage st, scores sc
  auto attend = [&](f32x16 sc, const FwdBlock& f, int st) {
    const uint32_t vb = lds_addr(sm.ring[st][1]) + lane_v;
    // scores in log2 units: round_bf(q.k) * scale*log2(e) + slot bias * log2(e), one FMA for
    // every block (bias 0 outside the slot field), so that every block takes the same
    // instructions.  SR = false skips the rounding (fp32 scores, as the decoder step computes them).
    fx4 b4[4];
    if (f.bias) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) b4[r4] = lds_read_f4_nowait(f.bias + 8 * r4 + 4 * h);
      lds_wait4(b4[0], b4[1], b4[2], b4[3]);
    } else {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) b4[r4] = fx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      float x[4] = {sc[4 * r4], sc[4 * r4 + 1], sc[4 * r4 + 2], sc[4 * r4 + 3]};
      if constexpr (SR) {
        const uint32_t u0 = pack_bf2(x[0], x[1]), u1 = pack_bf2(x[2], x[3]);
        x[0] = bf_lo(u0);
        x[1] = bf_hi(u0);
        x[2] = bf_lo(u1);
        x[3] = bf_hi(u1);
      }
      sc[4 * r4] = fmaf(x[0], sL, b4[r4].x);
      sc[4 * r4 + 1] = fmaf(x[1], sL, b4[r4].y);
      sc[4 * r4 + 2] = fmaf(x[2], sL, b4[r4].z);
      sc[4 * r4 + 3] = fmaf(x[3], sL, b4[r4].w);
    }
    // masks: rows past the valid keys, and the causal diagonal (a current-chunk block wholly
    // before the wave's first query needs none)
    if (f.nvalid < KB || (f.kpos >= 0 && f.kpos + KB - 1 > wave_q0)) {
      const int lim = min(f.nvalid - 1, f.kpos >= 0 ? qi - f.kpos : KB - 1);
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = d_row(lane, r) <= lim ? sc[r] : -INFINITY;
    }
    // the first half of this block's V^T operand, read while the softmax runs
    u16x4 tv0[8];
    f2_vreads<NDB, 0>(tv0, vb);
    float bm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) bm = fmaxf(bm, sc[r]);
    bm = pair_max32(bm);
    // the running max moves only when it grows by more than 2^8 (probabilities up to 2^8
    // before the final normalisation are exact enough in fp32 and rescale-free)
    const bool grow = bm > m_run + 8.0f;
    const float m_use = grow ? bm : m_run;
    const float mu = m_use == -INFINITY ? 0.f : m_use;   // all keys so far masked: p = 0
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = __builtin_amdgcn_exp2f(sc[r] - mu);
      sc[r] = p;
      ps += p;
    }
    ps = pair_sum32(ps);
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - mu);   // m_run = -inf: alpha = 0
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      l_run *= alpha;
    }
    l_run += ps;
    m_run = m_use;
    u16x8 pv[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[kc][e] = f2bf(sc[8 * kc + e]);
    // ---- O^T[d][q] += V^T . P^T
    {
      lds_wait8(tv0);
      u16x4 tv1[8];
      f2_vreads<NDB, 1>(tv1, vb);
#pragma unroll
      for (int db = 0; db < NDB && db < 4; ++db) {
        u16x8 av;
#pragma unroll
        for (int e = 0; e < 4; ++e) { av[e] = tv0[2 * db][e]; av[4 + e] = tv0[2 * db + 1][e]; }
        mma_bf16(o[db], av, pv[0]);
      }
      lds_wait8(tv1);
#pragma unroll
      for (int db = 0; db < NDB && db < 4; ++db) {
        u16x8 av;
#pragma unroll
        for (int e = 0; e < 4; ++e) { av[e] = tv1[2 * db][e]; av[4 + e] = tv1[2 * db + 1][e]; }
        mma_bf16(o[db], av, pv[1]);
      }
    }
  };

  for (int pr = 0; pr < npair; ++pr) {
    // wait for pair pr while pair pr + 1 (or, at the last pair, the M^T hi half) may still be
    // in flight (three slots; with two, nothing is issued after pair pr before its barrier)
    if constexpr (NPS == 3) {
      if (pr < P) {
        if (2 * pr + 3 < nb) wait_vm<2 * LPB>();
        else wait_vm<LPB>();
      } else if (readout) {
        wait_vm<LPMH>();
      } else {
        wait_vm<0>();
      }
    } else {
      wait_vm<0>();
    }
    sync_lds();   // pair pr is in LDS; every wave is done with pair pr - 1
    if constexpr (NPS == 3) {
      if (pr + 2 <= P) issue_pair(pr + 2);
      if (readout) {
        if (pr == P - 1) issue_mhalf(0, (P + 1) % 3);
        if (pr == P) issue_mhalf(1, (P + 2) % 3);
      }
    } else {
      if (pr + 1 <= P) issue_pair(pr + 1);
      if (readout && pr == P) issue_mhalf(0, (P + 1) % 2);
    }
    const int i0 = 2 * pr, i1 = 2 * pr + 1;
    const FwdBlock f0 = block(i0);
    const bool do0 = !(f0.kpos >= 0 && f0.kpos > wave_q0 + 31);   // the wave's queries all precede the block
    const bool has1 = i1 < nb;
    const FwdBlock f1 = block(has1 ? i1 : i0);
    const bool do1 = has1 && !(f1.kpos >= 0 && f1.kpos > wave_q0 + 31);
    const int st0 = 2 * (pr % NPS);
    // both blocks' products unconditionally (a block the wave skips, or the stage of a missing
    // second block, gives a tile that is never used), so that no register tile is merged
    // across branches (each merge would be a 16-register copy)
    f32x16 sc0 = qk(st0), sc1 = qk(st0 + 1);
    if (do0) attend(sc0, f0, st0);
    if (do1) attend(sc1, f1, st0 + 1);
  }

  // ---- the readout's global loads first (the q_raw fragment, eta), so that their latency
  // overlaps the normalisation and the barrier before the readout
  QFrag<uint16_t, HD> rf;
  float eta = 0.f;
  if constexpr (NPS == 2) {
    if (readout) {
      sync_lds();   // every wave is done with the last pair: its slot takes the M^T lo half
      issue_mhalf(1, P % 2);
    }
  }
  if (readout) {
    if (fuse_q) {
      QPrep<HD>::fetch_row(rf, a, b, hq, t_valid, h);
      eta = qok ? eta_from_gates(a, b, hq, t) : 0.f;
    } else {
      const uint16_t* rrow = reinterpret_cast<const uint16_t*>(a.q_raw) + b * a.q_sb + hq * a.q_sh + (long long)t * HD;
      rf.load(rrow, qok, h);
      eta = qok ? a.eta[b * a.e_sb + hq * a.e_sh + t] : 0.f;
    }
  }

  // ---- normalise; y = round(O), kept as bf16 pairs (features d_row(lane, 2j), +1)
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
  if (a.lse && qok && h == 0) a.lse[((long long)b * a.H + hq) * a.n_q + t] = (m_run + log2f(l_run)) / L2E;
  uint32_t yp[NDB][8];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int j = 0; j < 8; ++j) yp[db][j] = pack_bf2(o[db][2 * j] * inv_l, o[db][2 * j + 1] * inv_l);

  // ---- readout: y += round(eta * RMSNorm(normalize(q_raw) . M * (1-gamma)/sqrt(HD))), rounded.
  // The fp32 interior is reassociated: sum(ym^2) is taken over the raw products and scaled
  // once, and 1/|q|, (1-gamma)/sqrt(HD), the RMS scale and eta make one factor per query.
  if (readout) {
    wait_vm<0>();
    sync_lds();
    if (fuse_q && a.qn_w) {   // q_raw: the normalised row (the weight loads hit the cache)
      qp.fetch_w(a, h);
      float x[HD / 16][8];
      QPrep<HD>::unpack(rf, x);
      qp.scale(x, q_r);
      QPrep<HD>::pack(rf, x);
    }
    float qq = rf.sumsq();
    qq = pair_sum32(qq);
    const float inv_q = 1.0f / fmaxf(sqrtf(qq), 1e-12f);
    const float coef = div_rn(1.0f - a.gamma[hkv], sqrtf((float)HD));
    const uint16_t* mt_hi = reinterpret_cast<const uint16_t*>(sm.ring[2 * ((P + 1) % NPS)][0]);
    const uint16_t* mt_lo = reinterpret_cast<const uint16_t*>(sm.ring[2 * (NPS == 3 ? (P + 2) % 3 : P % 2)][0]);
    f32x16 rr[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      rr[db] = zero16();
      const int dr = 32 * db + n;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) {
        const int piece = (2 * ks + h) ^ (dr % NP);
        mma_bf16(rr[db], *reinterpret_cast<const u16x8*>(mt_hi + dr * HD + 8 * piece), rf.v[ks]);
        mma_bf16(rr[db], *reinterpret_cast<const u16x8*>(mt_lo + dr * HD + 8 * piece), rf.v[ks]);
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) ss = fmaf(rr[db][r], rr[db][r], ss);
    ss = pair_sum32(ss);
    const float k1 = inv_q * coef;
    const float rs = 1.0f / sqrtf(ss * (k1 * k1) * (1.0f / HD) + a.eps);
    const float kq = k1 * rs * eta;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float4 w4 = *reinterpret_cast<const float4*>(&sm.resw[32 * db + 8 * r4 + 4 * h]);
        const uint32_t e0 = pack_bf2(rr[db][4 * r4] * kq * w4.x, rr[db][4 * r4 + 1] * kq * w4.y);
        const uint32_t e1 = pack_bf2(rr[db][4 * r4 + 2] * kq * w4.z, rr[db][4 * r4 + 3] * kq * w4.w);
        uint32_t& y0 = yp[db][2 * r4];
        uint32_t& y1 = yp[db][2 * r4 + 1];
        y0 = pack_bf2(bf_lo(y0) + bf_lo(e0), bf_hi(y0) + bf_hi(e0));
        y1 = pack_bf2(bf_lo(y1) + bf_lo(e1), bf_hi(y1) + bf_hi(e1));
      }
  }

  // ---- write y[b][t][hq][d], 4 consecutive features per store
  if (qok) {
    uint16_t* yrow = reinterpret_cast<uint16_t*>(a.y) + b * a.y_sb + (long long)t * a.y_st + hq * HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<uint2*>(yrow + 32 * db + 8 * r4 + 4 * h) = make_uint2(yp[db][2 * r4], yp[db][2 * r4 + 1]);
  }
}

template <int HD, bool SR>
static void launch_fwd2(const b3_attn_args& ab, int G, int nw, int qlen, int n_chunks, dim3 grid, int nthreads, int QW,
                        hipStream_t st) {
  if (G == 4) {
    // one query tile of the four heads per workgroup (four wavefronts), two workgroups per CU
    const dim3 grid1((qlen + 31) / 32, n_chunks, ab.B * ab.HKV);
    hipLaunchKernelGGL((attn_fwd2_kernel<HD, 4, 2, SR>), grid1, dim3(256), 0, st, ab, 1);
  } else if (nw == 8) {
    hipLaunchKernelGGL((attn_fwd2_kernel<HD, 8, 3, SR>), grid, dim3(nthreads), 0, st, ab, QW);
  } else if (nw == 4) {
    hipLaunchKernelGGL((attn_fwd2_kernel<HD, 4, 3, SR>), grid, dim3(nthreads), 0, st, ab, QW);
  } else {
    hipLaunchKernelGGL((attn_fwd2_kernel<HD, 2, 3, SR>), grid, dim3(nthreads), 0, st, ab, QW);
  }
}

template <typename T, int HD>
static int launch_attn(const b3_attn_args& a, hipStream_t st) {
  const int G = a.H / a.HKV;
  const int QW = G <= 4 ? 2 : 1;
  const int per_wg = 32 * QW;
  const int all_chunks = a.mode == 0 ? (a.n_q + a.C - 1) / a.C : 1;
  int c0 = a.chunk_begin, c1 = a.chunk_end == 0 ? all_chunks : min(a.chunk_end, all_chunks);
  if (a.part == 2) c0 = max(c0, 2);   // the slot field exists from chunk 2 on
  const int n_chunks = c1 - c0;
  if (n_chunks <= 0) return B3_OK;
  const int qlen = a.mode == 0 ? a.C : a.n_q;
  dim3 grid((qlen + per_wg - 1) / per_wg, n_chunks, a.B * a.HKV);
  const int nthreads = 64 * G * QW;
  if constexpr (St<T>::is_bf16) {
    if (a.mode == 0 && (!a.m_res || a.m_split)) {
      b3_attn_args ab = a;
      ab.chunk_begin = c0;
      const int nw = nthreads / 64;
      if (a.part == 0 && (a.S == 128 || a.n_q <= 2 * a.C) && (nw == 2 || nw == 4 || nw == 8)) {
        if (a.score_round) launch_fwd2<HD, true>(ab, G, nw, qlen, n_chunks, grid, nthreads, QW, st);
        else launch_fwd2<HD, false>(ab, G, nw, qlen, n_chunks, grid, nthreads, QW, st);
        return (int)hipGetLastError();
      }
      if (a.q_lin) return B3_ERR_UNSUPPORTED;   // the in-kernel query preparation is fwd2's
      const int ipt = (KB * (HD / 8) + nthreads - 1) / nthreads;
      if (ipt <= 1) hipLaunchKernelGGL((attn_fwd_kernel<HD, 1>), grid, dim3(nthreads), 0, st, ab, QW);
      else if (ipt <= 2) hipLaunchKernelGGL((attn_fwd_kernel<HD, 2>), grid, dim3(nthreads), 0, st, ab, QW);
      else hipLaunchKernelGGL((attn_fwd_kernel<HD, 4>), grid, dim3(nthreads), 0, st, ab, QW);
      return (int)hipGetLastError();
    }
  }
  if (a.part != 0 || c0 != 0 || c1 != all_chunks || a.q_lin) return B3_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((attn_kernel<T, HD>), grid, dim3(nthreads), 0, st, a, QW);
  return (int)hipGetLastError();
}

}  // namespace b3

extern "C" int bolt3_chunk_attn(const b3_attn_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->n_q <= 0 || a->H % a->HKV != 0) return B3_ERR_ARG;
  if (a->H / a->HKV > 8 || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  const bool fuse_q = a->q_lin != nullptr;
  if (!a->win_k || !a->win_v || !a->y || !a->gamma || !a->res_w) return B3_ERR_ARG;
  if (!fuse_q && (!a->q_rope || !a->eta)) return B3_ERR_ARG;
  if (fuse_q) {
    const auto mis16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 != 0; };
    if (a->dtype != B3_BF16 || a->mode != 0 || a->part != 0) return B3_ERR_UNSUPPORTED;
    if (!a->rope_cs || !a->gates || a->gates_col < 0 || a->gates_stride < a->gates_col + a->H ||
        a->q_lin_stride < (int64_t)a->H * a->HD || (a->q_lin_stride * 2) % 16 || mis16(a->q_lin) ||
        mis16(a->rope_cs) || (a->qn_w && mis16(a->qn_w)))
      return B3_ERR_ARG;
  }
  if (a->mode == 0) {
    if (a->C <= 0 || a->n_sinks < 0) return B3_ERR_ARG;
    if (a->part == 0 && a->n_q > 2 * a->C && (!a->slot_k || !a->slot_v || !a->slot_bias)) return B3_ERR_ARG;
  } else if (a->mode == 1) {
    if (a->b_len < a->n_q || a->n_q > 256) return B3_ERR_ARG;
    if (a->has_slots && (!a->slot_k || !a->slot_v || !a->slot_bias)) return B3_ERR_ARG;
    if (a->n_sink_keys > 0 && (!a->sink_k || !a->sink_v)) return B3_ERR_ARG;
  } else {
    return B3_ERR_ARG;
  }
  if (a->m_res && !fuse_q && !a->q_raw) return B3_ERR_ARG;
  if (a->m_split && a->dtype != B3_BF16) return B3_ERR_ARG;
  if (a->part < 0 || a->part > 2 || (a->part != 0 && (a->mode != 0 || !a->partial))) return B3_ERR_ARG;
  if (a->chunk_begin < 0 || a->chunk_end < 0 || (a->chunk_end != 0 && a->chunk_end < a->chunk_begin) ||
      (a->mode != 0 && (a->chunk_begin != 0 || a->chunk_end != 0)))
    return B3_ERR_ARG;
  if (a->part == 2 && a->n_q > 2 * a->C && (!a->slot_k || !a->slot_v || !a->slot_bias)) return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return a->HD == 64 ? b3::launch_attn<float, 64>(*a, st) : b3::launch_attn<float, 128>(*a, st);
  if (a->dtype == B3_BF16)
    return a->HD == 64 ? b3::launch_attn<uint16_t, 64>(*a, st) : b3::launch_attn<uint16_t, 128>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

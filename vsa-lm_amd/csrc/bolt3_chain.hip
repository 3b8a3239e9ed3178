// Consolidation chain: successive attractor consolidations of every (batch,
// kv-head) row.
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
// The slot decisions never read M_res, so one launch of bolt3_chain runs three
// kernels on the stream:
//   decide_kernel  one 512-thread workgroup per bh walks all steps with the
//                  slot state in LDS and writes, per step, the delta-rule
//                  weight w_j = beta_j * [token j goes to M_res], the roped
//                  slot keys / values / bias snapshots and the decision log;
//   gersh_kernel   one workgroup per (step, bh), all in parallel: Gershgorin
//                  column sums of |Khat Khat^T| diag(w) -> bsafe_j, and 1/|k_j|;
//   mres_kernel    one workgroup per (bh, 32 columns of M): the columns of M
//                  evolve independently under the delta rule, so HD/32
//                  workgroups per bh walk the steps, each keeping its M^T block
//                  in LDS (fp32 and, for bf16 storage, bf16 hi + lo so every
//                  MFMA operand is exact bf16).
// bf16 storage multiplies exact bf16 operands (products are exact in fp32) and
// splits fp32 operands into hi + lo; fp32 storage uses the fp32 MFMA.
// Orderings are ranks computed by counting on monotone integer keys (one pass,
// stable): the larger value first (NaN first), equal values by lower index.
#include <mutex>
#include <type_traits>

#include "bolt3_common.h"
#include "bolt3_math.h"
#include "bolt3_amd.h"

namespace b3 {

constexpr int S = 128;     // attractor slots
constexpr int LMAX = 256;  // tokens per consolidation step
constexpr int TIE_STACK = 32;  // pending ranges of the tie-order sort
constexpr int DT = 512;    // decide_kernel threads
constexpr int DWAVES = DT / WAVE;
constexpr int MT = 256;    // gersh_kernel / mres_kernel threads
constexpr int MWAVES = MT / WAVE;
constexpr float SIM_K = 0.88f, SIM_V = 0.80f, UTIL_DECAY = 0.995f;

enum : int { F_MERGE = 1, F_DELTA = 2, F_INS = 4 };

// Workspace: roped slot keys per bh when they do not fit in LDS (fp32, HD=128), then
// three [n_steps][bh][LMAX] float arrays: w, bsafe, 1/|k|.
template <typename T, int HD>
struct Work {
  static constexpr bool KREAD_LDS = sizeof(T) == 2 || HD == 64;
  static constexpr long long KREAD = KREAD_LDS ? 0 : (long long)S * HD * sizeof(T);
  static long long bytes(long long bh, long long n_steps) { return bh * KREAD + 3 * n_steps * bh * LMAX * 4; }
};

// Token range of a step.  Steps are fill steps while slots are free; the slot count
// after each step depends only on the token counts, so every kernel derives it alike.
__device__ __forceinline__ int step_len(const b3_chain_args& a, int step) { return step == 0 ? a.len0 : a.step_len; }
__device__ __forceinline__ int step_off(const b3_chain_args& a, int step) {
  return step == 0 ? a.off0 : step * a.step_stride;
}

// ----------------------------------------------------------------- decide_kernel LDS

template <typename T, int HD>
struct DecSmem {
  static constexpr int KS = sizeof(T) == 2 ? HD + 8 : HD + 4;   // slot row stride (16-byte aligned rows)
  static constexpr bool KREAD_LDS = Work<T, HD>::KREAD_LDS;
  static constexpr bool BF = sizeof(T) == 2;                     // bf16: 16-token tiles, av^T kept
  static constexpr int VTS = S + 8;                               // av^T row stride
  alignas(16) T ak[S * KS];
  alignas(16) T av[S * KS];
  alignas(16) T kread[KREAD_LDS ? S * KS : 1];                    // roped slot keys
  // av^T [d][slot] (bf16); within each 32-slot block the slots are stored in the order
  // 0-3, 16-19, 4-7, 20-23, ..., so that the 8 K elements of lane group g of a 16x16x32 MFMA
  // operand (slots 4g..4g+3 and 16+4g..16+4g+3) are one 16-byte row piece
  alignas(16) T avt[BF ? HD * VTS : 1];
  float mass[S], util[S], pm[S], inv_nak[S], keep[S], bias[S];
  float tbl[S];   // bf16 scoring: bias * log2(e), -inf for slots masked in a fill step
  float tnn[S];   // bf16 scoring: 1/|ak|, 0 for slots masked in a fill step
  int act[S], dirty[S], vdirty[S];
  int any_merge;
  int tie;   // this step's tie handling: B3_TIE_* bits
  float invf[HD / 2];
  float rel[LMAX], score[LMAX];
  float tpos[LMAX], tbeta[LMAX];   // this step's token positions and delta-rule gates
  int slot[LMAX], flags[LMAX];
  float sk_a[LMAX];
  int si_a[LMAX];
  float sk_b[S];
  int si_b[S];
  // fp32 storage scores 32-token tiles in rounds of 128 tokens (4 wave pairs x 32); both
  // waves of a pair compute the whole softmax, then each forms v_hat and the value cosine on
  // half of the feature dims and leaves partial sums here for the combine pass.  bf16
  // storage needs none of it: one wave owns 16 tokens and all slots.
  static constexpr int SC = BF ? 1 : 128;
  static constexpr int NP = DWAVES / 2;
  union {  // phase-local buffers
    struct {
      float e2[2][SC], v2[2][SC], dv[2][SC], vv[2][SC], aa[2][SC], bv[2][SC];
      int bs[2][SC];
      uint32_t xkey[NP][2][BF ? 1 : 32];
      float xbv[NP][2][BF ? 1 : 32];
      int xbs[NP][2][BF ? 1 : 32];
    } sc;
    struct {
      int cnt[S], off[S], hits[S], mlist[LMAX];
      float psum[S];
      unsigned bits[S][LMAX / 32];   // bit j of row s: token j merges into slot s
      int nhit;
    } mg;
    struct { float mx[2][S]; int nan[2][S]; } kp;
    struct { alignas(16) uint64_t a[LMAX]; alignas(16) uint64_t b[S]; } ok;
    struct {   // tie order (one wavefront per ordering): packed elements, stop positions, ranges
      alignas(16) uint64_t e[2][LMAX];
      int pr[2][LMAX + 1];
      int stk[2][3 * TIE_STACK];
    } to;
  } u;
};
static_assert(sizeof(DecSmem<uint16_t, 128>) <= 160 * 1024, "decide_kernel LDS");
static_assert(sizeof(DecSmem<float, 128>) <= 160 * 1024, "decide_kernel LDS");
static_assert(sizeof(DecSmem<float, 64>) <= 160 * 1024, "decide_kernel LDS");

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
// 4 consecutive elements as floats
__device__ __forceinline__ void ld4(const uint16_t* p, float* o) {
  const u16x4 q = *reinterpret_cast<const u16x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = bf2f(q[i]);
}
__device__ __forceinline__ void ld4(const float* p, float* o) {
  const float4 q = *reinterpret_cast<const float4*>(p);
  o[0] = q.x; o[1] = q.y; o[2] = q.z; o[3] = q.w;
}

// 4 consecutive storage elements kept packed in registers (bf16: 2 VGPRs)
template <typename T> struct V4;
template <> struct V4<uint16_t> {
  u16x4 x;
  __device__ __forceinline__ void load(const uint16_t* p, bool ok) {
    if (ok) x = *reinterpret_cast<const u16x4*>(p);
    else { x[0] = 0; x[1] = 0; x[2] = 0; x[3] = 0; }
  }
  __device__ __forceinline__ float get(int q) const { return bf2f(x[q]); }
};
template <> struct V4<float> {
  float4 x;
  __device__ __forceinline__ void load(const float* p, bool ok) {
    x = ok ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __device__ __forceinline__ float get(int q) const { return q == 0 ? x.x : q == 1 ? x.y : q == 2 ? x.z : x.w; }
};

// 8 consecutive elements, 16-byte (bf16) or 2 x 16-byte (fp32) moves; both pointers aligned
__device__ __forceinline__ void copy8(uint16_t* d, const uint16_t* s) {
  *reinterpret_cast<u16x8*>(d) = *reinterpret_cast<const u16x8*>(s);
}
__device__ __forceinline__ void copy8(float* d, const float* s) {
  *reinterpret_cast<float4*>(d) = *reinterpret_cast<const float4*>(s);
  *reinterpret_cast<float4*>(d + 4) = *reinterpret_cast<const float4*>(s + 4);
}

// ----------------------------------------------------------------- orderings

// Monotone integer image of a float: a < b  <=>  ord(a) < ord(b); NaN maps above +inf, so
// it ranks first in a descending and last in an ascending order (torch.topk's placement).
// -0 and +0 map to adjacent keys.
__device__ __forceinline__ uint32_t ord_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// 64-bit sort keys that carry the tie rule: descending order = larger key first with the
// lower index on equal values; ascending order = smaller key first, lower index first.
__device__ __forceinline__ uint64_t desc_key(float f, int i) {
  return ((uint64_t)ord_key(f) << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
}
__device__ __forceinline__ uint64_t asc_key(float f, int i) { return ((uint64_t)ord_key(f) << 32) | (uint32_t)i; }

// Rank of key x among keys[0..n) (distinct keys, 16-byte aligned array): the number of keys
// above x (descending order) or below x (ascending order).  The range [i0, i1) of indices
// is counted, so several threads can share one rank.
__device__ __forceinline__ int count_above(const uint64_t* keys, int i0, int i1, uint64_t x) {
  int r = 0, i = i0;
#pragma unroll 8
  for (; i + 2 <= i1; i += 2) {
    const ulonglong2 y = *reinterpret_cast<const ulonglong2*>(keys + i);
    r += (y.x > x ? 1 : 0) + (y.y > x ? 1 : 0);
  }
  for (; i < i1; ++i) r += keys[i] > x ? 1 : 0;
  return r;
}
__device__ __forceinline__ int count_below(const uint64_t* keys, int i0, int i1, uint64_t x) {
  int r = 0, i = i0;
#pragma unroll 8
  for (; i + 2 <= i1; i += 2) {
    const ulonglong2 y = *reinterpret_cast<const ulonglong2*>(keys + i);
    r += (y.x < x ? 1 : 0) + (y.y < x ? 1 : 0);
  }
  for (; i < i1; ++i) r += keys[i] < x ? 1 : 0;
  return r;
}

// ----------------------------------------------------------------- the reference's tie order
//
// The reference orders with torch.topk on the CPU (vsa_lm/config/bolt3.py:137-138, :183).
// Among exactly equal values its order is that of the C++ library's algorithms it runs
// (aten TopKImpl.h): nth_element at k-1 followed by sort of the first k-1 elements
// (introselect / introsort: median-of-three pivot moved to the front, unguarded Hoare
// partition, ranges of at most 16 (sort) or 3 (select) elements finished by insertion sort),
// or partial_sort (a heap of k elements) when 64*k <= n.  tie_order_wave restates that order
// on one wavefront, so the kernel's slot decisions follow the reference on ties too:
//  * one Hoare partition in one pass: the left scan stops, in ascending position, at the
//    elements not ordered before the pivot (L), the right scan, descending, at those not
//    ordered after it (R); the i-th L and the i-th R swap while the L lies below the R (m
//    swaps), and the cut is the (m+1)-th L or the m-th R, whichever is lower.  Ballots and
//    prefix counts rank every stop, so the swaps are done at once;
//  * the ranges sort leaves to insertion sort keep equal elements in their order after the
//    partitions, and insertion sort is stable, so a stable rank of the whole sorted range
//    gives the final order;
//  * partial_sort (k <= 4) runs its heap steps uniformly on the whole wavefront.
// Elements are packed as (key << 32 | source index) with a 32-bit key that is lowest for the
// element that comes first (NaN first when largest, last otherwise; -0 equals +0, as in a float
// comparison).  A depth limit reached (heap fallback of the library, not restated) sets bit 0
// of the returned flags.
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t tie_key(float v, bool largest) {
  const uint32_t k = ord_key(v + 0.0f);
  return largest ? ~k : k;
}
__device__ __forceinline__ uint32_t pk_key(uint64_t e) { return (uint32_t)(e >> 32); }

// Median-of-three move and Hoare partition of e[f, l) (l - f > 3); returns the cut.
__device__ int tie_partition(uint64_t* e, int* pr, int f, int l, int lane, int& flags) {
  const int a = f + 1, b = f + (l - f) / 2, c = l - 1;
  const uint32_t ka = pk_key(e[a]), kb = pk_key(e[b]), kc = pk_key(e[c]);
  int t;
  if (ka < kb) t = kb < kc ? b : (ka < kc ? c : a);
  else t = ka < kc ? a : (kb < kc ? c : b);
  const uint64_t ef = e[f], et = e[t];
  wave_lds_fence();
  if (lane == 0) {
    e[f] = et;
    e[t] = ef;
  }
  wave_lds_fence();
  const uint32_t piv = pk_key(et);
  const unsigned long long below = (1ull << lane) - 1ull;
  uint64_t x[4];
  bool lf[4], rf[4];
  unsigned long long bl[4], br[4];
  int tot_r = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = a + lane + WAVE * j;
    x[j] = 0ull;
    if (q < l) x[j] = e[q];
    const uint32_t k = pk_key(x[j]);
    lf[j] = q < l && k >= piv;
    rf[j] = q < l && k <= piv;
    bl[j] = __ballot(lf[j]);
    br[j] = __ballot(rf[j]);
    tot_r += __popcll(br[j]);
  }
  int cl = 0, cr = 0, m = 0;
  int rank_l[4], above[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    rank_l[j] = cl + __popcll(bl[j] & below) + 1;
    above[j] = tot_r - (cr + __popcll(br[j] & below) + (rf[j] ? 1 : 0));   // R stops above q
    cl += __popcll(bl[j]);
    cr += __popcll(br[j]);
    m += __popcll(__ballot(lf[j] && above[j] >= rank_l[j]));
  }
  const int tot_l = cl;
  // pr[i] = position of the i-th right stop (i <= m); pr[0] = the (m+1)-th left stop
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = a + lane + WAVE * j;
    if (rf[j] && above[j] + 1 <= m) pr[above[j] + 1] = q;
    if (lf[j] && rank_l[j] == m + 1) pr[0] = q;
  }
  wave_lds_fence();
  uint64_t y[4];
  int pp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pp[j] = 0;
    y[j] = 0ull;
    if (lf[j] && rank_l[j] <= m) {
      pp[j] = pr[rank_l[j]];
      y[j] = e[pp[j]];
    }
  }
  const int l_next = tot_l > m ? pr[0] : INT_MAX;
  const int r_m = m > 0 ? pr[m] : INT_MAX;
  wave_lds_fence();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (lf[j] && rank_l[j] <= m) {
      e[a + lane + WAVE * j] = y[j];
      e[pp[j]] = x[j];
    }
  }
  wave_lds_fence();
  int cut = min(l_next, r_m);
  if (cut == INT_MAX) {   // no left stop at all: cannot happen after a median-of-three move
    flags |= 1;
    cut = l;
  }
  return __builtin_amdgcn_readfirstlane(cut);
}

// Stable order of e[f, l) by key, in place (insertion sort's result).
__device__ void tie_stable_range(uint64_t* e, int f, int l, int lane) {
  uint64_t x[4];
  int r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = f + lane + WAVE * j;
    x[j] = 0ull;
    r[j] = 0;
    if (i < l) x[j] = e[i];
  }
  for (int t = f; t < l; ++t) {
    const uint64_t y = e[t];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = f + lane + WAVE * j;
      r[j] += (pk_key(y) < pk_key(x[j]) || (pk_key(y) == pk_key(x[j]) && t < i)) ? 1 : 0;
    }
  }
  wave_lds_fence();
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (f + lane + WAVE * j < l) e[f + r[j]] = x[j];
  wave_lds_fence();
}

// Heap steps of the library's partial_sort, executed alike by every lane (k <= 4, so the heap
// is a few LDS words; the same value is stored by every lane).
__device__ __forceinline__ void heap_put(uint64_t* e, int i, uint64_t v) {
  e[i] = v;
  wave_lds_fence();
}
__device__ void heap_adjust(uint64_t* e, int hole, int len, uint64_t v) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (pk_key(e[child]) < pk_key(e[child - 1])) child--;
    heap_put(e, hole, e[child]);
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    heap_put(e, hole, e[child - 1]);
    hole = child - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && pk_key(e[parent]) < pk_key(v)) {
    heap_put(e, hole, e[parent]);
    hole = parent;
    parent = (hole - 1) / 2;
  }
  heap_put(e, hole, v);
}
__device__ void heap_pop(uint64_t* e, int len, int res) {
  const uint64_t v = e[res];
  heap_put(e, res, e[0]);
  heap_adjust(e, 0, len, v);
}

// torch.topk's order of the k first elements of e[0, n) (packed with tie_key): source indices
// into out[0, k).  One wavefront; pr holds LMAX + 1 ints, stk 3 * TIE_STACK ints.
__device__ int tie_order_wave(uint64_t* e, int* pr, int* stk, int n, int k, int* out, int lane) {
  int flags = 0;
  if (k <= 0) return 0;
  wave_lds_fence();
  if (k * 64 <= n) {
    if (k >= 2)
      for (int parent = (k - 2) / 2;; --parent) {
        heap_adjust(e, parent, k, e[parent]);
        if (parent == 0) break;
      }
    for (int i = k; i < n; ++i)
      if (pk_key(e[i]) < pk_key(e[0])) heap_pop(e, k, i);
    for (int last = k; last > 1;) {
      --last;
      heap_pop(e, last, last);
    }
  } else {
    // nth_element at k - 1
    int f = 0, l = n, depth = 2 * (31 - __clz(n));
    while (l - f > 3) {
      if (depth == 0) {
        flags |= 1;
        break;
      }
      --depth;
      const int cut = tie_partition(e, pr, f, l, lane, flags);
      if (cut <= k - 1) f = cut;
      else l = cut;
    }
    tie_stable_range(e, f, l, lane);
    // sort of [0, k - 1): the ranges above 16 elements are partitioned, the rest is left in
    // place for the final insertion sort
    const int ks = k - 1;
    if (ks > 16) {
      if (lane == 0) {
        stk[0] = 0;
        stk[1] = ks;
        stk[2] = 2 * (31 - __clz(ks));
      }
      wave_lds_fence();
      int sp = 1;
      while (sp > 0) {
        --sp;
        const int sf = stk[3 * sp], sl = stk[3 * sp + 1], d = stk[3 * sp + 2];
        wave_lds_fence();
        if (sl - sf <= 16) continue;
        if (d == 0 || sp + 2 > TIE_STACK) {
          flags |= 1;
          continue;
        }
        const int cut = tie_partition(e, pr, sf, sl, lane, flags);
        if (lane == 0) {
          stk[3 * sp + 0] = cut;
          stk[3 * sp + 1] = sl;
          stk[3 * sp + 2] = d - 1;
          stk[3 * sp + 3] = sf;
          stk[3 * sp + 4] = cut;
          stk[3 * sp + 5] = d - 1;
        }
        sp += 2;
        wave_lds_fence();
      }
    }
    tie_stable_range(e, 0, ks, lane);
  }
  for (int i = lane; i < k; i += WAVE) out[i] = (int)(uint32_t)e[i];
  wave_lds_fence();
  return flags;
}

// Whether sorted[i] equals a neighbour of the sorted array (length n), by order key.
__device__ __forceinline__ bool tie_at(const float* sorted, int i, int n) {
  const uint32_t k = ord_key(sorted[i] + 0.0f);
  return (i > 0 && ord_key(sorted[i - 1] + 0.0f) == k) || (i + 1 < n && ord_key(sorted[i + 1] + 0.0f) == k);
}

// ----------------------------------------------------------------- decide: helpers

// Roped copies of the dirty slot keys (rotation at the slot's mean position), into the
// LDS copy (bf16) or the workspace copy (fp32, HD=128).  8 rotation pairs per item.
template <typename T, int HD>
__device__ void rope_dirty(DecSmem<T, HD>& sm, T* kread_g, int tid) {
  constexpr int HALF = HD / 2, P8 = HALF / 8;
  T* dst = sm.KREAD_LDS ? sm.kread : kread_g;
  const int rs = sm.KREAD_LDS ? sm.KS : HD;
  // the changed slots, found by every wavefront from two ballots (no barrier): item it takes
  // the (it / P8)-th changed slot in ascending order, so that the rows spread over every thread
  static_assert(S == 2 * WAVE, "two ballots of slots");
  const int lane = tid & (WAVE - 1);
  const unsigned long long m0 = __ballot(sm.dirty[lane] != 0), m1 = __ballot(sm.dirty[WAVE + lane] != 0);
  const int n0 = __popcll(m0);
  const int nd = n0 + __popcll(m1);
  for (int it = tid; it < nd * P8; it += DT) {
    int k = it / P8;
    unsigned long long m = k < n0 ? m0 : m1;
    int base = k < n0 ? 0 : WAVE;
    if (k >= n0) k -= n0;
    // position of the k-th set bit of m (k < popcount(m)) by halving
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) {
      const unsigned long long lo = m & ((1ull << w) - 1);
      const int c = __popcll(lo);
      if (k >= c) {
        k -= c;
        m >>= w;
        base += w;
      } else {
        m = lo;
      }
    }
    const int s = base, i0 = (it % P8) * 8;
    float x0[8], x1[8];
    ld8(&sm.ak[s * sm.KS + i0], x0);
    ld8(&sm.ak[s * sm.KS + i0 + HALF], x1);
    const float p = sm.pm[s];
    alignas(16) T r0[8];
    alignas(16) T r1[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float sn, cs;
      sincos_rope(mul_rn(p, sm.invf[i0 + q]), &sn, &cs);
      const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
      r0[q] = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x0[q], c)), St<T>::rnd(mul_rn(-x1[q], si))));
      r1[q] = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x1[q], c)), St<T>::rnd(mul_rn(x0[q], si))));
    }
    copy8(dst + s * rs + i0, r0);
    copy8(dst + s * rs + i0 + HALF, r1);
  }
}

// Step token rows into slots: for each i < n where pick(i, j, s) holds, slot s takes token j's
// un-roped key and value (and, with kp_copy, its roped key).  n <= S and every picked slot is
// distinct, so a thread's items (at most S*HD/8/DT) are independent: all their global loads go
// out before the first store, one memory round trip instead of one per item.
template <typename T, int HD, typename Pick>
__device__ __forceinline__ void take_rows(DecSmem<T, HD>& sm, T* kread_w, int krs, bool kp_copy, const T* kr,
                                          const T* v, const T* kp, int n, Pick pick, int tid) {
  constexpr int NC8 = HD / 8, PER = (S * NC8 + DT - 1) / DT;
  Vec8<T> kx[PER], vx[PER], px[PER];
  int dst[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int it = tid + u * DT, i = it / NC8, d8 = 8 * (it % NC8);
    int j = 0, s = -1;
    if (i < n && pick(i, j, s)) {
      kx[u].load(kr + (long long)j * HD + d8);
      vx[u].load(v + (long long)j * HD + d8);
      if (kp_copy) px[u].load(kp + (long long)j * HD + d8);
    } else {
      s = -1;
    }
    dst[u] = s;
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    if (dst[u] < 0) continue;
    const int d8 = 8 * ((tid + u * DT) % NC8);
    kx[u].store(&sm.ak[dst[u] * sm.KS + d8]);
    vx[u].store(&sm.av[dst[u] * sm.KS + d8]);
    if (kp_copy) px[u].store(kread_w + dst[u] * krs + d8);
  }
}

// 1 / max(||ak_s||, 1e-12) for every slot (four threads per slot).
template <typename T, int HD>
__device__ void slot_norms(DecSmem<T, HD>& sm, int tid) {
  const int s = tid >> 2, q = tid & 3;
  float ss = 0.f;
#pragma unroll
  for (int d = q * (HD / 4); d < (q + 1) * (HD / 4); d += 8) {
    float x[8];
    ld8(&sm.ak[s * sm.KS + d], x);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  if (q == 0) sm.inv_nak[s] = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
}

// Inverse slot norms for the bf16 cosine match: 0 for the slots a fill step masks (their
// rows are zero in every state the chain builds, so the cosine is exactly 0 either way).
template <typename T, int HD>
__device__ __forceinline__ void masked_norms(DecSmem<T, HD>& sm, int tid, bool steady) {
  if (tid < S) sm.tnn[tid] = (steady || sm.act[tid]) ? sm.inv_nak[tid] : 0.f;
}

// ----------------------------------------------------------------- decide: retrieval

// Token data of one 32-token tile for wave `half` of a pair: the roped key fragment and
// the values on this wave's half of the feature dims (the un-roped key fragment is loaded
// by the tile itself).
template <typename T, int HD>
struct TileIn {
  static constexpr int HDB = HD / 64;
  Frag<T, HD> fq;
  V4<T> vx[HDB][4];   // v[tok][32*(half*HDB + i) + 8*g + 4*h + q]
  __device__ __forceinline__ void load(const T* kp, const T* kr, const T* v, int t0, int l, int half, int lane) {
    const int n = lane & 31, h = lane >> 5, tok = t0 + n;
    fq.load(kp, tok, l, lane);
#pragma unroll
    for (int i = 0; i < HDB; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        vx[i][g].load(v + (long long)tok * HD + 32 * (half * HDB + i) + 8 * g + 4 * h, tok < l);
  }
};

// fp32 storage: one 32-token tile, one half of the work, for wave `half` of wave pair
// `pair`.  Both waves compute the whole softmax; each cosine-matches half of the slots and
// one LDS exchange gives the pair the best slot.  Then wave `half` forms v_hat and the
// value cosine on its half of the feature dims and leaves partial sums in LDS for the
// combine pass.  Contains barriers: every thread of the workgroup calls it the same number
// of times (tokens past l are inert).
template <typename T, int HD>
__device__ void score_tile(DecSmem<T, HD>& sm, const T* kread, const TileIn<T, HD>& td, const T* kr, int t0, int l,
                           bool steady, float scale, int pair, int half, int lane) {
  static_assert(!St<T>::is_bf16, "bf16 storage uses score_tile16");
  using Sm = DecSmem<T, HD>;
  constexpr int NMB = 4;
  constexpr int HDB = TileIn<T, HD>::HDB;
  const int n = lane & 31, h = lane >> 5;
  const int tok = t0 + n;
  const bool in = tok < l;

  Frag<T, HD> fk;   // un-roped keys: consumed after the softmax, so their latency hides behind it
  fk.load(kr, tok, l, lane);

  // scores^T[slot][tok] = kread . kp^T
  f32x16 acc[NMB];
#pragma unroll
  for (int m2 = 0; m2 < NMB; ++m2) {
    acc[m2] = zero16();
    if constexpr (Sm::KREAD_LDS) mm_rows_frag<HD>(acc[m2], sm.kread, Sm::KS, 32 * m2, td.fq, lane);
    else mm_rows_frag<HD>(acc[m2], kread, HD, 32 * m2, td.fq, lane);
  }

  // softmax over the slots (column of this lane pair)
  float mx = -INFINITY;
#pragma unroll
  for (int m2 = 0; m2 < NMB; ++m2)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int s0 = 32 * m2 + 8 * r4 + 4 * h;
      const float4 b4 = *reinterpret_cast<const float4*>(&sm.bias[s0]);
      const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float x = add_rn(mul_rn(acc[m2][4 * r4 + q], scale), bb[q]);
        if (!steady && !sm.act[s0 + q]) x = -1e9f;
        acc[m2][4 * r4 + q] = x;
        mx = fmaxf(mx, x);
      }
    }
  mx = fmaxf(mx, xor32(mx));
  float sum = 0.f;
#pragma unroll
  for (int m2 = 0; m2 < NMB; ++m2)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = expf(acc[m2][r] - mx);
      acc[m2][r] = e;
      sum += e;
    }
  sum += xor32(sum);
  // cos^T[slot][tok] = ak . kr^T / (|ak| |kr|) on this wave's half of the slots; argmax on
  // integer keys: slots ascend along the scan, so a strictly larger key keeps the lower index
  // on ties, and NaN (largest key) wins as torch.max does
  float kk = fk.sumsq();
  kk += xor32(kk);
  const float inv_nk = 1.0f / fmaxf(sqrtf(kk), 1e-12f);
  uint32_t bkey = 0;
  float bv = 0.f;
  int bs = -1;
#pragma unroll
  for (int m2 = 0; m2 < 2; ++m2) {
    const int mb = 2 * half + m2;
    f32x16 c = zero16();
    mm_rows_frag<HD>(c, sm.ak, Sm::KS, 32 * mb, fk, lane);
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int s0 = 32 * mb + 8 * r4 + 4 * h;
      const float4 n4 = *reinterpret_cast<const float4*>(&sm.inv_nak[s0]);
      const float nn[4] = {n4.x, n4.y, n4.z, n4.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float cv = c[4 * r4 + q] * (nn[q] * inv_nk);
        if (!steady && !sm.act[s0 + q]) cv = 0.f;
        const uint32_t k = ord_key(cv + 0.0f);   // -0 ranks with +0, as in a float compare
        if (bs < 0 || k > bkey) { bkey = k; bv = cv; bs = s0 + q; }
      }
    }
  }
  {
    const uint32_t ok = (uint32_t)__shfl_xor((int)bkey, 32, 64);
    const float ov = xor32(bv);
    const int os = xor32i(bs);
    if (ok > bkey || (ok == bkey && os < bs)) { bkey = ok; bv = ov; bs = os; }
  }
  const float rs = 1.0f / sum;
  // the pair's best slot through one exchange
  if (h == 0) {
    sm.u.sc.xkey[pair][half][n] = bkey;
    sm.u.sc.xbv[pair][half][n] = bv;
    sm.u.sc.xbs[pair][half][n] = bs;
  }
  sync_lds();
  {
    const int o = half ^ 1;
    const uint32_t ko = sm.u.sc.xkey[pair][o][n];
    const int so = sm.u.sc.xbs[pair][o][n];
    if (ko > bkey || (ko == bkey && so < bs)) { bkey = ko; bv = sm.u.sc.xbv[pair][o][n]; bs = so; }
  }
#pragma unroll
  for (int m2 = 0; m2 < NMB; ++m2)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[m2][r] = mul_rn(acc[m2][r], rs);

  // value cosine with the best slot, partial over this wave's feature half (from registers)
  float dvv = 0.f, vv = 0.f, aa = 0.f;
  if (steady) {
    const int bsr = bs < 0 ? 0 : bs;
#pragma unroll
    for (int i = 0; i < HDB; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float y[4];
        ld4(&sm.av[bsr * Sm::KS + 32 * (half * HDB + i) + 8 * g + 4 * h], y);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = td.vx[i][g].get(q);
          dvv += x * y[q];
          vv += x * x;
          aa += y[q] * y[q];
        }
      }
    dvv += xor32(dvv);
    vv += xor32(vv);
    aa += xor32(aa);
  }

  // v_hat^T[d][tok] = av^T . P^T on this wave's feature half; partial rel_err sums
  float e2 = 0.f, v2 = 0.f;
#pragma unroll
  for (int i = 0; i < HDB; ++i) {
    const int db = half * HDB + i;
    f32x16 vh = zero16();
    const int d = 32 * db + n;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s = 32 * mb + d_row(lane, r);
        mma_f32(vh, sm.av[s * Sm::KS + d], acc[mb][r]);
      }
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float x = td.vx[i][g].get(q);
        const float dv = x - vh[4 * g + q];
        e2 += dv * dv;
        v2 += x * x;
      }
  }
  e2 += xor32(e2);
  v2 += xor32(v2);
  if (h == 0 && in) {
    const int pt = tok & 127;   // index within the round
    sm.u.sc.e2[half][pt] = e2;
    sm.u.sc.v2[half][pt] = v2;
    sm.u.sc.dv[half][pt] = dvv;
    sm.u.sc.vv[half][pt] = vv;
    sm.u.sc.aa[half][pt] = aa;
    sm.u.sc.bv[half][pt] = bv;
    sm.u.sc.bs[half][pt] = bs;
  }
}

// Combine the two halves for token tok of the current round (one thread per token):
// rel_err, score, value cosine with the best slot (steady), merge flag; the decision log
// gets the best cosine and value cosine here.  Returns the token's merge flag.
template <typename T, int HD>
__device__ bool score_combine(DecSmem<T, HD>& sm, int l, bool steady, int tok, float* log) {
  if (tok >= l) return false;
  const int pt = tok & 127;
  const float e2 = sm.u.sc.e2[0][pt] + sm.u.sc.e2[1][pt];
  const float v2 = sm.u.sc.v2[0][pt] + sm.u.sc.v2[1][pt];
  const float rel = sqrtf(e2) / (sqrtf(v2) + 1e-6f);
  const float bv = sm.u.sc.bv[0][pt];
  const int bs = sm.u.sc.bs[0][pt];
  const float score = rel * (1.0f - fminf(fmaxf(bv, 0.0f), 1.0f));
  float simv = 0.f;
  if (steady) {
    const float dvv = sm.u.sc.dv[0][pt] + sm.u.sc.dv[1][pt];
    const float vv = sm.u.sc.vv[0][pt] + sm.u.sc.vv[1][pt];
    const float aa = sm.u.sc.aa[0][pt] + sm.u.sc.aa[1][pt];
    simv = dvv / (fmaxf(sqrtf(vv), 1e-8f) * fmaxf(sqrtf(aa), 1e-8f));
  }
  const bool merge = steady && bv >= SIM_K && simv >= SIM_V;
  sm.rel[tok] = rel;
  sm.score[tok] = score;
  sm.slot[tok] = bs;
  sm.flags[tok] = merge ? F_MERGE : 0;
  if (log) {
    log[B3_LOG_BEST * B3_LOG_COLS + tok] = steady ? bv : 0.f;
    log[B3_LOG_SIMV * B3_LOG_COLS + tok] = simv;
  }
  return merge;
}

// Eviction candidate value of token j: its score, or -1e9 when it merged.
template <typename T, int HD>
__device__ __forceinline__ float cand_value(const DecSmem<T, HD>& sm, int j) {
  return (sm.flags[j] & F_MERGE) ? -1e9f : sm.score[j];
}

// All tiles of a step in rounds of 128 tokens (4 wave pairs x 32), each round followed by
// the combine pass of its tokens.  `td` holds the first round's tile data on entry when
// `ready`.  Returns this thread's merge flag; the caller's barrier publishes the results.
template <typename T, int HD>
__device__ bool score_phase(DecSmem<T, HD>& sm, const T* kread, TileIn<T, HD>& td, bool ready, const T* kr,
                            const T* kp, const T* v, int l, bool steady, float scale, int wave, int lane, int tid,
                            float* log) {
  const int pair = wave >> 1, half = wave & 1;
  if (l <= 128) {   // one round: the tile data may already be in registers
    if (!ready) td.load(kp, kr, v, 32 * pair, l, half, lane);
    score_tile<T, HD>(sm, kread, td, kr, 32 * pair, l, steady, scale, pair, half, lane);
    sync_lds();
    return tid < 128 && score_combine<T, HD>(sm, l, steady, tid, log);
  }
  bool merge = false;
  for (int r = 0; r < (l + 127) / 128; ++r) {
    const int t0 = 128 * r + 32 * pair;
    TileIn<T, HD> tr;
    tr.load(kp, kr, v, t0, l, half, lane);
    score_tile<T, HD>(sm, kread, tr, kr, t0, l, steady, scale, pair, half, lane);
    sync_lds();
    if (tid < 128) merge |= score_combine<T, HD>(sm, l, steady, 128 * r + tid, log);
  }
  return merge;
}

// bf16 storage: one wavefront owns 16 tokens and all S slots, with 16x16x32 MFMAs, so a
// token's softmax, best slot, v_hat and rel_err stay within the wavefront (the 128 slots
// of a token column spread over the four lane groups l / 16).  Lane (n = l % 16, g = l / 16)
// holds the operands of token t0 + n: K group g of every 32-feature step for the keys, and
// features 16*db + 4*g + i of the values (the rows of the v_hat^T tile it owns).
template <int HD>
struct Tile16 {
  static constexpr int NK = HD / 32;   // K steps
  static constexpr int ND = HD / 16;   // 16-feature blocks
  u16x8 q[NK];   // roped keys kp[tok][32*ks + 8*g + i]
  u16x8 k[NK];   // un-roped keys kr[tok][32*ks + 8*g + i]
  u16x4 v[ND];   // values v[tok][16*db + 4*g + i]
  // part 1: roped keys, 2: un-roped keys, 4: values (a mask), so that the loads of a prefetch
  // can be spread over the phases of a step
  __device__ __forceinline__ void load(const uint16_t* kp, const uint16_t* kr, const uint16_t* vv, int t0, int l,
                                       int lane, int parts = 7) {
    const int n = lane & 15, g = lane >> 4, tok = t0 + n;
    const bool ok = tok < l;
    const long long o = (long long)tok * HD;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      if (parts & 1) {
        if (ok) q[ks] = *reinterpret_cast<const u16x8*>(kp + o + 32 * ks + 8 * g);
        else {
#pragma unroll
          for (int i = 0; i < 8; ++i) q[ks][i] = 0;
        }
      }
      if (parts & 2) {
        if (ok) k[ks] = *reinterpret_cast<const u16x8*>(kr + o + 32 * ks + 8 * g);
        else {
#pragma unroll
          for (int i = 0; i < 8; ++i) k[ks][i] = 0;
        }
      }
    }
    if (parts & 4) {
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        if (ok) v[db] = *reinterpret_cast<const u16x4*>(vv + o + 16 * db + 4 * g);
        else { v[db][0] = 0; v[db][1] = 0; v[db][2] = 0; v[db][3] = 0; }
      }
    }
  }
};

// reductions over the four lane groups (the slot rows of one token column)
__device__ __forceinline__ float sum4g(float v) {
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float max4g(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

// Scores, softmax, v_hat, rel_err, best slot and value cosine of the 16 tokens
// [t0, t0 + 16) of one wavefront (bf16 storage).  Writes rel / score / slot / flags (and
// the log's best cosine and value cosine) of its tokens; no barrier inside.  Returns the
// merge flag of token t0 + lane (lanes 0..15).
// The softmax runs in base 2: x' = round_bf(q.k) * scale*log2(e) + bias*log2(e) (one FMA),
// p = exp2(x' - max x'), which equals the reference's exp(x - max x) up to the last bits of
// the exponent argument; slots masked in a fill step carry a -inf bias (at least one slot is
// active whenever the slots are read).
template <int HD>
__device__ bool score_tile16(DecSmem<uint16_t, HD>& sm, const Tile16<HD>& td, int t0, int l, bool steady,
                             float scale, int lane, float* log) {
  using Sm = DecSmem<uint16_t, HD>;
  constexpr int NK = Tile16<HD>::NK, ND = Tile16<HD>::ND, NMB = S / 16;
  const int n = lane & 15, g = lane >> 4;
  const int tok = t0 + n;

  // cos^T[slot][tok] = ak . kr^T / (|ak| |kr|); torch.max semantics: the largest value,
  // the first NaN if there is one, ties to the lower slot (each lane scans its slots in
  // ascending order; the cross-lane merge compares indices)
  float kk = 0.f;
#pragma unroll
  for (int ks = 0; ks < NK; ++ks)
#pragma unroll
    for (int i = 0; i < 8; ++i) { const float x = bf2f(td.k[ks][i]); kk += x * x; }
  kk = sum4g(kk);
  const float inv_nk = 1.0f / fmaxf(sqrtf(kk), 1e-12f);
  float bv = -INFINITY;
  int bs = -1;
  bool bnan = false;
  // A operands of the next slot block are read from LDS while the current one multiplies
  u16x8 op[2][NK];
#pragma unroll
  for (int ks = 0; ks < NK; ++ks) op[0][ks] = *reinterpret_cast<const u16x8*>(&sm.ak[n * Sm::KS + 32 * ks + 8 * g]);
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
    if (mb + 1 < NMB) {
#pragma unroll
      for (int ks = 0; ks < NK; ++ks)
        op[(mb + 1) & 1][ks] = *reinterpret_cast<const u16x8*>(&sm.ak[(16 * (mb + 1) + n) * Sm::KS + 32 * ks + 8 * g]);
    }
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) mma16_bf16(c, op[mb & 1][ks], td.k[ks]);
    const int s0 = 16 * mb + 4 * g;
    const float4 n4 = *reinterpret_cast<const float4*>(&sm.tnn[s0]);
    const float nn[4] = {n4.x, n4.y, n4.z, n4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float cv = c[i] * (nn[i] * inv_nk);
      const bool isn = cv != cv;
      const bool take = !bnan && (cv > bv || isn);   // selects, no branches
      bv = take ? cv : bv;
      bs = take ? s0 + i : bs;
      bnan = bnan || isn;
    }
  }
#pragma unroll
  for (int o = 16; o <= 32; o <<= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int os = __shfl_xor(bs, o, 64);
    const bool onan = ov != ov;
    const bool take = onan ? (!bnan || os < bs) : (!bnan && (ov > bv || (ov == bv && os < bs)));
    if (take) { bv = ov; bs = os; bnan = onan; }
  }

  // scores^T[slot][tok] = kread . kp^T, rounded to bf16, in base-2 units with the slot bias
  f32x4 acc[NMB];
#pragma unroll
  for (int ks = 0; ks < NK; ++ks) op[0][ks] = *reinterpret_cast<const u16x8*>(&sm.kread[n * Sm::KS + 32 * ks + 8 * g]);
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
    if (mb + 1 < NMB) {
#pragma unroll
      for (int ks = 0; ks < NK; ++ks)
        op[(mb + 1) & 1][ks] =
            *reinterpret_cast<const u16x8*>(&sm.kread[(16 * (mb + 1) + n) * Sm::KS + 32 * ks + 8 * g]);
    }
    acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) mma16_bf16(acc[mb], op[mb & 1][ks], td.q[ks]);
  }
  const float sL = scale * 1.4426950408889634f;
  float mx = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
    const float4 b4 = *reinterpret_cast<const float4*>(&sm.tbl[16 * mb + 4 * g]);
    const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = fmaf(round_bf(acc[mb][i]), sL, bb[i]);
      acc[mb][i] = x;
      mx = fmaxf(mx, x);
    }
  }
  mx = max4g(mx);
  float sum = 0.f;
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = __builtin_amdgcn_exp2f(acc[mb][i] - mx);
      acc[mb][i] = e;
      sum += e;
    }
  sum = sum4g(sum);
  const float rs = 1.0f / sum;
  // probabilities rounded to bf16 as the B operand of v_hat^T = av^T . P^T; K step kk covers
  // slots 32*kk .. 32*kk+31 with lane group g holding slots 32*kk + {4g..4g+3, 16+4g..16+4g+3}
  u16x8 pb[S / 32];
#pragma unroll
  for (int kk2 = 0; kk2 < S / 32; ++kk2)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pb[kk2][i] = f2bf(acc[2 * kk2][i] * rs);
      pb[kk2][4 + i] = f2bf(acc[2 * kk2 + 1][i] * rs);
    }

  // v_hat^T[d][tok], rel_err sums; this lane owns features 16*db + 4*g + i of token tok
  float e2 = 0.f, v2 = 0.f;
  u16x8 vo[2][S / 32];
#pragma unroll
  for (int kk2 = 0; kk2 < S / 32; ++kk2)
    vo[0][kk2] = *reinterpret_cast<const u16x8*>(&sm.avt[n * Sm::VTS + 8 * g + 32 * kk2]);
#pragma unroll
  for (int db = 0; db < ND; ++db) {
    if (db + 1 < ND) {
#pragma unroll
      for (int kk2 = 0; kk2 < S / 32; ++kk2)
        vo[(db + 1) & 1][kk2] =
            *reinterpret_cast<const u16x8*>(&sm.avt[(16 * (db + 1) + n) * Sm::VTS + 8 * g + 32 * kk2]);
    }
    f32x4 vh = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk2 = 0; kk2 < S / 32; ++kk2) mma16_bf16(vh, vo[db & 1][kk2], pb[kk2]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = bf2f(td.v[db][i]);
      const float dv = x - round_bf(vh[i]);
      e2 = fmaf(dv, dv, e2);
      v2 = fmaf(x, x, v2);
    }
  }
  e2 = sum4g(e2);
  v2 = sum4g(v2);

  // value cosine with the best slot
  float simv = 0.f;
  if (steady) {
    const int bsr = bs < 0 ? 0 : bs;
    float dvv = 0.f, aa = 0.f;
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const u16x4 y4 = *reinterpret_cast<const u16x4*>(&sm.av[bsr * Sm::KS + 16 * db + 4 * g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = bf2f(td.v[db][i]), y = bf2f(y4[i]);
        dvv = fmaf(x, y, dvv);
        aa = fmaf(y, y, aa);
      }
    }
    dvv = sum4g(dvv);
    aa = sum4g(aa);
    simv = dvv / (fmaxf(sqrtf(v2), 1e-8f) * fmaxf(sqrtf(aa), 1e-8f));
  }
  const float rel = sqrtf(e2) / (sqrtf(v2) + 1e-6f);
  const float score = rel * (1.0f - fminf(fmaxf(bv, 0.0f), 1.0f));
  const bool merge = steady && bv >= SIM_K && simv >= SIM_V;
  if (g == 0 && tok < l) {
    sm.rel[tok] = rel;
    sm.score[tok] = score;
    sm.slot[tok] = bs;
    sm.flags[tok] = merge ? F_MERGE : 0;
    if (log) {
      log[B3_LOG_BEST * B3_LOG_COLS + tok] = steady ? bv : 0.f;
      log[B3_LOG_SIMV * B3_LOG_COLS + tok] = simv;
    }
  }
  return g == 0 && tok < l && merge;
}

// All tokens of a step, 16 per wavefront per round of 128.  `td` holds the first round's
// tile data on entry when `ready`.  Returns this thread's merge flag; the caller's barrier
// publishes the results.
template <int HD>
__device__ bool score_phase16(DecSmem<uint16_t, HD>& sm, Tile16<HD>& td, bool ready, const uint16_t* kr,
                              const uint16_t* kp, const uint16_t* v, int l, bool steady, float scale, int wave,
                              int lane, float* log) {
  if (l <= 128) {
    if (!ready) td.load(kp, kr, v, 16 * wave, l, lane);
    return score_tile16<HD>(sm, td, 16 * wave, l, steady, scale, lane, log);
  }
  bool merge = false;
  for (int r = 0; r < (l + 127) / 128; ++r) {
    Tile16<HD> tr;
    tr.load(kp, kr, v, 128 * r + 16 * wave, l, lane);
    merge |= score_tile16<HD>(sm, tr, 128 * r + 16 * wave, l, steady, scale, lane, log);
  }
  return merge;
}

// av^T columns of the slots whose values changed (vdirty): an item is two adjacent slots
// (adjacent in the permuted column order too) and 8 features, written as 8 dwords; lanes of
// a wavefront take adjacent slot pairs, so their writes fall into distinct banks.
template <typename T, int HD>
__device__ void transpose_dirty_v(DecSmem<T, HD>& sm, int tid) {
  if constexpr (DecSmem<T, HD>::BF) {
    for (int it = tid; it < (S / 2) * (HD / 8); it += DT) {
      const int s = 2 * (it % (S / 2)), d8 = (it / (S / 2)) * 8;
      if (!sm.vdirty[s] && !sm.vdirty[s + 1]) continue;
      const u16x8 x0 = *reinterpret_cast<const u16x8*>(&sm.av[s * sm.KS + d8]);
      const u16x8 x1 = *reinterpret_cast<const u16x8*>(&sm.av[(s + 1) * sm.KS + d8]);
      const int r = s & 31, col = (s & ~31) + 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        *reinterpret_cast<uint32_t*>(&sm.avt[(d8 + q) * sm.VTS + col]) = (uint32_t)x0[q] | ((uint32_t)x1[q] << 16);
    }
  }
}

// ----------------------------------------------------------------- decide_kernel

template <typename T, int HD>
__global__ void __launch_bounds__(DT) decide_kernel(b3_chain_args a) {
  __shared__ DecSmem<T, HD> sm;
  const int bh = blockIdx.x;
  const int tid0 = threadIdx.x;
  const int tid = tid0;
  const int hkv = bh % a.HKV;
  const float kap = a.kappa[hkv];
  const float scale = 1.0f / sqrtf((float)HD);
  const int KS = sm.KS;
  const long long BH = (long long)a.B * a.HKV;

  T* g_ak = reinterpret_cast<T*>(a.ak) + (long long)bh * S * HD;
  T* g_av = reinterpret_cast<T*>(a.av) + (long long)bh * S * HD;
  char* ws = reinterpret_cast<char*>(a.work);
  T* kread_g = reinterpret_cast<T*>(ws) + (long long)bh * S * HD;   // used only when !KREAD_LDS
  float* w_all = reinterpret_cast<float*>(ws + BH * Work<T, HD>::KREAD);
  const T* kread = sm.KREAD_LDS ? sm.kread : kread_g;
  T* kread_w = sm.KREAD_LDS ? sm.kread : kread_g;   // writable view of the roped slot keys
  const int krs = sm.KREAD_LDS ? KS : HD;
  const bool kp_copy = a.kp_exact != 0;              // a slot taken from token j gets kp_j as its roped key
  if (a.started && tid == 0) __hip_atomic_fetch_add(a.started, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // state in; with n_filled == 0 the empty state (zero slots, mass 1) is built here
  const bool fresh = a.n_filled == 0;
  if (!fresh && St<T>::is_bf16) {
    // every load of the thread's rows before their stores: one memory round trip
    constexpr int NI = S * (HD / 8) / DT;
    static_assert(NI * DT == S * (HD / 8), "state rows over the threads");
    u16x8 kx[NI], vx[NI];
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int it = tid + DT * q, s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
      kx[q] = *reinterpret_cast<const u16x8*>(g_ak + s * HD + d8);
      vx[q] = *reinterpret_cast<const u16x8*>(g_av + s * HD + d8);
    }
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int it = tid + DT * q, s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
      *reinterpret_cast<u16x8*>(&sm.ak[s * KS + d8]) = kx[q];
      *reinterpret_cast<u16x8*>(&sm.av[s * KS + d8]) = vx[q];
    }
  } else {
    for (int it = tid; it < S * (HD / 8); it += DT) {
      const int s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
      if (fresh) {
        alignas(16) T z[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) z[q] = St<T>::from_f(0.f);
        copy8(&sm.ak[s * KS + d8], z);
        copy8(&sm.av[s * KS + d8], z);
      } else {
        copy8(&sm.ak[s * KS + d8], g_ak + s * HD + d8);
        copy8(&sm.av[s * KS + d8], g_av + s * HD + d8);
      }
    }
  }
  if (tid < S) {
    sm.mass[tid] = fresh ? 1.0f : a.mass[bh * S + tid];
    sm.util[tid] = fresh ? 0.0f : a.util[bh * S + tid];
    sm.pm[tid] = fresh ? 0.0f : a.pm[bh * S + tid];
    sm.act[tid] = fresh ? 0 : (a.act[bh * S + tid] ? 1 : 0);
    sm.dirty[tid] = 1;
    sm.vdirty[tid] = 1;
  }
  if (tid < HD / 2) sm.invf[tid] = a.inv_freq[tid];
  sync_lds();
  int nf = a.n_filled;
  rope_dirty<T, HD>(sm, kread_g, tid);   // every slot, empty ones included (their rows stay zero)
  transpose_dirty_v<T, HD>(sm, tid);
  __threadfence_block();
  __syncthreads();

  // tile data of the next step's first round, loaded while the current step finishes (bf16)
  constexpr bool BF = St<T>::is_bf16;
  using TD = std::conditional_t<BF, Tile16<HD>, TileIn<T, HD>>;
  TD td;
  bool td_ready = false;
  // parts: 1 roped keys, 2 un-roped keys, 4 values; a steady step issues them after the
  // scoring, the keep scores and the orderings, a fill step all at once
  auto prefetch = [&](int step, int wave, int lane, int parts) {
    if constexpr (BF) {
      if (step + 1 < a.n_steps) {
        const long long nb = (long long)bh * a.tok_bh_stride + (long long)step_off(a, step + 1) * HD;
        td.load(reinterpret_cast<const T*>(a.kp) + nb, reinterpret_cast<const T*>(a.kr) + nb,
                reinterpret_cast<const T*>(a.v) + nb, 16 * wave, step_len(a, step + 1), lane, parts);
        td_ready = true;
      }
    }
  };

  for (int step = 0; step < a.n_steps; ++step) {
    // Thread indices re-derived from an opaque copy each step: the lane-dependent LDS
    // addresses are then recomputed per step instead of hoisted out of the loop and spilled.
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int off = step_off(a, step), l = step_len(a, step);
    const long long tb = (long long)bh * a.tok_bh_stride + (long long)off * HD;
    const T* kr = reinterpret_cast<const T*>(a.kr) + tb;
    const T* kp = reinterpret_cast<const T*>(a.kp) + tb;
    const T* v = reinterpret_cast<const T*>(a.v) + tb;
    const float* pos = a.pos + off;
    const float* beta = a.beta + (long long)bh * a.beta_bh_stride + off;
    const int nT = (l + 31) / 32;
    const bool steady = nf >= S;
    float* log = a.log ? a.log + ((long long)step * BH + bh) * (B3_LOG_ROWS * B3_LOG_COLS) : nullptr;
    float* w_out = w_all + ((long long)step * BH + bh) * LMAX;
    // positions and gates of the step's tokens: loaded here, stored to LDS after the scoring,
    // so that their latency overlaps it
    const float pos_t = tid < l ? pos[tid] : 0.f;
    const float beta_t = tid < l ? beta[tid] : 0.f;

    if (tid == 0) {
      sm.any_merge = 0;
      sm.tie = 0;
    }
    if (tid < S) {
      sm.util[tid] = mul_rn(sm.util[tid], UTIL_DECAY);
      const float lm = logf(fmaxf(sm.mass[tid], 1.0f));
      sm.bias[tid] = steady ? mul_rn(kap, lm) : lm;
      sm.tbl[tid] = (steady || sm.act[tid]) ? sm.bias[tid] * 1.4426950408889634f : -INFINITY;
      sm.dirty[tid] = 0;
      sm.vdirty[tid] = 0;
    }
    slot_norms<T, HD>(sm, tid);
    sync_lds();
    if constexpr (BF) {
      masked_norms<T, HD>(sm, tid, steady);
      sync_lds();
    }

    // ---------------- retrieval scores: first fill ranks by value variance; later fills and
    // steady steps read the slots
    bool has = false;
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
      if constexpr (BF) has = score_phase16<HD>(sm, td, td_ready, kr, kp, v, l, steady, scale, wave, lane, log);
      else has = score_phase<T, HD>(sm, kread, td, td_ready, kr, kp, v, l, steady, scale, wave, lane, tid, log);
    }
    td_ready = false;
    prefetch(step, wave, lane, steady ? 1 : 7);
    if (has) sm.any_merge = 1;
    if (tid < l) {
      sm.tpos[tid] = pos_t;
      sm.tbeta[tid] = beta_t;
    }
    sync_lds();

    if (!steady) {
      // ---------------- fill
      const int m = min(S - nf, l);
      if (tid < l) sm.u.ok.a[tid] = desc_key(sm.score[tid], tid);
      sync_lds();
      {
        // two threads per token, each counting half of the keys
        const int j = tid >> 1, part = tid & 1, mid = (l >> 1) & ~1;
        int r = 0;
        if (j < l) r = count_above(sm.u.ok.a, part ? mid : 0, part ? l : mid, sm.u.ok.a[j]);
        r += __shfl_xor(r, 1, 64);
        if (j < l && part == 0) {
          sm.si_a[r] = j;
          sm.sk_a[r] = sm.score[j];
        }
      }
      sync_lds();
      // exactly equal scores among the picked tokens or at the cut: the reference's order
      if (tid < m && tie_at(sm.sk_a, tid, l)) atomicOr(&sm.tie, B3_TIE_TOP);
      sync_lds();
      if (sm.tie) {
        if (wave == 0) {
          for (int j = lane; j < l; j += WAVE)
            sm.u.to.e[0][j] = ((uint64_t)tie_key(sm.score[j], true) << 32) | (uint32_t)j;
          const int fl = tie_order_wave(sm.u.to.e[0], sm.u.to.pr[0], sm.u.to.stk[0], l, m, sm.si_a, lane);
          if (fl && lane == 0) atomicOr(&sm.tie, B3_TIE_LIMIT);
        }
        sync_lds();
      }
      // slots nf + i <- token si_a[i]
      take_rows<T, HD>(sm, kread_w, krs, kp_copy, kr, v, kp, m,
                       [&](int i, int& j, int& s) {
                         j = sm.si_a[i];
                         s = nf + i;
                         return true;
                       },
                       tid);
      if (tid < m) {
        const int j = sm.si_a[tid], s = nf + tid;
        sm.pm[s] = sm.tpos[j];
        sm.mass[s] = 1.0f;
        sm.util[s] = sm.rel[j];
        sm.act[s] = 1;
        sm.vdirty[s] = 1;
        if (!kp_copy) sm.dirty[s] = 1;
      }
      if (log) {
        for (int j = tid; j < B3_LOG_COLS; j += DT) {
          log[B3_LOG_REL * B3_LOG_COLS + j] = j < l ? sm.rel[j] : 0.f;
          log[B3_LOG_SCORE * B3_LOG_COLS + j] = j < l ? sm.score[j] : 0.f;
          log[B3_LOG_TOPTOK * B3_LOG_COLS + j] = j < m ? (float)sm.si_a[j] : -1.f;
          log[B3_LOG_INFO * B3_LOG_COLS + j] = j == 0 ? (float)sm.tie : 0.f;
        }
      }
      nf += m;
      sync_lds();
    } else {
      const int any_merge = sm.any_merge;
      // ---------------- merge: per-slot mass-weighted means, tokens in ascending order
      if (any_merge) {
        // which tokens merge into which slot, as a bitmap [slot][token]
        constexpr int LW = LMAX / 32;
        for (int i = tid; i < S * LW; i += DT) (&sm.u.mg.bits[0][0])[i] = 0u;
        sync_lds();
        if (tid < l && (sm.flags[tid] & F_MERGE)) atomicOr(&sm.u.mg.bits[sm.slot[tid]][tid >> 5], 1u << (tid & 31));
        sync_lds();
        // per slot: count and position sum, its tokens in ascending order
        if (tid < S) {
          int c = 0;
          float ps = 0.f;
#pragma unroll
          for (int w = 0; w < LW; ++w) {
            unsigned m = sm.u.mg.bits[tid][w];
            while (m) {
              const int j = 32 * w + __builtin_ctz(m);
              m &= m - 1;
              ++c;
              ps += sm.tpos[j];
            }
          }
          sm.u.mg.cnt[tid] = c;
          sm.u.mg.psum[tid] = ps;
        }
        sync_lds();
        // slot offsets (exclusive prefix of the counts) and the hit slots in ascending order, by
        // wavefront 0 with two slots per lane
        static_assert(S == 2 * WAVE, "two slots per lane");
        if (wave == 0) {
          const int c0 = sm.u.mg.cnt[2 * lane], c1 = sm.u.mg.cnt[2 * lane + 1];
          const int hh = (c0 > 0 ? 1 : 0) + (c1 > 0 ? 1 : 0);
          int ic = c0 + c1, ih = hh;   // inclusive prefix sums over the lanes
#pragma unroll
          for (int o = 1; o < WAVE; o <<= 1) {
            const int tc = __shfl_up(ic, o, WAVE), th = __shfl_up(ih, o, WAVE);
            if (lane >= o) {
              ic += tc;
              ih += th;
            }
          }
          const int ec = ic - c0 - c1;
          int k = ih - hh;
          sm.u.mg.off[2 * lane] = ec;
          sm.u.mg.off[2 * lane + 1] = ec + c0;
          if (c0 > 0) sm.u.mg.hits[k++] = 2 * lane;
          if (c1 > 0) sm.u.mg.hits[k] = 2 * lane + 1;
          if (lane == WAVE - 1) sm.u.mg.nhit = ih;
        }
        sync_lds();
        const int nhit = sm.u.mg.nhit;
        // the merged tokens of each slot at its offset, in ascending order
        if (tid < S && sm.u.mg.cnt[tid] > 0) {
          int k = sm.u.mg.off[tid];
#pragma unroll
          for (int w = 0; w < LW; ++w) {
            unsigned m = sm.u.mg.bits[tid][w];
            while (m) {
              sm.u.mg.mlist[k++] = 32 * w + __builtin_ctz(m);
              m &= m - 1;
            }
          }
        }
        sync_lds();
        // one thread per (hit slot, 8 features): the merged rows in ascending token order, four
        // tokens' loads in flight at a time
        constexpr int NC8 = HD / 8;
        for (int it = tid; it < nhit * NC8; it += DT) {
          const int s = sm.u.mg.hits[it / NC8], d0 = 8 * (it % NC8);
          const int cnt = sm.u.mg.cnt[s], o0 = sm.u.mg.off[s];
          float ks[8], vs[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) ks[e] = vs[e] = 0.f;
          for (int q0 = 0; q0 < cnt; q0 += 4) {
            Vec8<T> kx[4], vx[4];   // rows kept in the storage dtype until they are added
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (q0 + u < cnt) {
                const int j = sm.u.mg.mlist[o0 + q0 + u];
                kx[u].load(kr + (long long)j * HD + d0);
                vx[u].load(v + (long long)j * HD + d0);
              }
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (q0 + u < cnt)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                  ks[e] += kx[u].get(e);
                  vs[e] += vx[u].get(e);
                }
          }
          const float m0 = sm.mass[s], nm = add_rn(m0, (float)cnt);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int d = d0 + e;
            sm.ak[s * KS + d] = St<T>::from_f(div_rn(add_rn(mul_rn(m0, St<T>::to_f(sm.ak[s * KS + d])), ks[e]), nm));
            sm.av[s * KS + d] = St<T>::from_f(div_rn(add_rn(mul_rn(m0, St<T>::to_f(sm.av[s * KS + d])), vs[e]), nm));
          }
        }
        sync_lds();
        if (tid < S && sm.u.mg.cnt[tid] > 0) {
          const float m0 = sm.mass[tid], nm = add_rn(m0, (float)sm.u.mg.cnt[tid]);
          sm.pm[tid] = div_rn(add_rn(mul_rn(m0, sm.pm[tid]), sm.u.mg.psum[tid]), nm);
          sm.mass[tid] = nm;
          sm.dirty[tid] = 1;
          sm.vdirty[tid] = 1;
        }
        sync_lds();
        slot_norms<T, HD>(sm, tid);
        sync_lds();
      }

      // ---------------- keep score: util * (1 - clamp(max_{s'!=s} cos(ak_s, ak_s'), 0, .98))
      {
        const int n = lane & 31;
        const int cb = wave & 3, rh = wave >> 2;
        const int col = 32 * cb + n;
        Frag<T, HD> fc;
        fc.load_lds(sm.ak, KS, col, lane);
        float mx = -INFINITY;
        bool has_nan = false;
        if constexpr (BF) {
          // operands of a block read together; inverse norms as float4 (rows 4*(r/4)+.. are
          // consecutive); NaN tracked through c*0
          const float inv_c = sm.inv_nak[col];
          const int h = lane >> 5;
          float chk = 0.f;
#pragma unroll
          for (int m2 = 0; m2 < 2; ++m2) {
            const int mb = 2 * rh + m2;
            u16x8 ab[HD / 16];
#pragma unroll
            for (int ks = 0; ks < HD / 16; ++ks)
              ab[ks] = *reinterpret_cast<const u16x8*>(&sm.ak[(32 * mb + n) * KS + 16 * ks + 8 * h]);
            f32x16 acc = zero16();
#pragma unroll
            for (int ks = 0; ks < HD / 16; ++ks) mma_bf16(acc, ab[ks], fc.v[ks]);
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
              const float4 i4 = *reinterpret_cast<const float4*>(&sm.inv_nak[32 * mb + 8 * r4 + 4 * h]);
              const float iv[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int row = 32 * mb + 8 * r4 + 4 * h + q;
                // one rounded product of the two inverse norms keeps the matrix bitwise
                // symmetric, so mutual nearest slots (equal utility) get bit-equal keep values
                const float c = row == col ? -1.0f : acc[4 * r4 + q] * (iv[q] * inv_c);
                chk = fmaf(c, 0.f, chk);
                mx = fmaxf(mx, c);
              }
            }
          }
          has_nan = chk != chk;
        } else {
#pragma unroll
          for (int m2 = 0; m2 < 2; ++m2) {
            const int mb = 2 * rh + m2;
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
        }
        mx = fmaxf(mx, xor32(mx));
        has_nan |= __shfl_xor((int)has_nan, 32, 64) != 0;
        if ((lane >> 5) == 0) {
          sm.u.kp.mx[rh][col] = mx;
          sm.u.kp.nan[rh][col] = has_nan ? 1 : 0;
        }
      }
      sync_lds();
      prefetch(step, wave, lane, 2);
      float keep_v = 0.f, ck_v = 0.f;   // keep value of slot tid, candidate value of token tid
      if (tid < S) {
        float mx = fmaxf(sm.u.kp.mx[0][tid], sm.u.kp.mx[1][tid]);
        if (sm.u.kp.nan[0][tid] | sm.u.kp.nan[1][tid]) mx = NAN;
        keep_v = mul_rn(sm.util[tid], 1.0f - fminf(fmaxf(mx, 0.0f), 0.98f));
        sm.keep[tid] = keep_v;
      }
      if (tid < l) {
        ck_v = cand_value(sm, tid);
      }
      sync_lds();
      if (tid < l) sm.u.ok.a[tid] = desc_key(ck_v, tid);
      if (tid < S) sm.u.ok.b[tid] = asc_key(keep_v, tid);
      sync_lds();
      // ---------------- orderings: best free tokens (desc) against least useful slots (asc)
      {
        // l + S items, two threads each, each counting half of the keys
        const int item = tid >> 1, part = tid & 1;
        for (int base = 0; base < l + S; base += DT / 2) {
          const int it = base + item;
          int r = 0;
          if (it < l) {
            const int mid = (l >> 1) & ~1;
            r = count_above(sm.u.ok.a, part ? mid : 0, part ? l : mid, sm.u.ok.a[it]);
          } else if (it < l + S) {
            r = count_below(sm.u.ok.b, part ? S / 2 : 0, part ? S : S / 2, sm.u.ok.b[it - l]);
          }
          r += __shfl_xor(r, 1, 64);
          if (part == 0) {
            if (it < l) {
              sm.sk_a[r] = cand_value(sm, it);
              sm.si_a[r] = it;
            } else if (it < l + S) {
              sm.sk_b[r] = sm.keep[it - l];
              sm.si_b[r] = it - l;
            }
          }
        }
      }
      sync_lds();
      prefetch(step, wave, lane, 4);
      const int kc = min(l, S);
      // Exactly equal values where they decide a swap (win_i is a prefix of the ranks, and the
      // values by rank do not depend on the order among equal ones): the reference's order.
      if (tid < kc && sm.sk_a[tid] > sm.sk_b[tid] && sm.sk_a[tid] > -1e8f) {
        if (tie_at(sm.sk_a, tid, l)) atomicOr(&sm.tie, B3_TIE_TOP);
        if (tie_at(sm.sk_b, tid, S)) atomicOr(&sm.tie, B3_TIE_BOT);
      }
      sync_lds();
      if (const int tie = sm.tie) {
        int fl = 0;
        if (wave == 0 && (tie & B3_TIE_TOP)) {
          for (int j = lane; j < l; j += WAVE)
            sm.u.to.e[0][j] = ((uint64_t)tie_key(cand_value(sm, j), true) << 32) | (uint32_t)j;
          fl = tie_order_wave(sm.u.to.e[0], sm.u.to.pr[0], sm.u.to.stk[0], l, kc, sm.si_a, lane);
        }
        if (wave == 1 && (tie & B3_TIE_BOT)) {
          for (int j = lane; j < S; j += WAVE)
            sm.u.to.e[1][j] = ((uint64_t)tie_key(sm.keep[j], false) << 32) | (uint32_t)j;
          fl = tie_order_wave(sm.u.to.e[1], sm.u.to.pr[1], sm.u.to.stk[1], S, kc, sm.si_b, lane);
        }
        if (fl && lane == 0) atomicOr(&sm.tie, B3_TIE_LIMIT);
        sync_lds();
      }
      // win_i = top_i > bot_i and top_i > -1e8 ; token top_i replaces slot bot_i
      if (tid < kc) {
        const float tv = sm.sk_a[tid], bv = sm.sk_b[tid];
        if (tv > bv && tv > -1e8f) {
          const int j = sm.si_a[tid], s = sm.si_b[tid];
          sm.flags[j] |= F_INS;
          sm.pm[s] = sm.tpos[j];
          sm.mass[s] = 1.0f;
          sm.util[s] = sm.rel[j];
          sm.vdirty[s] = 1;
          if (!kp_copy) sm.dirty[s] = 1;
        }
      }
      take_rows<T, HD>(sm, kread_w, krs, kp_copy, kr, v, kp, kc,
                       [&](int i, int& j, int& s) {
                         const float tv = sm.sk_a[i], bv = sm.sk_b[i];
                         j = sm.si_a[i];
                         s = sm.si_b[i];
                         return tv > bv && tv > -1e8f;
                       },
                       tid);
      sync_lds();
      if (tid < l) {
        const int f = sm.flags[tid];
        const bool dl = !(f & F_MERGE) && !(f & F_INS);
        if (dl) sm.flags[tid] = f | F_DELTA;
        w_out[tid] = dl ? sm.tbeta[tid] : 0.f;
      }
      sync_lds();
      if (log) {
        for (int j = tid; j < B3_LOG_COLS; j += DT) {
          const bool in = j < l;
          log[B3_LOG_REL * B3_LOG_COLS + j] = in ? sm.rel[j] : 0.f;
          log[B3_LOG_SCORE * B3_LOG_COLS + j] = in ? sm.score[j] : 0.f;
          if (!in) {
            log[B3_LOG_BEST * B3_LOG_COLS + j] = 0.f;
            log[B3_LOG_SIMV * B3_LOG_COLS + j] = 0.f;
          }
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
          log[B3_LOG_INFO * B3_LOG_COLS + j] = j == 0 ? (float)sm.tie : 0.f;
        }
      }
    }

    // ---------------- per-step outputs; the roped keys also serve the next step
    rope_dirty<T, HD>(sm, kread_g, tid);
    transpose_dirty_v<T, HD>(sm, tid);
    if constexpr (DecSmem<T, HD>::KREAD_LDS) {
      sync_lds();
    } else {
      __threadfence_block();   // roped keys in the workspace are read by other threads
      __syncthreads();
    }
    if (a.snap_k) {
      T* kd = reinterpret_cast<T*>(a.snap_k) + (step * BH + bh) * S * HD;
      for (int it = tid; it < S * (HD / 8); it += DT) {
        const int s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
        copy8(kd + s * HD + d8, kread + s * krs + d8);
      }
    }
    if (a.snap_v) {
      T* vd = reinterpret_cast<T*>(a.snap_v) + (step * BH + bh) * S * HD;
      for (int it = tid; it < S * (HD / 8); it += DT) {
        const int s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
        copy8(vd + s * HD + d8, &sm.av[s * KS + d8]);
      }
    }
    if (a.snap_bias && tid < S) {
      a.snap_bias[(step * BH + bh) * S + tid] =
          sm.act[tid] ? mul_rn(kap, logf(fmaxf(sm.mass[tid], 1.0f))) : -INFINITY;
    }
    if (a.snap_mass && tid < S) a.snap_mass[(step * BH + bh) * S + tid] = sm.mass[tid];
    if (a.snap_pm && tid < S) a.snap_pm[(step * BH + bh) * S + tid] = sm.pm[tid];
  }

  // store the slot state
  for (int it = tid; it < S * (HD / 8); it += DT) {
    const int s = it / (HD / 8), d8 = (it % (HD / 8)) * 8;
    copy8(g_ak + s * HD + d8, &sm.ak[s * KS + d8]);
    copy8(g_av + s * HD + d8, &sm.av[s * KS + d8]);
  }
  if (tid < S) {
    a.mass[bh * S + tid] = sm.mass[tid];
    a.util[bh * S + tid] = sm.util[tid];
    a.pm[bh * S + tid] = sm.pm[tid];
    a.act[bh * S + tid] = (uint8_t)sm.act[tid];
  }
}

// ----------------------------------------------------------------- gersh_kernel

// For steady step blockIdx.x and row blockIdx.y:
//   inv_j   = 1 / max(|k_j|, 1e-12)
//   bsafe_j = w_j / max(sum_i |khat_i . khat_j| w_i, 1)
// bf16: the step's keys come into LDS once (thread t stages row t and takes its 1/|k| from the
// same registers), 16-byte piece p of row r at p ^ (r % (HD/8)), and the products read their
// operands there: one global round trip per workgroup.  The products and the summation order
// are those of the fp32-storage path below.
template <int HD>
__device__ __forceinline__ void gersh_bf16(const b3_chain_args& a, const uint16_t* kr, const float* w, float* bsafe,
                                           float* inv, int l) {
  constexpr int NP = HD / 8;
  extern __shared__ __attribute__((aligned(16))) unsigned char gsm_raw[];
  uint16_t* kt = reinterpret_cast<uint16_t*>(gsm_raw);   // [32 * ceil(l / 32)][HD]
  __shared__ float s_inv[LMAX], s_w[LMAX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 31, h = lane >> 5;
  const int nT = (l + 31) / 32;
  if (tid < 32 * nT) {
    u16x8 x[NP];
    if (tid < l) {
#pragma unroll
      for (int p = 0; p < NP; ++p) x[p] = *reinterpret_cast<const u16x8*>(kr + (long long)tid * HD + 8 * p);
    } else {
#pragma unroll
      for (int p = 0; p < NP; ++p) x[p] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    const float wv = tid < l ? w[tid] : 0.f;
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float f = bf2f(x[p][i]);
        ss += f * f;
      }
#pragma unroll
    for (int p = 0; p < NP; ++p) *reinterpret_cast<u16x8*>(&kt[tid * HD + 8 * (p ^ (tid % NP))]) = x[p];
    if (tid < l) {
      const float iv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      s_inv[tid] = iv;
      s_w[tid] = wv;
      inv[tid] = iv;
    }
  }
  __syncthreads();
  auto piece = [&](int r, int p) { return *reinterpret_cast<const u16x8*>(&kt[r * HD + 8 * (p ^ (r % NP))]); };
  for (int tj = wave; tj < nT; tj += MWAVES) {
    const int j = 32 * tj + n;
    u16x8 fj[HD / 16];
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) fj[ks] = piece(j, 2 * ks + h);
    const float inj = j < l ? s_inv[j] : 0.f;
    float colsum = 0.f;
    for (int ti = 0; ti < nT; ++ti) {
      f32x16 acc = zero16();
#pragma unroll
      for (int ks = 0; ks < HD / 16; ++ks) mma_bf16(acc, piece(32 * ti + n, 2 * ks + h), fj[ks]);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * ti + d_row(lane, r);
        if (i < l) colsum += fabsf(acc[r] * (s_inv[i] * inj)) * s_w[i];
      }
    }
    colsum += xor32(colsum);
    if (h == 0 && j < l) bsafe[j] = s_w[j] / fmaxf(colsum, 1.0f);
  }
}

template <typename T, int HD>
__global__ void __launch_bounds__(MT) gersh_kernel(b3_chain_args a) {
  const int step = blockIdx.x, bh = blockIdx.y;
  int nf = a.n_filled;
  for (int s = 0; s < step && nf < S; ++s) nf += min(S - nf, step_len(a, s));
  if (nf < S) return;  // fill step: M_res untouched
  const long long BH = (long long)a.B * a.HKV;
  const int l = step_len(a, step);
  const T* kr =
      reinterpret_cast<const T*>(a.kr) + (long long)bh * a.tok_bh_stride + (long long)step_off(a, step) * HD;
  char* ws = reinterpret_cast<char*>(a.work) + BH * Work<T, HD>::KREAD;
  const long long row = ((long long)step * BH + bh) * LMAX;
  const long long plane = (long long)a.n_steps * BH * LMAX;
  const float* w = reinterpret_cast<const float*>(ws) + row;
  float* bsafe = reinterpret_cast<float*>(ws) + plane + row;
  float* inv = reinterpret_cast<float*>(ws) + 2 * plane + row;
  if constexpr (St<T>::is_bf16) {
    gersh_bf16<HD>(a, kr, w, bsafe, inv, l);
  } else {
    __shared__ float s_inv[LMAX], s_w[LMAX];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 31;
    if (tid < l) {
      float ss = 0.f;
      for (int d = 0; d < HD; d += 8) {
        float x[8];
        ld8(kr + (long long)tid * HD + d, x);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
      }
      const float iv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
      s_inv[tid] = iv;
      s_w[tid] = w[tid];
      inv[tid] = iv;
    }
    __syncthreads();
    const int nT = (l + 31) / 32;
    for (int tj = wave; tj < nT; tj += MWAVES) {
      const int j = 32 * tj + n;
      Frag<T, HD> fj;
      fj.load(kr, j, l, lane);
      const float inj = j < l ? s_inv[j] : 0.f;
      float colsum = 0.f;
      for (int ti = 0; ti < nT; ++ti) {
        f32x16 acc = zero16();
        Frag<T, HD> fi;
        fi.load(kr, 32 * ti + n, l, lane);
        // rows i of tile ti as the A operand: same fragment layout as a B fragment
#pragma unroll 8
        for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, fi.v[ks], fj.v[ks]);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 32 * ti + d_row(lane, r);
          if (i < l) colsum += fabsf(acc[r] * (s_inv[i] * inj)) * s_w[i];
        }
      }
      colsum += xor32(colsum);
      if ((lane >> 5) == 0 && j < l) bsafe[j] = s_w[j] / fmaxf(colsum, 1.0f);
    }
  }
}

// ----------------------------------------------------------------- mres_kernel

template <typename T, int HD>
struct MSmem {
  static constexpr int MS = HD + 4;                               // fp32 M^T row stride
  static constexpr int BS = HD + 8;                               // bf16 M^T row stride
  static constexpr int ES = sizeof(T) == 2 ? LMAX + 8 : LMAX + 1; // E^T row stride
  static constexpr int KC = 128;                                  // tokens per K^T staging chunk
  static constexpr int KTS = sizeof(T) == 2 ? KC + 8 : KC + 1;    // K^T row stride
  alignas(16) float mt[32 * MS];                                  // M^T rows d of this block
  alignas(16) uint16_t mhi[sizeof(T) == 2 ? 32 * BS : 1];
  alignas(16) uint16_t mlo[sizeof(T) == 2 ? 32 * BS : 1];
  alignas(16) T ert[32 * ES];                                     // E^T[d][j] (bf16: hi)
  alignas(16) uint16_t erl[sizeof(T) == 2 ? 32 * ES : 1];         // E^T lo
  alignas(16) T krt[HD * KTS];                                    // K^T[c][j] of one chunk
  float bsafe[LMAX], inv[LMAX];
};

// Global inputs of one step for one thread of mres_kernel when the step has at most
// MSmem::KC tokens: the token tile of wave w (tokens 32w..32w+31: key fragment, values of
// the column block, 1/|k| and bsafe) and one 8 x 8 block of keys for the K^T staging.
template <typename T, int HD>
struct MStepIn {
  Frag<T, HD> fj;
  V4<T> vx[4];
  float inj, bj;
  T kb[8][8];
  __device__ __forceinline__ void load(const T* kr, const T* v, const float* inv, const float* bsafe, int l, int db,
                                       int tid, int lane, int wave) {
    const int n = lane & 31, h = lane >> 5, j = 32 * wave + n;
    fj.load(kr, j, l, lane);
#pragma unroll
    for (int g = 0; g < 4; ++g) vx[g].load(v + (long long)j * HD + 32 * db + 8 * g + 4 * h, j < l);
    inj = j < l ? inv[j] : 0.f;
    bj = j < l ? bsafe[j] : 0.f;
    constexpr int KC = 128;
    const int jb = (tid % (KC / 8)) * 8, c8 = (tid / (KC / 8)) * 8;
    if (tid < (KC / 8) * (HD / 8)) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        if (jb + r < l) copy8(kb[r], kr + (long long)(jb + r) * HD + c8);
        else {
#pragma unroll
          for (int q = 0; q < 8; ++q) kb[r][q] = St<T>::from_f(0.f);
        }
      }
    }
  }
};

// Columns [32*db, 32*db + 32) of M for row bh (workgroup bh * (HD/32) + db in XCD-aware order):
//   E^T[d][j] = (v[j][d] - (K M)[j][d] / |k_j|) * bsafe_j / |k_j|
//   M^T[d][c] <- gamma * M^T[d][c] + sum_j E^T[d][j] k[j][c]
// Steps of at most 128 tokens (every forward and decoder step) keep the next step's inputs
// in registers across LDS-only barriers; longer steps load per chunk.
template <typename T, int HD>
__global__ void __launch_bounds__(MT) mres_kernel(b3_chain_args a) {
  __shared__ MSmem<T, HD> sm;
  using Sm = MSmem<T, HD>;
  constexpr int NDB = HD / 32, NCB = HD / 32;
  // XCD-aware order: the NDB column blocks of one bh read the same keys and values
  const int wg = xcd_grid_pos().x;
  const int bh = wg / NDB, db = wg % NDB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 31, h = lane >> 5;
  const int hkv = bh % a.HKV;
  const float gam = a.gamma[hkv];
  const long long BH = (long long)a.B * a.HKV;
  float* M = a.m_res + (long long)bh * HD * HD;
  const char* ws = reinterpret_cast<const char*>(a.work) + BH * Work<T, HD>::KREAD;
  const long long plane = (long long)a.n_steps * BH * LMAX;
  const float* bsafe_all = reinterpret_cast<const float*>(ws) + plane;
  const float* inv_all = reinterpret_cast<const float*>(ws) + 2 * plane;
  auto tok_base = [&](int step) { return (long long)bh * a.tok_bh_stride + (long long)step_off(a, step) * HD; };
  auto row_base = [&](int step) { return ((long long)step * BH + bh) * LMAX; };

  // M^T block: mt[dd][c] = M[c][32*db + dd]; every load of the thread before its stores (one
  // memory round trip)
  constexpr int NMI = HD * 32 / MT;
  static_assert(NMI * MT == HD * 32, "M^T block over the threads");
  float mx[NMI];
#pragma unroll
  for (int q = 0; q < NMI; ++q) {
    const int it = tid + MT * q, c = it / 32, dd = it % 32;
    mx[q] = a.n_filled == 0 ? 0.0f : M[c * HD + 32 * db + dd];   // empty state: M_res = 0
  }
#pragma unroll
  for (int q = 0; q < NMI; ++q) {
    const int it = tid + MT * q, c = it / 32, dd = it % 32;
    const float x = mx[q];
    sm.mt[dd * Sm::MS + c] = x;
    if constexpr (St<T>::is_bf16) {
      const uint16_t hb = f2bf(x);
      sm.mhi[dd * Sm::BS + c] = hb;
      sm.mlo[dd * Sm::BS + c] = f2bf(x - bf2f(hb));
    }
  }
  __syncthreads();

  // steady steps and whether their inputs are prefetched
  int nf = a.n_filled;
  int first_steady = -1;
  {
    int f = nf;
    for (int s = 0; s < a.n_steps && first_steady < 0; ++s) {
      if (f >= S) first_steady = s;
      else f += min(S - f, step_len(a, s));
    }
  }
  MStepIn<T, HD> in;
  bool in_ready = false;
  auto fetch = [&](int step) {   // step must be steady with at most KC tokens; bf16 only (registers)
    if constexpr (St<T>::is_bf16) {
      const long long tb = tok_base(step), row = row_base(step);
      in.load(reinterpret_cast<const T*>(a.kr) + tb, reinterpret_cast<const T*>(a.v) + tb, inv_all + row,
              bsafe_all + row, step_len(a, step), db, tid, lane, wave);
      in_ready = true;
    }
  };
  if (first_steady >= 0 && step_len(a, first_steady) <= Sm::KC) fetch(first_steady);

  for (int step = 0; step < a.n_steps; ++step) {
    const int l = step_len(a, step);
    float* snap = a.snap_m ? a.snap_m + (step * BH + bh) * HD * HD : nullptr;
    if (nf >= S) {
      const long long tb = tok_base(step);
      const T* kr = reinterpret_cast<const T*>(a.kr) + tb;
      const T* v = reinterpret_cast<const T*>(a.v) + tb;
      f32x16 upd = zero16();
      const int cb = wave;
      if (St<T>::is_bf16 && l <= Sm::KC && in_ready) {
        // ---- E^T for this wave's tile; K^T staging from registers
        {
          const int j = 32 * wave + n;
          f32x16 acc = zero16();
          if constexpr (St<T>::is_bf16) {
#pragma unroll
            for (int ks = 0; ks < HD / 16; ++ks) {
              const u16x8 hi = *reinterpret_cast<const u16x8*>(&sm.mhi[n * Sm::BS + 16 * ks + 8 * h]);
              const u16x8 lo = *reinterpret_cast<const u16x8*>(&sm.mlo[n * Sm::BS + 16 * ks + 8 * h]);
              mma_bf16(acc, hi, in.fj.v[ks]);
              mma_bf16(acc, lo, in.fj.v[ks]);
            }
          } else {
#pragma unroll 8
            for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, sm.mt[n * Sm::MS + 2 * ks + h], in.fj.v[ks]);
          }
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int dd = 8 * g + 4 * h + q;
              const float e = ((in.vx[g].get(q) - acc[4 * g + q] * in.inj) * in.bj) * in.inj;
              if constexpr (St<T>::is_bf16) {
                const uint16_t hb = f2bf(e);
                sm.ert[dd * Sm::ES + j] = hb;
                sm.erl[dd * Sm::ES + j] = f2bf(e - bf2f(hb));
              } else {
                sm.ert[dd * Sm::ES + j] = e;
              }
            }
          if (tid < (Sm::KC / 8) * (HD / 8)) {
            const int jb = (tid % (Sm::KC / 8)) * 8, c8 = (tid / (Sm::KC / 8)) * 8;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              if constexpr (St<T>::is_bf16) {
                u16x8 col;
#pragma unroll
                for (int r = 0; r < 8; ++r) col[r] = in.kb[r][q];
                *reinterpret_cast<u16x8*>(&sm.krt[(c8 + q) * Sm::KTS + jb]) = col;
              } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) sm.krt[(c8 + q) * Sm::KTS + jb + r] = in.kb[r][q];
              }
            }
          }
        }
        in_ready = false;
        // the next steady step's inputs load while this one finishes
        if (step + 1 < a.n_steps && step_len(a, step + 1) <= Sm::KC) fetch(step + 1);
        sync_lds();
        if (cb < NCB) {
          const int c = 32 * cb + n;
          if constexpr (St<T>::is_bf16) {
#pragma unroll
            for (int kc = 0; kc < Sm::KC / 16; ++kc) {
              const u16x8 ka = *reinterpret_cast<const u16x8*>(&sm.krt[c * Sm::KTS + 16 * kc + 8 * h]);
              const u16x8 eh = *reinterpret_cast<const u16x8*>(&sm.ert[n * Sm::ES + 16 * kc + 8 * h]);
              const u16x8 el = *reinterpret_cast<const u16x8*>(&sm.erl[n * Sm::ES + 16 * kc + 8 * h]);
              mma_bf16(upd, ka, eh);
              mma_bf16(upd, ka, el);
            }
          } else {
#pragma unroll 8
            for (int kc = 0; kc < Sm::KC / 2; ++kc)
              mma_f32(upd, sm.krt[c * Sm::KTS + 2 * kc + h], sm.ert[n * Sm::ES + 2 * kc + h]);
          }
        }
      } else {
        // ---- general path (steps longer than KC tokens)
        const long long row = row_base(step);
        const int nT = ((l + Sm::KC - 1) / Sm::KC) * (Sm::KC / 32);
        for (int t = wave; t < nT; t += MWAVES) {
          const int j = 32 * t + n;
          Frag<T, HD> fj;
          fj.load(kr, j, l, lane);
          V4<T> vx[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) vx[g].load(v + (long long)j * HD + 32 * db + 8 * g + 4 * h, j < l);
          f32x16 acc = zero16();
          if constexpr (St<T>::is_bf16) {
#pragma unroll
            for (int ks = 0; ks < HD / 16; ++ks) {
              const u16x8 hi = *reinterpret_cast<const u16x8*>(&sm.mhi[n * Sm::BS + 16 * ks + 8 * h]);
              const u16x8 lo = *reinterpret_cast<const u16x8*>(&sm.mlo[n * Sm::BS + 16 * ks + 8 * h]);
              mma_bf16(acc, hi, fj.v[ks]);
              mma_bf16(acc, lo, fj.v[ks]);
            }
          } else {
#pragma unroll 8
            for (int ks = 0; ks < HD / 2; ++ks) mma_f32(acc, sm.mt[n * Sm::MS + 2 * ks + h], fj.v[ks]);
          }
          const float inj = j < l ? inv_all[row + j] : 0.f;
          const float bj = j < l ? bsafe_all[row + j] : 0.f;
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int dd = 8 * g + 4 * h + q;
              const float e = ((vx[g].get(q) - acc[4 * g + q] * inj) * bj) * inj;
              if constexpr (St<T>::is_bf16) {
                const uint16_t hb = f2bf(e);
                sm.ert[dd * Sm::ES + j] = hb;
                sm.erl[dd * Sm::ES + j] = f2bf(e - bf2f(hb));
              } else {
                sm.ert[dd * Sm::ES + j] = e;
              }
            }
        }
        for (int j0 = 0; j0 < l; j0 += Sm::KC) {
          const int jn = min(Sm::KC, l - j0);
          for (int it = tid; it < (Sm::KC / 8) * (HD / 8); it += MT) {
            const int jb = (it % (Sm::KC / 8)) * 8, c8 = (it / (Sm::KC / 8)) * 8;
            float x[8][8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              if (jb + r < jn) ld8(kr + (long long)(j0 + jb + r) * HD + c8, x[r]);
              else {
#pragma unroll
                for (int q = 0; q < 8; ++q) x[r][q] = 0.f;
              }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              if constexpr (St<T>::is_bf16) {
                u16x8 col;
#pragma unroll
                for (int r = 0; r < 8; ++r) col[r] = f2bf(x[r][q]);
                *reinterpret_cast<u16x8*>(&sm.krt[(c8 + q) * Sm::KTS + jb]) = col;
              } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) sm.krt[(c8 + q) * Sm::KTS + jb + r] = x[r][q];
              }
            }
          }
          sync_lds();
          if (cb < NCB) {
            const int c = 32 * cb + n;
            if constexpr (St<T>::is_bf16) {
#pragma unroll
              for (int kc = 0; kc < Sm::KC / 16; ++kc) {
                const u16x8 ka = *reinterpret_cast<const u16x8*>(&sm.krt[c * Sm::KTS + 16 * kc + 8 * h]);
                const u16x8 eh = *reinterpret_cast<const u16x8*>(&sm.ert[n * Sm::ES + j0 + 16 * kc + 8 * h]);
                const u16x8 el = *reinterpret_cast<const u16x8*>(&sm.erl[n * Sm::ES + j0 + 16 * kc + 8 * h]);
                mma_bf16(upd, ka, eh);
                mma_bf16(upd, ka, el);
              }
            } else {
#pragma unroll 8
              for (int kc = 0; kc < Sm::KC / 2; ++kc)
                mma_f32(upd, sm.krt[c * Sm::KTS + 2 * kc + h], sm.ert[n * Sm::ES + j0 + 2 * kc + h]);
            }
          }
          sync_lds();
        }
      }
      // M = gamma*M + upd (two rounded ops, as the reference evaluates them); lane holds
      // column d = n of the block and rows c = 32*cb + d_row(lane, r)
      if (cb < NCB) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = 32 * cb + d_row(lane, r);
          const float nw = add_rn(mul_rn(gam, sm.mt[n * Sm::MS + c]), upd[r]);
          sm.mt[n * Sm::MS + c] = nw;
          if constexpr (St<T>::is_bf16) {
            const uint16_t hb = f2bf(nw);
            sm.mhi[n * Sm::BS + c] = hb;
            sm.mlo[n * Sm::BS + c] = f2bf(nw - bf2f(hb));
          }
        }
      }
      sync_lds();
    } else {
      nf += min(S - nf, l);
    }
    // snapshot of this block after the step (a fill step leaves M unchanged)
    if (snap) {
      if constexpr (St<T>::is_bf16) {
        uint16_t* sh = reinterpret_cast<uint16_t*>(snap);
        for (int it = tid; it < 32 * (HD / 8); it += MT) {
          const int dd = it / (HD / 8), c8 = (it % (HD / 8)) * 8;
          const int d = 32 * db + dd;
          copy8(sh + d * HD + c8, &sm.mhi[dd * Sm::BS + c8]);
          copy8(sh + HD * HD + d * HD + c8, &sm.mlo[dd * Sm::BS + c8]);
        }
      } else {
        for (int it = tid; it < HD * 32; it += MT) {
          const int c = it / 32, dd = it % 32;
          snap[c * HD + 32 * db + dd] = sm.mt[dd * Sm::MS + c];
        }
      }
    }
  }
  for (int it = tid; it < HD * 32; it += MT) {
    const int c = it / 32, dd = it % 32;
    M[c * HD + 32 * db + dd] = sm.mt[dd * Sm::MS + c];
  }
}

// Holds its stream until *counter reaches target (modulo 2^32) or after max_polls polls.
__global__ void __launch_bounds__(64) wait_count_kernel(const uint32_t* counter, uint32_t target, int max_polls) {
  for (int i = 0; i < max_polls; ++i) {
    const uint32_t c = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((int32_t)(c - target) >= 0) break;
    __builtin_amdgcn_s_sleep(8);
  }
}

// Roped slot keys and attention bias of a slot state, with the chain's own rounding: one
// workgroup per bh, 8 rotation pairs per item (the per-step snapshot the decode step reads).
template <typename T, int HD>
__global__ void __launch_bounds__(MT) slot_keys_kernel(b3_slot_keys_args a) {
  constexpr int HALF = HD / 2, P8 = HALF / 8;
  const int bh = blockIdx.x, hkv = bh % a.HKV;
  const T* ak = reinterpret_cast<const T*>(a.ak) + (long long)bh * S * HD;
  T* dst = reinterpret_cast<T*>(a.slot_k) + (long long)bh * S * HD;
  for (int it = threadIdx.x; it < S * P8; it += MT) {
    const int s = it / P8, i0 = (it % P8) * 8;
    float x0[8], x1[8];
    ld8(ak + s * HD + i0, x0);
    ld8(ak + s * HD + i0 + HALF, x1);
    const float p = a.pm[bh * S + s];
    alignas(16) T r0[8];
    alignas(16) T r1[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float sn, cs;
      sincos_rope(mul_rn(p, a.inv_freq[i0 + q]), &sn, &cs);
      const float c = St<T>::rnd(cs), si = St<T>::rnd(sn);
      r0[q] = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x0[q], c)), St<T>::rnd(mul_rn(-x1[q], si))));
      r1[q] = St<T>::from_f(add_rn(St<T>::rnd(mul_rn(x1[q], c)), St<T>::rnd(mul_rn(x0[q], si))));
    }
    copy8(dst + s * HD + i0, r0);
    copy8(dst + s * HD + i0 + HALF, r1);
  }
  for (int s = threadIdx.x; s < S; s += MT)
    a.slot_bias[bh * S + s] = a.act[bh * S + s] ? mul_rn(a.kappa[hkv], logf(fmaxf(a.mass[bh * S + s], 1.0f)))
                                                : -INFINITY;
}

template <typename T, int HD>
static int launch_chain(const b3_chain_args& a, hipStream_t st) {
  const int BH = a.B * a.HKV;
  if (a.phase != 2) {
    hipLaunchKernelGGL((decide_kernel<T, HD>), dim3(BH), dim3(DT), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.phase == 1) return (int)e;
  }
  // bf16: LDS for the longest step's keys, rows padded to a multiple of 32
  const int lmax = a.n_steps > 1 ? std::max(a.len0, a.step_len) : a.len0;
  const size_t gsm = St<T>::is_bf16 ? (size_t)32 * ((lmax + 31) / 32) * HD * sizeof(T) : 0;
  hipLaunchKernelGGL((gersh_kernel<T, HD>), dim3(a.n_steps, BH), dim3(MT), gsm, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((mres_kernel<T, HD>), dim3(BH * (HD / 32)), dim3(MT), 0, st, a);
  return (int)hipGetLastError();
}

// ----------------------------------------------------------------- allocation-free entry
//
// bolt3_chain_noalloc takes its workspace from this file-scope array instead of the caller.
// Host code never uses the array's name as an address: the device address of each GPU's copy
// comes from hipGetSymbolAddress, taken once per device (with that device current) on the
// first call there.
static __device__ __align__(256) uint8_t scratch[B3_CHAIN_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES];

static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return B3_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return B3_ERR_UNSUPPORTED;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return B3_OK;
}

}  // namespace b3

extern "C" int64_t bolt3_chain_workspace_bytes(int32_t dtype, int32_t B, int32_t HKV, int32_t HD, int32_t S,
                                               int32_t n_steps) {
  const int64_t bh = (int64_t)B * HKV;
  if (dtype == B3_BF16)
    return HD == 64 ? b3::Work<uint16_t, 64>::bytes(bh, n_steps) : b3::Work<uint16_t, 128>::bytes(bh, n_steps);
  return HD == 64 ? b3::Work<float, 64>::bytes(bh, n_steps) : b3::Work<float, 128>::bytes(bh, n_steps);
}

extern "C" int bolt3_wait_count(const uint32_t* counter, uint32_t target, int32_t max_polls, void* stream) {
  if (!counter || max_polls < 0) return B3_ERR_ARG;
  hipLaunchKernelGGL(b3::wait_count_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), counter,
                     target, max_polls);
  return (int)hipGetLastError();
}

extern "C" int bolt3_chain(const b3_chain_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->n_steps < 0) return B3_ERR_ARG;
  if (a->S != b3::S || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  if (a->n_steps == 0) return B3_OK;
  if (a->len0 < 1 || a->len0 > b3::LMAX || (a->n_steps > 1 && (a->step_len < 1 || a->step_len > b3::LMAX)))
    return B3_ERR_UNSUPPORTED;
  if (a->n_filled < 0 || a->n_filled > b3::S || a->phase < 0 || a->phase > 2) return B3_ERR_ARG;
  if (!a->kr || !a->kp || !a->v || !a->pos || !a->beta || !a->ak || !a->av || !a->mass || !a->util || !a->pm ||
      !a->act || !a->m_res || !a->kappa || !a->gamma || !a->inv_freq || !a->work)
    return B3_ERR_ARG;
  if (a->work_bytes < bolt3_chain_workspace_bytes(a->dtype, a->B, a->HKV, a->HD, a->S, a->n_steps))
    return B3_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == B3_F32) return a->HD == 64 ? b3::launch_chain<float, 64>(*a, st) : b3::launch_chain<float, 128>(*a, st);
  if (a->dtype == B3_BF16)
    return a->HD == 64 ? b3::launch_chain<uint16_t, 64>(*a, st) : b3::launch_chain<uint16_t, 128>(*a, st);
  return B3_ERR_UNSUPPORTED;
}

extern "C" int bolt3_slot_keys(const b3_slot_keys_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0) return B3_ERR_ARG;
  if (a->S != b3::S || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  if (!a->ak || !a->pm || !a->mass || !a->act || !a->kappa || !a->inv_freq || !a->slot_k || !a->slot_bias)
    return B3_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(a->B * a->HKV), block(b3::MT);
  if (a->dtype == B3_F32) {
    if (a->HD == 64) hipLaunchKernelGGL((b3::slot_keys_kernel<float, 64>), grid, block, 0, st, *a);
    else hipLaunchKernelGGL((b3::slot_keys_kernel<float, 128>), grid, block, 0, st, *a);
  } else if (a->dtype == B3_BF16) {
    if (a->HD == 64) hipLaunchKernelGGL((b3::slot_keys_kernel<uint16_t, 64>), grid, block, 0, st, *a);
    else hipLaunchKernelGGL((b3::slot_keys_kernel<uint16_t, 128>), grid, block, 0, st, *a);
  } else {
    return B3_ERR_UNSUPPORTED;
  }
  return (int)hipGetLastError();
}

extern "C" int bolt3_chain_noalloc(const b3_chain_args* a, void* stream) {
  if (!a || a->B <= 0 || a->HKV <= 0 || a->n_steps < 0) return B3_ERR_ARG;
  if (a->S != b3::S || (a->HD != 64 && a->HD != 128)) return B3_ERR_UNSUPPORTED;
  if (a->dtype != B3_F32 && a->dtype != B3_BF16) return B3_ERR_UNSUPPORTED;
  if (bolt3_chain_workspace_bytes(a->dtype, a->B, a->HKV, a->HD, a->S, a->n_steps) > B3_CHAIN_NOALLOC_SCRATCH_BYTES)
    return B3_ERR_WORKSPACE;
  void* p = nullptr;
  const int rc = b3::scratch_address(&p);
  if (rc != B3_OK) return rc;
  b3_chain_args c = *a;
  c.work = p;
  c.work_bytes = B3_CHAIN_NOALLOC_SCRATCH_BYTES;
  return bolt3_chain(&c, stream);
}

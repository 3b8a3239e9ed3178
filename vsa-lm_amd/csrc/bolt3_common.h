// Shared device helpers for the Bolt-3 gfx950 kernels.
//
// Matrix products use the CDNA3/CDNA4 32x32 MFMA family.  For every variant
// used here the accumulator ("D") layout is the same: lane l of the 64-wide
// wavefront holds column n = l % 32 and rows
//     m(l, r) = 8 * (r / 4) + 4 * (l / 32) + (r % 4),   r = 0..15.
// The A operand holds row m = l % 32 and the B operand column n = l % 32; both
// carry the same K sub-index k(l, i), so any K permutation that A and B agree
// on gives the same product.  bf16 products are exact in fp32, which lets a
// bf16 operand pair reproduce fp32 dot products of bf16 data bit-for-bit up to
// summation order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace b3 {

// Grid position in XCD-aware order.  Consecutive workgroups go to the 8 XCDs in turn, so
// linear id L runs task (L % 8) * (N / 8) + L / 8 of the x-fastest grid order: neighbouring
// tasks (which read the same tiles) share one XCD's L2.  Identity when the grid size N is not
// a multiple of 8.
struct GridPos { int x, y, z; };
__device__ __forceinline__ GridPos xcd_grid_pos() {
  const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
  int wg = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int n = gx * gy * gz;
  if (n % 8 == 0) wg = (wg % 8) * (n / 8) + wg / 8;
  return GridPos{wg % gx, (wg / gx) % gy, wg / (gx * gy)};
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// ---------------------------------------------------------------- bf16 <-> f32

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Round-to-nearest-even (torch's fp32 -> bf16 cast): gfx950's v_cvt_pk_bf16_f32, which
// rounds to nearest even and keeps NaN a NaN.
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Two values rounded to bf16 by one v_cvt_pk_bf16_f32: a in the low half (the lower address
// in memory), b in the high half; bf_lo / bf_hi give them back as floats.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Storage-type traits: T is float (fp32 modules) or uint16_t holding bf16 bits.
template <typename T> struct St;
template <> struct St<float> {
  static __device__ __forceinline__ float ld(const float* p) { return *p; }
  static __device__ __forceinline__ float to_f(float v) { return v; }
  static __device__ __forceinline__ float from_f(float v) { return v; }
  static __device__ __forceinline__ float rnd(float v) { return v; }   // rounding to storage precision
  static constexpr bool is_bf16 = false;
};
template <> struct St<uint16_t> {
  static __device__ __forceinline__ float ld(const uint16_t* p) { return bf2f(*p); }
  static __device__ __forceinline__ float to_f(uint16_t v) { return bf2f(v); }
  static __device__ __forceinline__ uint16_t from_f(float v) { return f2bf(v); }
  static __device__ __forceinline__ float rnd(float v) { return round_bf(v); }
  static constexpr bool is_bf16 = true;
};

// 8 consecutive storage elements: one 16-byte (bf16) or two 16-byte (fp32) moves
template <typename T> struct Vec8;
template <> struct Vec8<uint16_t> {
  u16x8 x;
  __device__ __forceinline__ void load(const uint16_t* p) { x = *reinterpret_cast<const u16x8*>(p); }
  __device__ __forceinline__ void store(uint16_t* p) const { *reinterpret_cast<u16x8*>(p) = x; }
  __device__ __forceinline__ float get(int i) const { return bf2f(x[i]); }
  __device__ __forceinline__ void set(int i, float v) { x[i] = f2bf(v); }
};
template <> struct Vec8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ __forceinline__ void store(float* p) const {
    *reinterpret_cast<float4*>(p) = a;
    *reinterpret_cast<float4*>(p + 4) = b;
  }
  __device__ __forceinline__ float get(int i) const {
    const float4& q = i < 4 ? a : b;
    const int k = i & 3;
    return k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w;
  }
  __device__ __forceinline__ void set(int i, float v) {
    float4& q = i < 4 ? a : b;
    const int k = i & 3;
    if (k == 0) q.x = v; else if (k == 1) q.y = v; else if (k == 2) q.z = v; else q.w = v;
  }
};

// IEEE single ops that the compiler must not contract into FMAs (the
// reference evaluates these as separate tensor ops).  HIP's __fmul_rn / __fadd_rn
// are plain operators, which hipcc (fp-contract=fast) fuses with a neighbouring
// add wherever inlining puts one; the instructions emitted here carry no
// contraction flag, so every call site rounds alike.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}
__device__ __forceinline__ float div_rn(float a, float b) { return __fdiv_rn(a, b); }

// A head's RMS statistic, partial over one piece pair: the 8 elements of a piece of the head's
// first half (u) and the 8 of its RoPE partner piece in the second half (w), in element order.
// The head preparation and the attention's in-kernel query preparation reduce these partials
// over the head's HD/16 piece pairs in one tree (pairs p and p ^ HD/32 first, ..., p and p ^ 1
// last), so both reach the same value.
__device__ __forceinline__ float sumsq_pair8(const float* u, const float* w) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s = fmaf(u[e], u[e], s);
    s = fmaf(w[e], w[e], s);
  }
  return s;
}

// ---------------------------------------------------------------- MFMA

__device__ __forceinline__ int d_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// D += A * B for one K=16 step with bf16 operands given as raw bf16 bits.
__device__ __forceinline__ void mma_bf16(f32x16& acc, const u16x8& a, const u16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 acc, 0, 0, 0);
}

// 16x16 tiles (K = 32 per step): lane l holds A row l % 16, B column l % 16 and the K group
// l / 16 (8 elements); D column l % 16, rows 4 * (l / 16) + i, i = 0..3.
__device__ __forceinline__ void mma16_bf16(f32x4& acc, const u16x8& a, const u16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 acc, 0, 0, 0);
}

// D += A * B for one K=2 step with fp32 operands.
__device__ __forceinline__ void mma_f32(f32x16& acc, float a, float b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
}

// Split fp32 values into bf16 hi + bf16 lo (hi + lo carries ~16 mantissa bits).
__device__ __forceinline__ void split8(const float* v, u16x8& hi, u16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint16_t h = f2bf(v[i]);
    hi[i] = h;
    lo[i] = f2bf(v[i] - bf2f(h));
  }
}

// ---------------------------------------------------------------- barriers

// Workgroup barrier for data exchanged through LDS only: waits for this wave's LDS
// operations, not for its outstanding global loads (which __syncthreads' workgroup fence
// would drain), so register prefetches stay in flight across it.
__device__ __forceinline__ void sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------- reductions

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }
// max / sum of v over the lane pair (l, l ^ 32), in both lanes: one v_permlane32_swap gives
// every lane the two values (in either order; both operations are commutative), with no
// cross-lane LDS exchange and its wait
__device__ __forceinline__ float pair_max32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ int xor32i(int v) { return __shfl_xor(v, 32, 64); }

template <typename F>
__device__ __forceinline__ float wave_reduce(float v, F op) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

// Ordering used by every "largest first" selection: NaN ranks above numbers
// (torch.topk / torch.max treat NaN as the largest value); among equal values
// the lower index wins.
__device__ __forceinline__ bool ranks_before_desc(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}
// "smallest first" (torch.topk(largest=False)): NaN ranks last.
__device__ __forceinline__ bool ranks_before_asc(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return nb && (!na || ia < ib);
  return a < b || (a == b && ia < ib);
}

// ---- transposed LDS operands (ds_read_b64_tr_b16) and accumulator operands

// Lane offsets of the transposed reads in a [32 rows][HD] tile whose 16-byte pieces p of row r
// sit at p ^ (r % (HD/8)): off[fb][s] for feature block fb (features 32 fb ..) and the read of
// rows 4 h + (lane % 16) / 4 + 8 s.  A K chunk kc adds 16 kc rows, which leaves r % (HD/8) as it
// is, so every read is one of these offsets plus a constant.
template <int HD>
struct TrLanes {
  int off[HD / 32][2];
  __device__ __forceinline__ explicit TrLanes(int lane) {
    constexpr int NP = HD / 8;
    const int jv = lane & 15, grp = lane >> 4, h = lane >> 5;
#pragma unroll
    for (int fb = 0; fb < HD / 32; ++fb)
#pragma unroll
      for (int sc = 0; sc < 2; ++sc) {
        const int r = 4 * h + (jv >> 2) + 8 * sc, f0 = 32 * fb + 16 * (grp & 1) + 4 * (jv & 3);
        off[fb][sc] = r * HD + 8 * ((f0 >> 3) ^ (r % NP)) + (f0 & 7);
      }
  }
};

// TrLanes::off[fb][sc] for a feature block known only at run time
template <int HD>
__device__ __forceinline__ int tr_off(int lane, int fb, int sc) {
  constexpr int NP = HD / 8;
  const int jv = lane & 15, grp = lane >> 4, h = lane >> 5;
  const int r = 4 * h + (jv >> 2) + 8 * sc, f0 = 32 * fb + 16 * (grp & 1) + 4 * (jv & 3);
  return r * HD + 8 * ((f0 >> 3) ^ (r % NP)) + (f0 & 7);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4 lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// the transposed operand of tile `t`: the result's row m is feature 32 fb + lane % 32; K chunk
// kc covers tile rows 16 kc + {4h..4h+3, 8+4h..8+4h+3} in the order of an accumulator's rows
template <int HD>
__device__ __forceinline__ u16x8 tr_operand(const uint16_t* t, const TrLanes<HD>& L, int fb, int kc) {
  const uint16_t* p = t + 16 * kc * HD;
  const s16x4 a = lds_tr16(p + L.off[fb][0]), b = lds_tr16(p + L.off[fb][1]);
  return __builtin_bit_cast(u16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// the accumulator's rows 8 kc .. 8 kc + 7 as a B operand split into bf16 hi and lo
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void acc_operand_split(const f32x16& v, int kc, u16x8& hi, u16x8& lo) {
  u32x4v h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x0 = v[8 * kc + 2 * e], x1 = v[8 * kc + 2 * e + 1];
    const uint32_t u = pack_bf2(x0, x1);
    h[e] = u;
    l[e] = pack_bf2(x0 - bf_lo(u), x1 - bf_hi(u));
  }
  hi = __builtin_bit_cast(u16x8, h);
  lo = __builtin_bit_cast(u16x8, l);
}

// ---------------------------------------------------------------- host

// Compute units of the current device (cached per device; callers that race store the same
// value), or minus the HIP error code.
static inline int cu_count() {
  static int cache[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  int n = dev >= 0 && dev < 64 ? cache[dev] : 0;
  if (n <= 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return -(int)e;
    if (dev >= 0 && dev < 64) cache[dev] = n;
  }
  return n;
}

}  // namespace b3

// LDS staging helpers shared by the bf16 attention kernels (forward and backward): tiles of
// 32 rows x HD bf16 brought into LDS by global->LDS loads (global_load_lds_dwordx4, 64 lanes x
// 16 bytes per instruction, no staging registers) in the "f2" layout, and LDS reads by inline
// assembly.
//
// f2 layout: a tile is stored as blocks of 8 rows x 8 sixteen-byte pieces (one global->LDS
// instruction each: lane L carries row L % 8, piece L / 8 of its block), piece-major inside a
// block, with 128 bytes of padding between blocks.  Every operand read is then a per-lane base
// plus a compile-time offset, the row reads (ds_read_b128) are conflict-free and the
// transposed reads (ds_read_b64_tr_b16) take the minimum two LDS cycles.
//
// The compiler cannot tell LDS reads from the destinations of outstanding global->LDS loads and
// would wait for every such load before an ordinary LDS read; the reads below are inline
// assembly, and their users wait for them explicitly (lds_wait*).
#pragma once
#include "bolt3_common.h"

namespace b3 {

constexpr int F2_ROWS = 32;             // rows of a staged tile
constexpr int F2_BLK = 1024 + 128;      // bytes of one 8-row x 8-piece block and its padding

// Byte offset of 16-byte piece p (elements 8p .. 8p+7) of row r in a staged K or V tile:
// block (p / 8, r / 8) at F2_BLK * ((p / 8) * (F2_ROWS / 8) + r / 8), and inside it the piece at
// 16 * ((r % 8) + 8 * (p % 8)).
__host__ __device__ constexpr int f2_off(int r, int p) {
  return F2_BLK * ((p >> 3) * (F2_ROWS / 8) + (r >> 3)) + 16 * ((r & 7) + 8 * (p & 7));
}

__device__ __forceinline__ void lds_dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (((N >> 4) & 3) << 14) | (7 << 4) | (15 << 8));
}
// ds_read_b64_tr_b16 as inline assembly, at a compile-time byte offset from the address (the
// instruction's offset field): the compiler cannot tell these reads from the LDS-DMA
// destinations and would otherwise wait for every outstanding tile load before them.  The
// caller waits for LDS (lds_wait8) before using the results.
template <int OFF>
__device__ __forceinline__ u16x4 lds_read_tr_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  u16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
// The V^T operand reads of rows 16 H2 .. 16 H2 + 15 of a staged V tile (f2_off layout) for the
// NDB feature blocks: tv[2 db] holds rows 16 H2 + r1, tv[2 db + 1] rows 16 H2 + 8 + r1, where the
// lane's row r1 and piece are in its base address.
template <int NDB, int H2>
__device__ __forceinline__ void f2_vreads(u16x4 (&tv)[8], uint32_t base) {
  tv[0] = lds_read_tr_at<f2_off(16 * H2, 0)>(base);
  tv[1] = lds_read_tr_at<f2_off(16 * H2 + 8, 0)>(base);
  tv[2] = lds_read_tr_at<f2_off(16 * H2, 4)>(base);
  tv[3] = lds_read_tr_at<f2_off(16 * H2 + 8, 4)>(base);
  if constexpr (NDB > 2) {
    tv[4] = lds_read_tr_at<f2_off(16 * H2, 8)>(base);
    tv[5] = lds_read_tr_at<f2_off(16 * H2 + 8, 8)>(base);
    tv[6] = lds_read_tr_at<f2_off(16 * H2, 12)>(base);
    tv[7] = lds_read_tr_at<f2_off(16 * H2 + 8, 12)>(base);
  }
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)((__attribute__((address_space(3))) const unsigned char*)p);
}
// The slot bias row goes through LDS by inline assembly as well (the compiler cannot separate
// it from the LDS-DMA destinations either).
__device__ __forceinline__ void lds_write_f32(float* p, float v) {
  const uint32_t addr = (uint32_t)(size_t)((__attribute__((address_space(3))) const float*)p);
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ float4 lds_read_f4(const float* p) {
  float4 r;
  const uint32_t addr = (uint32_t)(size_t)((__attribute__((address_space(3))) const float*)p);
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
typedef float fx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ fx4 lds_read_f4_nowait(const float* p) {
  fx4 r;
  const uint32_t addr = (uint32_t)(size_t)((__attribute__((address_space(3))) const float*)p);
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
// lgkmcnt(0), tied to four 16-byte LDS read results
__device__ __forceinline__ void lds_wait4(fx4& r0, fx4& r1, fx4& r2, fx4& r3) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3));
}
// lgkmcnt(0), tied to the transposed-read results so that their users follow it
__device__ __forceinline__ void lds_wait8(u16x4* r) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]));
}

// 4 bytes per lane (64 lanes: 256 contiguous bytes of LDS)
__device__ __forceinline__ void lds_dma4(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}
// wait_vm for a count known only at run time (0 .. 31)
__device__ __forceinline__ void wait_vm_rt(int n) {
  switch (n) {
#define B3_WAIT_CASE(k) case k: wait_vm<k>(); break;
    B3_WAIT_CASE(0) B3_WAIT_CASE(1) B3_WAIT_CASE(2) B3_WAIT_CASE(3) B3_WAIT_CASE(4) B3_WAIT_CASE(5)
    B3_WAIT_CASE(6) B3_WAIT_CASE(7) B3_WAIT_CASE(8) B3_WAIT_CASE(9) B3_WAIT_CASE(10) B3_WAIT_CASE(11)
    B3_WAIT_CASE(12) B3_WAIT_CASE(13) B3_WAIT_CASE(14) B3_WAIT_CASE(15) B3_WAIT_CASE(16) B3_WAIT_CASE(17)
    B3_WAIT_CASE(18) B3_WAIT_CASE(19) B3_WAIT_CASE(20) B3_WAIT_CASE(21) B3_WAIT_CASE(22) B3_WAIT_CASE(23)
    B3_WAIT_CASE(24) B3_WAIT_CASE(25) B3_WAIT_CASE(26) B3_WAIT_CASE(27) B3_WAIT_CASE(28) B3_WAIT_CASE(29)
    B3_WAIT_CASE(30)
#undef B3_WAIT_CASE
    default: wait_vm<31>(); break;
  }
}
// ds_read_b128 at a compile-time byte offset from the address (see above: the caller waits)
template <int OFF>
__device__ __forceinline__ u16x8 lds_read_b128_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  u16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
template <int OFF>
__device__ __forceinline__ fx4 lds_read_f4_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  fx4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}
// ds_write_b128 (see above: the writer waits before the data is used)
__device__ __forceinline__ void lds_write_f4(uint32_t addr, fx4 v) {
  asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
// lgkmcnt(0), tied to two 16-byte LDS read results
__device__ __forceinline__ void lds_wait2(u16x8& r0, u16x8& r1) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r0), "+v"(r1));
}

}  // namespace b3

// Device sine/cosine for RoPE angles.
//
// Argument reduction by k = rint(x * 2/pi) with pi/2 split into three fp32
// parts and fused multiply-adds (Cody & Waite, "Software Manual for the
// Elementary Functions", 1980); the reduced argument |r| <= ~pi/4 feeds the
// Taylor series of sin (to r^9) and cos (to r^10), whose truncation error on
// that interval is below 2e-10.  Valid for |x| < 2^20 (RoPE angles here are
// position * inverse frequency <= 65536 * 1); max error about 2 ulp.  Host and device
// evaluate the same IEEE operations (fmaf, rintf), so a host build reproduces the device
// values bit for bit (tests/test_rope_math.py checks the whole range that way).
#pragma once
#include <hip/hip_runtime.h>

namespace b3 {

__host__ __device__ __forceinline__ void sincos_rope(float x, float* s_out, float* c_out) {
  const float k = rintf(x * 0.636619772367581343f);
  // pi/2 = P1 + P2 + P3 (each the fp32 rounding of what remains)
  const float P1 = 1.57079637050628662109375f;
  const float P2 = -4.37113900018624283e-08f;
  const float P3 = -1.71512451532829103e-15f;
  float r = fmaf(-k, P1, x);
  r = fmaf(-k, P2, r);
  r = fmaf(-k, P3, r);
  const float r2 = r * r;
  float sp = fmaf(r2, 2.7557319223985893e-06f, -1.9841269841269841e-04f);
  sp = fmaf(r2, sp, 8.3333333333333332e-03f);
  sp = fmaf(r2, sp, -1.6666666666666666e-01f);
  const float sn = fmaf(r * r2, sp, r);
  float cp = fmaf(r2, -2.7557319223985888e-07f, 2.4801587301587302e-05f);
  cp = fmaf(r2, cp, -1.3888888888888889e-03f);
  cp = fmaf(r2, cp, 4.1666666666666664e-02f);
  cp = fmaf(r2, cp, -0.5f);
  const float cs = fmaf(r2, cp, 1.0f);
  const int q = ((int)k) & 3;
  const float s0 = (q & 1) ? cs : sn;
  const float c0 = (q & 1) ? sn : cs;
  *s_out = (q & 2) ? -s0 : s0;
  *c_out = ((q + 1) & 2) ? -c0 : c0;
}

}  // namespace b3

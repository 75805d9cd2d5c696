// sin and cos of rotation angles for the angle-fused scans.
//
// Cody-Waite reduction by the nearest multiple q of pi/2 (pi/2 as a float head
// and tail), near-minimax polynomials on [-pi/4, pi/4] -- sin to r^7, cos to r^8
// -- and the quadrant applied as a rotation by q pi/2 read from a 4-entry LDS
// table: (s, c) = (S cr + C sr, C cr - S sr) with (C, S) = (cos, sin)(q pi/2),
// every entry 0 or +-1, so the combination is exact and costs four VALU
// instructions instead of the selects and sign flips of a branch-free quadrant
// switch.
//
// Polynomial coefficients: Lawson-weighted least squares of the relative error
// over [0, pi/4] (sin: 3.8e-9, cos: 1.2e-10 before rounding to float), then the
// r^5 coefficient of sin moved up 15 float ulps, which leaves the maximum error
// unchanged and brings the mean of s^2 + c^2 - 1 over uniformly distributed
// angles from -9.5e-10 to below 1e-10 (a Taylor pair one degree higher gives
// -3.5e-10): products of tens of thousands of rotations keep the state's norm.
// Accuracy against float64 sin/cos: at most 1.5 ulp for |x| <= 4, 7.2e-8
// absolute for |x| up to a few thousand (float emulation of this exact
// sequence of fmaf operations on 2e7 random angles per range).
#pragma once

#include <hip/hip_runtime.h>

namespace mg {
namespace {

// Entries 0..3: cos(q pi/2); entries 4..7: sin(q pi/2), q = 0..3.
__shared__ float mg_quadrant[8];

}  // namespace

// Fills the quadrant table.  Every thread of the workgroup calls it before its
// first mg_sincos (it ends in a workgroup barrier).
__device__ __forceinline__ void mg_sincos_setup() {
  if (threadIdx.x < 8) {
    const int q = threadIdx.x & 3;
    const float cq = q == 0 ? 1.f : (q == 2 ? -1.f : 0.f);
    const float sq = q == 1 ? 1.f : (q == 3 ? -1.f : 0.f);
    mg_quadrant[threadIdx.x] = threadIdx.x < 4 ? cq : sq;
  }
  __syncthreads();
}

__device__ __forceinline__ void mg_sincos(float x, float& s, float& c) {
  const float q = rintf(x * 0.636619772367581343f);  // x / (pi/2)
  float r = fmaf(-q, 1.57079637050628662f, x);
  r = fmaf(-q, -4.37113900018624283e-8f, r);
  const int i = (int)q & 3;
  const float C = mg_quadrant[i], S = mg_quadrant[4 + i];
  const float z = r * r;
  float ps = fmaf(z, -1.951497397e-04f, 8.332172409e-03f);
  ps = fmaf(ps, z, -1.666665524e-01f);
  const float sr = fmaf(ps * z, r, r);
  float pc = fmaf(z, 2.443279664e-05f, -1.388731296e-03f);
  pc = fmaf(pc, z, 4.166664556e-02f);
  pc = fmaf(pc, z, -0.5f);
  const float cr = fmaf(pc, z, 1.0f);
  s = fmaf(S, cr, C * sr);
  c = fmaf(C, cr, -S * sr);
}

}  // namespace mg

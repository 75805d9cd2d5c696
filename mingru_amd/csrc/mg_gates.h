// Gate arithmetic shared by the fused gate scans and the decode step kernels
// (gfx950): the coefficients (a, b) of h = a h_prev + b formed from a mixer's
// pre-activations.
//   GATE_SIGNED (/_COUPLED): SignedMinGRU (reference src/mingru/min_gru.py:
//     1788-1857): a = tanh(s) [* (1 - sigmoid(z))], b = sigmoid(z) * hpre.
//   GATE_MINGRU: MinGRU (reference :1366-1397): a = sigmoid(-k) = 1 - z,
//     b = sigmoid(k) g(hpre), g(x) = x + 1/2 for x >= 0, sigmoid(x) otherwise.
#pragma once

#include <hip/hip_runtime.h>

enum : int { GATE_SIGNED = 0, GATE_SIGNED_COUPLED = 1, GATE_MINGRU = 2 };

// sigmoid(x) = 1 / (1 + e^-x) on the hardware exp2 and reciprocal (each about
// 1 ulp; e^-x overflowing to inf gives 0, underflowing to 0 gives 1), and
// tanh(s) = 2 sigmoid(2 s) - 1 (absolute error a few 1e-8 near 0).
__device__ __forceinline__ float mg_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504088896341f * x));
}
__device__ __forceinline__ float mg_tanh(float x) { return fmaf(2.f, mg_sigmoid(2.f * x), -1.f); }
__device__ __forceinline__ float mg_g(float x) { return x >= 0.f ? x + 0.5f : mg_sigmoid(x); }

template <int G>
__device__ __forceinline__ void gate_coeffs(float p0, float p1, float p2, float& a, float& b) {
  if constexpr (G == GATE_MINGRU) {
    a = mg_sigmoid(-p0);
    b = mg_sigmoid(p0) * mg_g(p1);
  } else {
    const float sg = mg_sigmoid(p1), th = mg_tanh(p0);
    a = G == GATE_SIGNED_COUPLED ? (1.f - sg) * th : th;
    b = sg * p2;
  }
}


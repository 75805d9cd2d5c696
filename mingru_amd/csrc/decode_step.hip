// Streaming decode: one recurrent step of a mixer per call (gfx950), the
// token-by-token path of serving.  No reference kernel: these replace the
// eager torch bodies of the mixers' step() (reference src/mingru/min_gru.py:
// 1399-1448 MinGRU, SignedMinGRU's step, 3611-3688 DeltaMinGRU), which launch a
// handful of small kernels per step.
//
//   gate_step_kernel: h = gamma * a * h_prev + b elementwise, (a, b) from the
//     mixer's pre-activations by the same gate arithmetic as the fused gate
//     scans (mg_gates.h); gamma is the optional decay factor per element.
//   delta_step_kernel: per head, H <- gamma H, then for each micro-step
//     H <- H + beta k (v - H^T k)^T, then y = H^T q.  One wave owns one head and
//     lane j owns column j of H (d_k values in registers), so the micro-steps
//     need no cross-lane traffic: k and q are broadcast from the lane holding
//     each element with v_readlane.  H is read once and written once.
#include "mg_common.h"
#include "mg_gates.h"

namespace {

constexpr int STEP_NT = 256;

template <int G>
__global__ __launch_bounds__(STEP_NT) void gate_step_kernel(
    const float* __restrict__ p0, const float* __restrict__ p1, const float* __restrict__ p2,
    const float* __restrict__ gamma, const float* __restrict__ hp, float* __restrict__ h,
    int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * STEP_NT + threadIdx.x;
  if (i >= n) return;
  float a, b;
  gate_coeffs<G>(p0[i], p1[i], G == GATE_MINGRU ? 0.f : p2[i], a, b);
  if (gamma) a *= gamma[i];
  h[i] = fmaf(a, hp[i], b);
}

__device__ __forceinline__ float lane_bcast(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

constexpr int STEP_DK = 64;  // rows of H held per lane

__global__ __launch_bounds__(STEP_NT) void delta_step_kernel(
    const float* __restrict__ Hin, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ beta, const float* __restrict__ lg,
    float* __restrict__ Hout, float* __restrict__ y, int64_t BH, int nh, int dk, int dv) {
  const int64_t head = (int64_t)blockIdx.x * (STEP_NT / 64) + (threadIdx.x >> 6);
  if (head >= BH) return;  // whole waves: the head index is uniform within a wave
  const int j = threadIdx.x & 63;
  const bool col = j < dv;
  const float* Hh = Hin + head * dk * dv;
  float hc[STEP_DK];
#pragma unroll
  for (int i = 0; i < STEP_DK; ++i) hc[i] = (col && i < dk) ? Hh[i * dv + j] : 0.f;
  if (lg) {
    const float gm = expf(lg[head]);
#pragma unroll
    for (int i = 0; i < STEP_DK; ++i) hc[i] *= gm;
  }
  for (int m = 0; m < nh; ++m) {
    const int64_t row = head * nh + m;
    const float kv = j < dk ? k[row * dk + j] : 0.f;  // lane i holds k_i
    float kh = 0.f;
#pragma unroll
    for (int i = 0; i < STEP_DK; ++i) kh = fmaf(lane_bcast(kv, i), hc[i], kh);
    const float u = (col ? v[row * dv + j] : 0.f) - kh;
    const float bu = beta[row] * u;
#pragma unroll
    for (int i = 0; i < STEP_DK; ++i) hc[i] = fmaf(lane_bcast(kv, i), bu, hc[i]);
  }
  const float qv = j < dk ? q[head * dk + j] : 0.f;
  float yy = 0.f;
#pragma unroll
  for (int i = 0; i < STEP_DK; ++i) yy = fmaf(lane_bcast(qv, i), hc[i], yy);
  if (col) {
    y[head * dv + j] = yy;
    float* Ho = Hout + head * dk * dv;
#pragma unroll
    for (int i = 0; i < STEP_DK; ++i)
      if (i < dk) Ho[i * dv + j] = hc[i];
  }
}

}  // namespace

extern "C" {

int mg_gate_step(int kind, const float* p0, const float* p1, const float* p2, const float* gamma,
                 const float* h_prev, float* h, int64_t n, hipStream_t stream) {
  if (!p0 || !p1 || !h_prev || !h || n < 0 || kind < 0 || kind > 2) return MG_ERR_ARG;
  if (kind != GATE_MINGRU && !p2) return MG_ERR_ARG;
  if (n == 0) return MG_OK;
  const unsigned grid = (unsigned)((n + STEP_NT - 1) / STEP_NT);
  if (kind == GATE_SIGNED)
    hipLaunchKernelGGL(gate_step_kernel<GATE_SIGNED>, dim3(grid), dim3(STEP_NT), 0, stream, p0, p1,
                       p2, gamma, h_prev, h, n);
  else if (kind == GATE_SIGNED_COUPLED)
    hipLaunchKernelGGL(gate_step_kernel<GATE_SIGNED_COUPLED>, dim3(grid), dim3(STEP_NT), 0, stream,
                       p0, p1, p2, gamma, h_prev, h, n);
  else
    hipLaunchKernelGGL(gate_step_kernel<GATE_MINGRU>, dim3(grid), dim3(STEP_NT), 0, stream, p0, p1,
                       p2, gamma, h_prev, h, n);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

int mg_delta_step(const float* H, const float* q, const float* k, const float* v,
                  const float* beta, const float* log_gamma, float* H_out, float* y, int64_t BH,
                  int nh, int dk, int dv, hipStream_t stream) {
  if (!H || !q || !k || !v || !beta || !H_out || !y) return MG_ERR_ARG;
  if (BH <= 0 || nh <= 0 || dk <= 0 || dk > STEP_DK || dv <= 0 || dv > 64) return MG_ERR_ARG;
  const int64_t grid = (BH + STEP_NT / 64 - 1) / (STEP_NT / 64);
  if (grid > 0x7fffffff) return MG_ERR_ARG;
  hipLaunchKernelGGL(delta_step_kernel, dim3((unsigned)grid), dim3(STEP_NT), 0, stream, H, q, k, v,
                     beta, log_gamma, H_out, y, BH, nh, dk, dv);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

}  // extern "C"

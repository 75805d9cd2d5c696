// Angle-fused rotation scan driven by run-time plane tables, fwd + bwd.
//
// Same recurrence and table semantics as the reference kernel
// (src/mingru/triton_scans.py:1039-1291, tables described at :1063-1070):
//   v = S_t h_{t-1}                (coordinate 1 scaled by d_t when has_scale)
//   for each round r:  v'[p] = c_p v[p] + sgn[r][p] s_p v[perm[r][p]]
//                      with (c_p, s_p) = (cos, sin) of theta[r][p2p[r][p]]
//   h_t = gamma_t v + b_t          (gamma only when has_decay)
// A position whose partner is itself is left untouched by its round.  The host
// accepts only tables that describe disjoint plane rotations (perm an
// involution, partners sharing one angle, opposite unit signs), so every round
// is orthogonal and its inverse is its transpose.
//
// This is the general path: k in {2, 4, 8, 16}, any such tables, any number of
// rounds.  The compiled-schedule kernels in scan_angle.hip cover the brick-wall
// and lexicographic schedules of k <= 8 with a chunk-parallel scan.
//
// Layout of the work: one lane per (batch row, block, coordinate p), k
// consecutive lanes per block, so h, b and the gradients move as contiguous
// rows; a round reads the partner coordinate with one ds_bpermute.  Each lane
// walks its block's sequence in order (the reference kernel's decomposition),
// prefetching the next token's inputs.  The backward walks in reverse: it
// recomputes the token's rounds from h_{t-1} (read from the forward output),
// then sweeps them backwards, recovering each round's input by the transposed
// rotation and accumulating dtheta per angle in LDS.
#include "mg_common.h"

#include <algorithm>

namespace {

constexpr int AT_THREADS = 256;
constexpr int AT_MAX_HALF = 64;  // angles per round held in LDS per block

// Cody-Waite sin/cos (same method as the compiled-schedule kernels): reduction
// by the nearest multiple of pi/2 with pi/2 in two parts, Taylor polynomials on
// [-pi/4, pi/4], quadrant select.
__device__ __forceinline__ void at_sincos(float x, float& s, float& c) {
  const float q = rintf(x * 0.636619772367581343f);
  float r = fmaf(-q, 1.57079637050628662f, x);
  r = fmaf(-q, -4.37113900018624283e-8f, r);
  const float r2 = r * r;
  float ps = fmaf(r2, 2.75573192239858907e-6f, -1.98412698412698413e-4f);
  ps = fmaf(ps, r2, 8.33333333333333333e-3f);
  ps = fmaf(ps, r2, -1.66666666666666667e-1f);
  const float sr = fmaf(ps * r2, r, r);
  float pc = fmaf(r2, -2.75573192239858907e-7f, 2.48015873015873016e-5f);
  pc = fmaf(pc, r2, -1.38888888888888889e-3f);
  pc = fmaf(pc, r2, 4.16666666666666667e-2f);
  pc = fmaf(pc, r2, -0.5f);
  const float cr = fmaf(pc, r2, 1.0f);
  const int quad = (int)q & 3;
  const float ss = (quad & 1) ? cr : sr;
  const float cc = (quad & 1) ? sr : cr;
  s = (quad & 2) ? -ss : ss;
  c = ((quad + 1) & 2) ? -cc : cc;
}

// Value of `v` held by lane `src` of this wave.
__device__ __forceinline__ float at_shfl(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

struct AtArgs {
  const float* theta;  // (B, T, n, R, half)
  const float* scale;  // (B, T, n)
  const float* gamma;  // (B, T, n)
  const float* b;      // (B, T, n, k)
  const float* h0;     // (B, n, k)
  const int* perm;     // (R, k)
  const float* sgn;    // (R, k)
  const int* p2p;      // (R, k)
  const float* h;      // forward output (backward input)
  const float* gh;     // upstream grad (backward)
  float* out;          // forward: h; backward: db
  float* dtheta;
  float* dscale;
  float* dgamma;
  float* dh0;
  int64_t B, T, n;
  int k, R, half;
  int has_scale, has_decay;
};

// One lane's coordinate within the problem.
struct AtLane {
  int64_t blk;   // b * n + block
  int64_t bb;    // batch row
  int p;         // coordinate within the block
  int lane, base;  // lane in the wave, lane of coordinate 0 of this block
  bool ok;
};

__device__ __forceinline__ AtLane at_lane(const AtArgs& a) {
  AtLane L;
  const int64_t gid = (int64_t)blockIdx.x * AT_THREADS + threadIdx.x;
  L.lane = threadIdx.x & (MG_WAVE - 1);
  L.p = (int)(gid % a.k);
  L.base = L.lane - L.p;
  L.blk = gid / a.k;
  L.ok = L.blk < a.B * a.n;
  L.bb = L.ok ? L.blk / a.n : 0;
  if (!L.ok) L.blk = 0;
  return L;
}

// Round r's table entries for coordinate p (indices clamped into range).
struct AtRound {
  int partner;  // lane of the partner coordinate
  int ang;      // angle index within the round
  float sg;     // sign of this coordinate
  bool act;     // false when the partner is the coordinate itself
};

__device__ __forceinline__ AtRound at_round(const AtArgs& a, const AtLane& L, int r) {
  AtRound q;
  const int pp = min(max(a.perm[r * a.k + L.p], 0), a.k - 1);
  q.act = pp != L.p;
  q.partner = L.base + pp;
  q.ang = min(max(a.p2p[r * a.k + L.p], 0), a.half - 1);
  q.sg = a.sgn[r * a.k + L.p];
  return q;
}

__device__ __forceinline__ int64_t at_tok(const AtArgs& a, const AtLane& L, int64_t t) {
  return (L.bb * a.T + t) * a.n + (L.blk - L.bb * a.n);
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(AT_THREADS) void angle_tables_fwd(AtArgs a) {
  const AtLane L = at_lane(a);
  float v = L.ok ? a.h0[L.blk * a.k + L.p] : 0.f;
  for (int64_t t = 0; t < a.T; ++t) {
    const int64_t tk = at_tok(a, L, t);
    if (a.has_scale && L.p == 1) v *= L.ok ? a.scale[tk] : 1.f;
    for (int r = 0; r < a.R; ++r) {
      const AtRound q = at_round(a, L, r);
      float s = 0.f, c = 1.f;
      if (L.ok) at_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
      const float vp = at_shfl(v, q.partner);
      if (q.act) v = fmaf(c, v, q.sg * s * vp);
    }
    if (L.ok) {
      if (a.has_decay) v *= a.gamma[tk];
      v += a.b[tk * a.k + L.p];
      a.out[tk * a.k + L.p] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(AT_THREADS) void angle_tables_bwd(AtArgs a) {
  // dtheta of one round for each block of the workgroup: [block in workgroup][angle]
  __shared__ float s_dth[(AT_THREADS / 2) * AT_MAX_HALF];
  const AtLane L = at_lane(a);
  float* slot = s_dth + (threadIdx.x / a.k) * a.half;
  float y = 0.f;  // adjoint on h_t arriving from t + 1
  for (int64_t t = a.T - 1; t >= 0; --t) {
    const int64_t tk = at_tok(a, L, t);
    const float x = y + (L.ok ? a.gh[tk * a.k + L.p] : 0.f);  // dL/dh_t in total
    float hp = 0.f, d = 1.f, gm = 1.f;
    if (L.ok) {
      hp = t > 0 ? a.h[(tk - a.n) * a.k + L.p] : a.h0[L.blk * a.k + L.p];
      if (a.has_scale) d = a.scale[tk];
      if (a.has_decay) gm = a.gamma[tk];
      a.out[tk * a.k + L.p] = x;  // db
    }
    // Forward through the token's rounds: u_R.
    float u = (a.has_scale && L.p == 1) ? hp * d : hp;
    for (int r = 0; r < a.R; ++r) {
      const AtRound q = at_round(a, L, r);
      float s = 0.f, c = 1.f;
      if (L.ok) at_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
      const float up = at_shfl(u, q.partner);
      if (q.act) u = fmaf(c, u, q.sg * s * up);
    }
    // dgamma = <x, u_R> over the block's k lanes (aligned groups of k lanes).
    if (a.has_decay) {
      float dg = x * u;
      for (int off = a.k >> 1; off > 0; off >>= 1) dg += at_shfl(dg, L.lane ^ off);
      if (L.ok && L.p == 0) a.dgamma[tk] = dg;
    }
    float adj = gm * x;  // adjoint on u_R
    for (int r = a.R - 1; r >= 0; --r) {
      const AtRound q = at_round(a, L, r);
      float s = 0.f, c = 1.f;
      if (L.ok) at_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
      // u holds u_r (after the rotation); recover u_{r-1} by the transposed rotation.
      const float up = at_shfl(u, q.partner);
      const float u_prev = q.act ? fmaf(c, u, -q.sg * s * up) : u;
      const float u_prev_p = at_shfl(u_prev, q.partner);
      const float ap = at_shfl(adj, q.partner);
      // d u_r[p] / d theta = -s u[p] + sgn c u[partner] (u = u_{r-1})
      const float e = q.act ? adj * fmaf(-s, u_prev, q.sg * c * u_prev_p) : 0.f;
      // adjoint on u_{r-1}: the transposed rotation
      if (q.act) adj = fmaf(c, adj, -q.sg * s * ap);
      u = u_prev;
      // dtheta[r][a] = sum of e over the coordinates that use angle a
      for (int j = L.p; j < a.half; j += a.k) slot[j] = 0.f;
      __syncthreads();
      if (q.act) atomicAdd(&slot[q.ang], e);
      __syncthreads();
      if (L.ok)
        for (int j = L.p; j < a.half; j += a.k) a.dtheta[(tk * a.R + r) * a.half + j] = slot[j];
      __syncthreads();
    }
    // u = u_0 = S h_{t-1}; adj on u_0 -> dscale and the adjoint on h_{t-1}.
    if (a.has_scale && L.p == 1) {
      if (L.ok) a.dscale[tk] = adj * hp;
      adj *= d;
    }
    y = adj;
  }
  if (L.ok) a.dh0[L.blk * a.k + L.p] = y;
}

}  // namespace

extern "C" {

int mg_angle_scan_tables_fwd(const float* theta, const float* scale, const float* gamma,
                             const float* b, const float* h0, const int* perm, const float* sgn,
                             const int* p2p, float* h, int64_t B, int64_t T, int64_t n, int k,
                             int R, int half, int flags, hipStream_t stream) {
  if (!theta || !b || !h0 || !perm || !sgn || !p2p || !h) return MG_ERR_ARG;
  if (B <= 0 || T <= 0 || n <= 0 || R <= 0 || half <= 0) return MG_ERR_ARG;
  if (!(k == 2 || k == 4 || k == 8 || k == 16) || half > AT_MAX_HALF) return MG_ERR_ARG;
  if (((flags & 1) && !scale) || ((flags & 2) && !gamma) || (flags & ~3)) return MG_ERR_ARG;
  const int64_t lanes = B * n * k;
  if (lanes >= (1ll << 31)) return MG_ERR_ARG;
  AtArgs a{theta, scale, gamma, b, h0, perm, sgn, p2p, nullptr, nullptr, h, nullptr, nullptr,
           nullptr, nullptr, B, T, n, k, R, half, flags & 1, (flags >> 1) & 1};
  hipLaunchKernelGGL(angle_tables_fwd, dim3((unsigned)((lanes + AT_THREADS - 1) / AT_THREADS)),
                     dim3(AT_THREADS), 0, stream, a);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

int mg_angle_scan_tables_bwd(const float* theta, const float* scale, const float* gamma,
                             const float* h0, const float* h, const float* gh, const int* perm,
                             const float* sgn, const int* p2p, float* dtheta, float* dscale,
                             float* dgamma, float* db, float* dh0, int64_t B, int64_t T,
                             int64_t n, int k, int R, int half, int flags, hipStream_t stream) {
  if (!theta || !h0 || !h || !gh || !perm || !sgn || !p2p || !dtheta || !db || !dh0)
    return MG_ERR_ARG;
  if (B <= 0 || T <= 0 || n <= 0 || R <= 0 || half <= 0) return MG_ERR_ARG;
  if (!(k == 2 || k == 4 || k == 8 || k == 16) || half > AT_MAX_HALF) return MG_ERR_ARG;
  if (((flags & 1) && (!scale || !dscale)) || ((flags & 2) && (!gamma || !dgamma)) ||
      (flags & ~3))
    return MG_ERR_ARG;
  const int64_t lanes = B * n * k;
  if (lanes >= (1ll << 31)) return MG_ERR_ARG;
  AtArgs a{theta, scale, gamma, nullptr, h0, perm, sgn, p2p, h, gh, db, dtheta, dscale, dgamma,
           dh0, B, T, n, k, R, half, flags & 1, (flags >> 1) & 1};
  hipLaunchKernelGGL(angle_tables_bwd, dim3((unsigned)((lanes + AT_THREADS - 1) / AT_THREADS)),
                     dim3(AT_THREADS), 0, stream, a);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

}  // extern "C"

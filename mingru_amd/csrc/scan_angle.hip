// Angle-fused block-rotation scan (RotationMinGRU, GivensMinGRU), fwd + bwd.
//
// Per block of k state coordinates and token t (reference kernel semantics,
// src/mingru/triton_scans.py:1039-1291; rotation rule src/mingru/min_gru.py:
// 2583-2602):
//   v = S_t h_{t-1}            S_t scales coordinate 1 by d_t   (has_scale)
//   v = G_last ... G_first v   plane rotations from the token's angles
//   h_t = gamma_t v + b_t                                     (has_decay)
// A rotation of plane (i, j) by theta: v_i <- c v_i - s v_j, v_j <- s v_i + c v_j.
// Transition matrices are never written to memory: every token's rotations are
// rebuilt from its angles in registers.
//
// Plane schedules (compile-time, so every coordinate index is a register):
//   BRICK: `rounds` rounds; even rounds rotate planes (0,1),(2,3),..., odd
//          rounds (1,2),(3,4),...,(k-1,0); k/2 angles per round
//          (GivensMinGRU, and RotationMinGRU as k=2, one round).
//   LEX:   one plane per round over all pairs i<j in lexicographic order,
//          k(k-1)/2 angles per token (the 28-rotation SO(8) workload).
//
// Parallel scan over time: the chunk aggregate of the affine recurrence is
// the map h -> P h + L with P the k x k product of the chunk's transitions;
// each thread builds it for its sub-chunk by pushing the k columns of P and
// the column L through the rotations (k+1 rotated columns per token), then
// the shared look-back (mg_affm.h) chains the chunks.  The final pass
// re-applies the rotations to the state vector only.
//
// Backward: exact stored-state recompute.  h_{t-1} is read from the forward
// output (never reconstructed by dividing out gamma or the scale), the
// per-rotation states are recovered from the recomputed v_R by applying each
// rotation's transpose (orthogonal, so no error amplification), and the
// adjoint y_t = M_t^T (g_t + y_{t+1}) runs through the same chunked
// look-back in reverse time.
#include "mg_affm.h"

#include <algorithm>
#include <utility>

namespace {

using namespace mg;

enum : int { SCHED_BRICK = 0, SCHED_LEX = 1 };

// Chunk = AN_WAVES * AN_TSUB tokens per workgroup.  64-token chunks keep the
// look-back chain short (32 hops at T = 2048) while the per-thread aggregate
// work (k + 1 rotated columns per token) stays in registers; chosen by timing
// on MI355X at the 28-rotation SO(8) workload.
constexpr int AN_WAVES = 8;
constexpr int AN_TSUB = 8;

constexpr int lex_first(int K, int r) {
  int i = 0;
  while (r >= K - 1 - i) {
    r -= K - 1 - i;
    ++i;
  }
  return i;
}

constexpr int lex_second(int K, int r) {
  int i = 0;
  while (r >= K - 1 - i) {
    r -= K - 1 - i;
    ++i;
  }
  return i + 1 + r;
}

template <int K, int SCHED>
constexpr int angles_per_round() {
  return SCHED == SCHED_LEX ? 1 : K / 2;
}

template <typename F, std::size_t... Is>
__device__ __forceinline__ void static_for(F&& f, std::index_sequence<Is...>) {
  (f(std::integral_constant<int, (int)Is>{}), ...);
}

// sin and cos of x (radians), about 1 ulp for |x| up to a few thousand.
// Cody-Waite reduction by the nearest multiple q of pi/2 (pi/2 split into a
// float head and tail), Taylor polynomials on [-pi/4, pi/4] (sin to r^9,
// cos to r^10: the first omitted terms are below 2e-9), then the quadrant
// q mod 4 selects and negates.  The hardware sine (about 6 ulp) drifts a
// state vector measurably over thousands of rotations; this costs about
// twice as many VALU instructions and keeps the drift at fp32 rounding.
__device__ __forceinline__ void mg_sincos(float x, float& s, float& c) {
  const float q = rintf(x * 0.636619772367581343f);  // x / (pi/2)
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

// Rows I, J of an NC-column block: row_I <- c row_I - s row_J, row_J <- s row_I + c row_J.
template <int K, int NC, int I, int J>
__device__ __forceinline__ void rot_rows(float (&X)[K][NC], float c, float s) {
#pragma unroll
  for (int q = 0; q < NC; ++q) {
    const float xi = X[I][q], xj = X[J][q];
    X[I][q] = fmaf(c, xi, -s * xj);
    X[J][q] = fmaf(s, xi, c * xj);
  }
}

// Transposed rotation (adjoint / inverse): row_I <- c row_I + s row_J, row_J <- -s row_I + c row_J.
template <int K, int NC, int I, int J>
__device__ __forceinline__ void rot_rows_t(float (&X)[K][NC], float c, float s) {
#pragma unroll
  for (int q = 0; q < NC; ++q) {
    const float xi = X[I][q], xj = X[J][q];
    X[I][q] = fmaf(c, xi, s * xj);
    X[J][q] = fmaf(-s, xi, c * xj);
  }
}

// One round of the brick-wall schedule (planes given by the round parity).
template <int K, int NC, bool TRANSPOSE>
__device__ __forceinline__ void brick_round(float (&X)[K][NC], int r, const float (&cs)[K / 2],
                                            const float (&sn)[K / 2]) {
  if ((r & 1) == 0) {
    static_for(
        [&](auto m) {
          constexpr int I = 2 * decltype(m)::value, J = I + 1;
          if (TRANSPOSE) rot_rows_t<K, NC, I, J>(X, cs[decltype(m)::value], sn[decltype(m)::value]);
          else rot_rows<K, NC, I, J>(X, cs[decltype(m)::value], sn[decltype(m)::value]);
        },
        std::make_index_sequence<K / 2>{});
  } else {
    static_for(
        [&](auto m) {
          constexpr int I = 2 * decltype(m)::value + 1, J = (I + 1) % K;
          if (TRANSPOSE) rot_rows_t<K, NC, I, J>(X, cs[decltype(m)::value], sn[decltype(m)::value]);
          else rot_rows<K, NC, I, J>(X, cs[decltype(m)::value], sn[decltype(m)::value]);
        },
        std::make_index_sequence<K / 2>{});
  }
}

// X <- M_t X for an NC-column block (M_t = gamma R S).
template <int K, int SCHED, bool HS, bool HD, int NC>
__device__ __forceinline__ void apply_M(float (&X)[K][NC], const float* __restrict__ th,
                                        int rounds, float d, float gm) {
  if (HS) {
#pragma unroll
    for (int q = 0; q < NC; ++q) X[1][q] *= d;
  }
  if constexpr (SCHED == SCHED_LEX) {
    constexpr int R = K * (K - 1) / 2;
    float ang[R];
    ld<R>(ang, th);
    static_for(
        [&](auto rc) {
          constexpr int r = decltype(rc)::value;
          float s, c;
          mg_sincos(ang[r], s, c);
          rot_rows<K, NC, lex_first(K, r), lex_second(K, r)>(X, c, s);
        },
        std::make_index_sequence<R>{});
  } else {
    constexpr int H = K / 2;
    for (int r = 0; r < rounds; ++r) {
      float ang[H], cs[H], sn[H];
      ld<H>(ang, th + r * H);
#pragma unroll
      for (int m = 0; m < H; ++m) mg_sincos(ang[m], sn[m], cs[m]);
      brick_round<K, NC, false>(X, r, cs, sn);
    }
  }
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
}

// X <- M_t^T X.
template <int K, int SCHED, bool HS, bool HD, int NC>
__device__ __forceinline__ void apply_Mt(float (&X)[K][NC], const float* __restrict__ th,
                                         int rounds, float d, float gm) {
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
  if constexpr (SCHED == SCHED_LEX) {
    constexpr int R = K * (K - 1) / 2;
    float ang[R];
    ld<R>(ang, th);
    static_for(
        [&](auto rc) {
          constexpr int r = R - 1 - decltype(rc)::value;
          float s, c;
          mg_sincos(ang[r], s, c);
          rot_rows_t<K, NC, lex_first(K, r), lex_second(K, r)>(X, c, s);
        },
        std::make_index_sequence<R>{});
  } else {
    constexpr int H = K / 2;
    for (int r = rounds - 1; r >= 0; --r) {
      float ang[H], cs[H], sn[H];
      ld<H>(ang, th + r * H);
#pragma unroll
      for (int m = 0; m < H; ++m) mg_sincos(ang[m], sn[m], cs[m]);
      brick_round<K, NC, true>(X, r, cs, sn);
    }
  }
  if (HS) {
#pragma unroll
    for (int q = 0; q < NC; ++q) X[1][q] *= d;
  }
}

// Gradient of one rotation step.  On entry v holds v_r (after the rotation)
// and a the adjoint on v_r; on exit v holds v_{r-1}, a the adjoint on
// v_{r-1}, and the return value is dL/dtheta of this rotation.
template <int K, int I, int J>
__device__ __forceinline__ float rot_grad(float (&v)[K][1], float (&a)[K][1], float c, float s) {
  const float wi = v[I][0], wj = v[J][0];
  const float vi = fmaf(c, wi, s * wj);   // inverse rotation
  const float vj = fmaf(-s, wi, c * wj);
  v[I][0] = vi;
  v[J][0] = vj;
  const float ai = a[I][0], aj = a[J][0];
  const float g = ai * fmaf(-s, vi, -c * vj) + aj * fmaf(c, vi, -s * vj);
  a[I][0] = fmaf(c, ai, s * aj);
  a[J][0] = fmaf(-s, ai, c * aj);
  return g;
}

struct AnArgs {
  const float* theta;
  const float* scale;
  const float* gamma;
  const float* b;
  const float* h0;
  const float* h;   // forward output (backward only)
  const float* gh;  // upstream grad (backward only)
  float* out;       // forward: h; backward: db
  float* dtheta;
  float* dscale;
  float* dgamma;
  float* dh0;
  int rounds;
  int na;  // angles per token
};

template <int K, int SCHED, bool HS, bool HD>
__global__ __launch_bounds__(MG_WAVE* AN_WAVES) void angle_fwd_kernel(AnArgs a, AfGeom g,
                                                                      unsigned* header,
                                                                      mg_slot_t* agg_data,
                                                                      mg_slot_t* incl_data) {
  AfThread th = af_thread<false>(g, header);
  if (!th.valid) return;
  const int64_t t0 = (int64_t)th.c * (AN_WAVES * AN_TSUB) + th.w * AN_TSUB;
  const int64_t T = g.T, n = g.n;

  // Local aggregate: push [P | L] through the sub-chunk's transitions.
  float X[K][K + 1];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int q = 0; q <= K; ++q) X[i][q] = (i == q) ? 1.f : 0.f;
#pragma unroll
  for (int s = 0; s < AN_TSUB; ++s) {
    const int64_t t = t0 + s;
    if (th.ok && t < T) {
      const int64_t lane_tok = (th.bb * T + t) * n + th.plane;
      const float d = HS ? a.scale[lane_tok] : 1.f;
      const float gm = HD ? a.gamma[lane_tok] : 1.f;
      apply_M<K, SCHED, HS, HD, K + 1>(X, a.theta + lane_tok * a.na, a.rounds, d, gm);
      float bt[K];
      ld<K>(bt, a.b + lane_tok * K);
#pragma unroll
      for (int i = 0; i < K; ++i) X[i][K] += bt[i];
    }
  }
  AffM<K, 1> loc, seed, carry;
#pragma unroll
  for (int i = 0; i < K; ++i) {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      loc.P[i][j] = X[i][j];
      seed.P[i][j] = 0.f;
    }
    loc.L[i][0] = X[i][K];
    seed.L[i][0] = 0.f;
  }
  if (th.c == 0 && th.ok) {
    float hz[K];
    ld<K>(hz, a.h0 + (th.bb * n + th.plane) * K);
#pragma unroll
    for (int i = 0; i < K; ++i) seed.L[i][0] = hz[i];
  }
  af_carry<K, 1, AN_WAVES, false>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data, incl_data, carry);

  // Final pass: the state entering the sub-chunk is carry.L (the seed's P = 0
  // turns every prefix into a constant map).
  float v[K][1];
#pragma unroll
  for (int i = 0; i < K; ++i) v[i][0] = carry.L[i][0];
#pragma unroll
  for (int s = 0; s < AN_TSUB; ++s) {
    const int64_t t = t0 + s;
    if (th.ok && t < T) {
      const int64_t lane_tok = (th.bb * T + t) * n + th.plane;
      const float d = HS ? a.scale[lane_tok] : 1.f;
      const float gm = HD ? a.gamma[lane_tok] : 1.f;
      apply_M<K, SCHED, HS, HD, 1>(v, a.theta + lane_tok * a.na, a.rounds, d, gm);
      float bt[K];
      ld<K>(bt, a.b + lane_tok * K);
#pragma unroll
      for (int i = 0; i < K; ++i) {
        v[i][0] += bt[i];
        bt[i] = v[i][0];
      }
      st<K, true>(a.out + lane_tok * K, bt);
    }
  }
}

// Gradient of one token: x = dL/dh_t (total), hp = h_{t-1}.  Writes the
// token's angle / scale / decay grads and returns y = M_t^T x in `x`.
template <int K, int SCHED, bool HS, bool HD>
__device__ __forceinline__ void token_grad(float (&x)[K][1], const float (&hp)[K],
                                           const float* __restrict__ th, float* __restrict__ dth,
                                           int rounds, float d, float gm, float& dd, float& dg) {
  float v[K][1];
#pragma unroll
  for (int i = 0; i < K; ++i) v[i][0] = hp[i];
  if (HS) v[1][0] *= d;
  if constexpr (SCHED == SCHED_LEX) {
    constexpr int R = K * (K - 1) / 2;
    float ang[R], cs[R], sn[R], gr[R];
    ld<R>(ang, th);
#pragma unroll
    for (int r = 0; r < R; ++r) mg_sincos(ang[r], sn[r], cs[r]);
    static_for(
        [&](auto rc) {
          constexpr int r = decltype(rc)::value;
          rot_rows<K, 1, lex_first(K, r), lex_second(K, r)>(v, cs[r], sn[r]);
        },
        std::make_index_sequence<R>{});
    if (HD) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < K; ++i) acc = fmaf(x[i][0], v[i][0], acc);
      dg = acc;
#pragma unroll
      for (int i = 0; i < K; ++i) x[i][0] *= gm;
    }
    static_for(
        [&](auto rc) {
          constexpr int r = R - 1 - decltype(rc)::value;
          gr[r] = rot_grad<K, lex_first(K, r), lex_second(K, r)>(v, x, cs[r], sn[r]);
        },
        std::make_index_sequence<R>{});
    st<R, true>(dth, gr);
  } else {
    constexpr int H = K / 2;
    for (int r = 0; r < rounds; ++r) {
      float ang[H], cs[H], sn[H];
      ld<H>(ang, th + r * H);
#pragma unroll
      for (int m = 0; m < H; ++m) mg_sincos(ang[m], sn[m], cs[m]);
      brick_round<K, 1, false>(v, r, cs, sn);
    }
    if (HD) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < K; ++i) acc = fmaf(x[i][0], v[i][0], acc);
      dg = acc;
#pragma unroll
      for (int i = 0; i < K; ++i) x[i][0] *= gm;
    }
    for (int r = rounds - 1; r >= 0; --r) {
      float ang[H], cs[H], sn[H], gr[H];
      ld<H>(ang, th + r * H);
#pragma unroll
      for (int m = 0; m < H; ++m) mg_sincos(ang[m], sn[m], cs[m]);
      if ((r & 1) == 0) {
        static_for(
            [&](auto mc) {
              constexpr int m = decltype(mc)::value;
              constexpr int I = 2 * m, J = I + 1;
              gr[m] = rot_grad<K, I, J>(v, x, cs[m], sn[m]);
            },
            std::make_index_sequence<H>{});
      } else {
        static_for(
            [&](auto mc) {
              constexpr int m = decltype(mc)::value;
              constexpr int I = 2 * m + 1, J = (I + 1) % K;
              gr[m] = rot_grad<K, I, J>(v, x, cs[m], sn[m]);
            },
            std::make_index_sequence<H>{});
      }
      st<H, true>(dth + r * H, gr);
    }
  }
  if (HS) {
    dd = x[1][0] * hp[1];
    x[1][0] *= d;
  }
}

template <int K, int SCHED, bool HS, bool HD>
__global__ __launch_bounds__(MG_WAVE* AN_WAVES) void angle_bwd_kernel(AnArgs a, AfGeom g,
                                                                      unsigned* header,
                                                                      mg_slot_t* agg_data,
                                                                      mg_slot_t* incl_data) {
  AfThread th = af_thread<true>(g, header);
  if (!th.valid) return;
  const int64_t t0 = (int64_t)th.c * (AN_WAVES * AN_TSUB) + th.w * AN_TSUB;
  const int64_t T = g.T, n = g.n;

  // Local reverse aggregate [Q | L]: X <- M_t^T (X + [0 | g_t]) from the end.
  float X[K][K + 1];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int q = 0; q <= K; ++q) X[i][q] = (i == q) ? 1.f : 0.f;
#pragma unroll
  for (int s = AN_TSUB - 1; s >= 0; --s) {
    const int64_t t = t0 + s;
    if (th.ok && t < T) {
      const int64_t lane_tok = (th.bb * T + t) * n + th.plane;
      const float d = HS ? a.scale[lane_tok] : 1.f;
      const float gm = HD ? a.gamma[lane_tok] : 1.f;
      float gt[K];
      ld<K>(gt, a.gh + lane_tok * K);
#pragma unroll
      for (int i = 0; i < K; ++i) X[i][K] += gt[i];
      apply_Mt<K, SCHED, HS, HD, K + 1>(X, a.theta + lane_tok * a.na, a.rounds, d, gm);
    }
  }
  AffM<K, 1> loc, seed, carry;
#pragma unroll
  for (int i = 0; i < K; ++i) {
#pragma unroll
    for (int j = 0; j < K; ++j) loc.P[i][j] = X[i][j];
    loc.L[i][0] = X[i][K];
  }
  affm_identity(seed);
  af_carry<K, 1, AN_WAVES, true>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data, incl_data, carry);

  float y[K][1];
#pragma unroll
  for (int i = 0; i < K; ++i) y[i][0] = carry.L[i][0];
#pragma unroll
  for (int s = AN_TSUB - 1; s >= 0; --s) {
    const int64_t t = t0 + s;
    if (th.ok && t < T) {
      const int64_t lane_tok = (th.bb * T + t) * n + th.plane;
      const float d = HS ? a.scale[lane_tok] : 1.f;
      const float gm = HD ? a.gamma[lane_tok] : 1.f;
      float gt[K], hp[K];
      ld<K>(gt, a.gh + lane_tok * K);
      if (t > 0) ld<K>(hp, a.h + lane_tok * K - n * K);
      else ld<K>(hp, a.h0 + (th.bb * n + th.plane) * K);
#pragma unroll
      for (int i = 0; i < K; ++i) {
        y[i][0] += gt[i];
        gt[i] = y[i][0];
      }
      st<K, true>(a.out + lane_tok * K, gt);  // db_t = dL/dh_t
      float dd = 0.f, dg = 0.f;
      token_grad<K, SCHED, HS, HD>(y, hp, a.theta + lane_tok * a.na, a.dtheta + lane_tok * a.na,
                                   a.rounds, d, gm, dd, dg);
      if (HS) a.dscale[lane_tok] = dd;
      if (HD) a.dgamma[lane_tok] = dg;
    }
  }
  if (t0 == 0 && th.ok) {
    float o[K];
#pragma unroll
    for (int i = 0; i < K; ++i) o[i] = y[i][0];
    st<K>(a.dh0 + (th.bb * n + th.plane) * K, o);
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

AfGeom an_geom(int64_t B, int64_t T, int64_t n) {
  AfGeom g;
  g.T = T;
  g.n = n;
  g.n_tiles = (int)((n + MG_WAVE - 1) / MG_WAVE);
  g.n_lg = (int)(B * g.n_tiles);
  const int64_t cl = (int64_t)AN_WAVES * AN_TSUB;
  g.n_chunks = (int)((T + cl - 1) / cl);
  return g;
}

size_t an_ws_bytes(int64_t B, int64_t T, int64_t n, int k) {
  const AfGeom g = an_geom(B, T, n);
  const size_t data = (size_t)g.n_lg * g.n_chunks * (size_t)(k * k + k) * MG_WAVE *
                      sizeof(mg_slot_t);
  return MG_HEADER_BYTES + 2 * mg_align_up(data, 256);
}

template <int K, int SCHED, bool HS, bool HD, bool BWD>
int an_launch(const AnArgs& a, int64_t B, int64_t T, int64_t n, void* ws, size_t ws_bytes,
              hipStream_t stream) {
  const AfGeom g = an_geom(B, T, n);
  const size_t total = an_ws_bytes(B, T, n, K);
  if (ws_bytes < total) return MG_ERR_WORKSPACE;
  const size_t data = (total - MG_HEADER_BYTES) / 2;
  unsigned* header = (unsigned*)ws;
  mg_slot_t* agg = (mg_slot_t*)((char*)ws + MG_HEADER_BYTES);
  mg_slot_t* incl = (mg_slot_t*)((char*)ws + MG_HEADER_BYTES + data);
  const dim3 grid((unsigned)(g.n_lg * g.n_chunks)), block(MG_WAVE * AN_WAVES);
  if (BWD)
    hipLaunchKernelGGL((angle_bwd_kernel<K, SCHED, HS, HD>), grid, block, 0, stream, a, g, header,
                       agg, incl);
  else
    hipLaunchKernelGGL((angle_fwd_kernel<K, SCHED, HS, HD>), grid, block, 0, stream, a, g, header,
                       agg, incl);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

template <bool BWD>
int an_dispatch(const AnArgs& a, int64_t B, int64_t T, int64_t n, int k, int sched, int flags,
                void* ws, size_t ws_bytes, hipStream_t stream) {
  const bool hs = flags & 1, hd = flags & 2;
#define MG_AN_CASE(KK, SS)                                                                     \
  if (k == KK && sched == SS) {                                                                \
    if (hs && hd) return an_launch<KK, SS, true, true, BWD>(a, B, T, n, ws, ws_bytes, stream);   \
    if (hs) return an_launch<KK, SS, true, false, BWD>(a, B, T, n, ws, ws_bytes, stream);        \
    if (hd) return an_launch<KK, SS, false, true, BWD>(a, B, T, n, ws, ws_bytes, stream);        \
    return an_launch<KK, SS, false, false, BWD>(a, B, T, n, ws, ws_bytes, stream);               \
  }
  MG_AN_CASE(2, SCHED_BRICK)
  MG_AN_CASE(4, SCHED_BRICK)
  MG_AN_CASE(8, SCHED_BRICK)
  MG_AN_CASE(2, SCHED_LEX)
  MG_AN_CASE(4, SCHED_LEX)
  MG_AN_CASE(8, SCHED_LEX)
#undef MG_AN_CASE
  return MG_ERR_ARG;
}

bool an_args_ok(int64_t B, int64_t T, int64_t n, int k, int sched, int rounds) {
  if (B <= 0 || T <= 0 || n <= 0) return false;
  if (k != 2 && k != 4 && k != 8) return false;
  if (sched == SCHED_LEX) return rounds == k * (k - 1) / 2;
  if (sched == SCHED_BRICK) return rounds >= 1 && rounds <= 64;
  return false;
}

bool an_geometry_ok(int64_t B, int64_t T, int64_t n) {
  const AfGeom g = an_geom(B, T, n);
  return (int64_t)g.n_lg * g.n_chunks < (1ll << 24);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

size_t mg_angle_scan_workspace_bytes(int64_t B, int64_t T, int64_t n, int k) {
  if (B <= 0 || T <= 0 || n <= 0 || k <= 0) return 256;
  return an_ws_bytes(B, T, n, k);
}

int mg_angle_scan_fwd(const float* theta, const float* scale, const float* gamma, const float* b,
                      const float* h0, float* h, int64_t B, int64_t T, int64_t n, int k,
                      int sched, int rounds, int flags, void* ws, size_t ws_bytes,
                      hipStream_t stream) {
  if (!theta || !b || !h0 || !h || !ws || !an_args_ok(B, T, n, k, sched, rounds) ||
      !an_geometry_ok(B, T, n))
    return MG_ERR_ARG;
  if (((flags & 1) && !scale) || ((flags & 2) && !gamma)) return MG_ERR_ARG;
  if (!aligned16(theta) || !aligned16(b) || !aligned16(h0) || !aligned16(h)) return MG_ERR_ARG;
  AnArgs a{};
  a.theta = theta;
  a.scale = scale;
  a.gamma = gamma;
  a.b = b;
  a.h0 = h0;
  a.out = h;
  a.rounds = rounds;
  a.na = sched == SCHED_LEX ? k * (k - 1) / 2 : rounds * (k / 2);
  return an_dispatch<false>(a, B, T, n, k, sched, flags, ws, ws_bytes, stream);
}

int mg_angle_scan_bwd(const float* theta, const float* scale, const float* gamma, const float* h0,
                      const float* h, const float* gh, float* dtheta, float* dscale,
                      float* dgamma, float* db, float* dh0, int64_t B, int64_t T, int64_t n,
                      int k, int sched, int rounds, int flags, void* ws, size_t ws_bytes,
                      hipStream_t stream) {
  if (!theta || !h0 || !h || !gh || !dtheta || !db || !dh0 || !ws ||
      !an_args_ok(B, T, n, k, sched, rounds) || !an_geometry_ok(B, T, n))
    return MG_ERR_ARG;
  if (((flags & 1) && (!scale || !dscale)) || ((flags & 2) && (!gamma || !dgamma)))
    return MG_ERR_ARG;
  if (!aligned16(theta) || !aligned16(h0) || !aligned16(h) || !aligned16(gh) ||
      !aligned16(dtheta) || !aligned16(db) || !aligned16(dh0))
    return MG_ERR_ARG;
  AnArgs a{};
  a.theta = theta;
  a.scale = scale;
  a.gamma = gamma;
  a.h0 = h0;
  a.h = h;
  a.gh = gh;
  a.out = db;
  a.dtheta = dtheta;
  a.dscale = dscale;
  a.dgamma = dgamma;
  a.dh0 = dh0;
  a.rounds = rounds;
  a.na = sched == SCHED_LEX ? k * (k - 1) / 2 : rounds * (k / 2);
  return an_dispatch<true>(a, B, T, n, k, sched, flags, ws, ws_bytes, stream);
}

}  // extern "C"

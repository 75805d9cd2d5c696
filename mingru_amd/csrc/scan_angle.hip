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
// Parallel scan over time, reduce-then-scan over chunks of AN_CHUNK tokens
// (no workgroup ever waits on another, so there is no serial chain of
// cross-workgroup hops):
//   pass 1  one lane per (block, chunk) builds the chunk's affine map
//           h -> P_c h + L_c by pushing the k columns of P and the column L
//           through the chunk's rotations (k+1 rotated columns per token);
//   pass 2  two lanes per block walk the chunk boundaries in order,
//           h_{c+1} = P_c h_c + L_c, carrying only its k-vector (half each);
//           for long sequences over groups of AN_GROUP chunks instead (group
//           maps composed in parallel, the walk over the groups, then each
//           group's chunk states filled in in parallel);
//   pass 3  one lane per (block, chunk) re-applies the rotations to the state
//           vector from its chunk-entry state and writes every h_t.
// The forward saves the chunk products P_c for the backward.
//
// Backward: exact stored-state recompute.  h_{t-1} is read from the forward
// output (never reconstructed by dividing out gamma or the scale), the
// per-rotation states are recovered from the recomputed v_R by applying each
// rotation's transpose (orthogonal, so no error amplification), and the
// adjoint y_t = M_t^T (g_t + y_{t+1}) runs through the same three passes in
// reverse time.  Its chunk maps are y -> P_c^T y + Lb_c: the linear part is
// the saved forward product transposed, so pass 1 only sweeps one column.
#include "mg_affm.h"
#include "mg_gates.h"
#include "mg_sincos.h"

#include <algorithm>
#include <utility>

namespace {

using namespace mg;

enum : int { SCHED_BRICK = 0, SCHED_LEX = 1 };
// flags: bit 0 scale, bit 1 decay, bit 2 the gated prologue (mg_angle_scan_gated_*).
constexpr int AN_FLAG_GATED = 4;

// Reduce-then-scan over chunks of AN_CHUNK tokens: pass 1 builds every chunk's
// affine map in parallel (one lane per (block, chunk)), pass 2 walks the chunk
// boundaries of each block carrying only its k-vector, pass 3 re-applies the
// rotations from each chunk's entry state.  No workgroup waits on another.
constexpr int AN_WAVES = 4;          // waves per workgroup of the chunk-parallel passes
constexpr int AN_CHUNK = 16;         // tokens per chunk
constexpr int AN_WALK_THREADS = 64;  // boundary walk: one wave per workgroup (each on its own CU)
constexpr int AN_WALK_AHEAD = 4;     // chunks prefetched ahead by the boundary walk
constexpr int AN_WALK_RING = AN_WALK_AHEAD + 1;
// Two-level boundary walk: the chunk maps of AN_GROUP consecutive chunks are
// composed into one group map (in parallel over groups), the walk runs over the
// groups, and each group's chunk-entry states are filled in from its entry state
// (in parallel again).  Used once a sequence has more than AN_GROUP_MIN chunks.
constexpr int AN_GROUP = 8;
constexpr int AN_GROUP_MIN = 2 * AN_GROUP;
// Up to this many groups the group walk and the fill run as one launch.
constexpr int AN_WALKFILL_GROUPS = 16;

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

// One plane of a brick-wall round: (I, J) rotated, or its transpose applied.
template <int K, int NC, bool TRANSPOSE, int I, int J>
__device__ __forceinline__ void brick_plane(float (&X)[K][NC], float c, float s) {
  if constexpr (TRANSPOSE) rot_rows_t<K, NC, I, J>(X, c, s);
  else rot_rows<K, NC, I, J>(X, c, s);
}

// The K/2 planes of a round of parity PAR: (2m + PAR, 2m + PAR + 1 mod K).  A fold
// over the plane index pack, with no lambda holding X, keeps X in registers when
// the caller loops over rounds at run time.
template <int K, int NC, bool TRANSPOSE, int PAR, int... M>
__device__ __forceinline__ void brick_planes(float (&X)[K][NC], const float (&cs)[K / 2],
                                             const float (&sn)[K / 2],
                                             std::integer_sequence<int, M...>) {
  (brick_plane<K, NC, TRANSPOSE, 2 * M + PAR, (2 * M + PAR + 1) % K>(X, cs[M], sn[M]), ...);
}

// Round r of the brick-wall schedule with its parity PAR fixed at compile time:
// the round's K/2 angles read from th + r K/2 and its planes rotated (TRANSPOSE:
// the transposed rotations).
template <int K, int NC, bool TRANSPOSE, int PAR>
__device__ __forceinline__ void brick_round_at(float (&X)[K][NC], const float* __restrict__ th,
                                               int r) {
  constexpr int H = K / 2;
  float ang[H], cs[H], sn[H];
  ld<H>(ang, th + r * H);
#pragma unroll
  for (int m = 0; m < H; ++m) mg_sincos(ang[m], sn[m], cs[m]);
  brick_planes<K, NC, TRANSPOSE, PAR>(X, cs, sn, std::make_integer_sequence<int, H>{});
}

// All `rounds` rounds of a token: 0 .. rounds-1 in order, or (TRANSPOSE) their
// transposes from rounds-1 down to 0.  Two rounds per iteration, even then odd
// (transposed: odd then even), so that no branch inside the loop depends on a
// round's parity: with one, the fwd reduce pass's state block [P | L] was kept in
// scratch memory instead of registers.
template <int K, int NC, bool TRANSPOSE>
__device__ __forceinline__ void brick_rounds(float (&X)[K][NC], const float* __restrict__ th,
                                             int rounds) {
  if constexpr (!TRANSPOSE) {
    int r = 0;
    for (; r + 2 <= rounds; r += 2) {
      brick_round_at<K, NC, false, 0>(X, th, r);
      brick_round_at<K, NC, false, 1>(X, th, r + 1);
    }
    if (r < rounds) brick_round_at<K, NC, false, 0>(X, th, r);
  } else {
    int r = rounds - 1;
    if (r >= 1 && (r & 1)) {  // the last round is odd: it goes first
      brick_round_at<K, NC, true, 1>(X, th, r);
      --r;
    }
    for (; r >= 2; r -= 2) {  // r even
      brick_round_at<K, NC, true, 0>(X, th, r);
      brick_round_at<K, NC, true, 1>(X, th, r - 1);
    }
    if (r == 0) brick_round_at<K, NC, true, 0>(X, th, 0);
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
    brick_rounds<K, NC, false>(X, th, rounds);
  }
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
}

// Lexicographic schedule with the token's R angles already in registers.
template <int K, bool HS, bool HD, int NC>
__device__ __forceinline__ void apply_M_lex(float (&X)[K][NC], const float (&ang)[K * (K - 1) / 2],
                                            float d, float gm) {
  constexpr int R = K * (K - 1) / 2;
  if (HS) {
#pragma unroll
    for (int q = 0; q < NC; ++q) X[1][q] *= d;
  }
  static_for(
      [&](auto rc) {
        constexpr int r = decltype(rc)::value;
        float sn, cs;
        mg_sincos(ang[r], sn, cs);
        rot_rows<K, NC, lex_first(K, r), lex_second(K, r)>(X, cs, sn);
      },
      std::make_index_sequence<R>{});
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
}

template <int K, bool HS, bool HD, int NC>
__device__ __forceinline__ void apply_Mt_lex(float (&X)[K][NC],
                                             const float (&ang)[K * (K - 1) / 2], float d,
                                             float gm) {
  constexpr int R = K * (K - 1) / 2;
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
  static_for(
      [&](auto rc) {
        constexpr int r = R - 1 - decltype(rc)::value;
        float sn, cs;
        mg_sincos(ang[r], sn, cs);
        rot_rows_t<K, NC, lex_first(K, r), lex_second(K, r)>(X, cs, sn);
      },
      std::make_index_sequence<R>{});
  if (HS) {
#pragma unroll
    for (int q = 0; q < NC; ++q) X[1][q] *= d;
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
    brick_rounds<K, NC, true>(X, th, rounds);
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
  float* prod;   // chunk products P_c, [chunk][block][K*K]: forward writes, backward reads
  float* lsum;   // chunk offsets (forward L_c, backward adjoint offsets), [chunk][block][K]
  float* bound;  // chunk-entry states (forward) / adjoints (backward), [chunk][block][K]
  // Two-level walk only: group maps [group][block][K*K] (the forward's, saved after
  // the chunk products) and group offsets [group][block][K] of the pass's direction.
  float* gprod;
  float* gsum;
  // Gated prologue (GP, brick-wall kernels): `b` holds z and `hpre` the candidate, so
  // b_t = sigmoid(z) hpre; `scale` holds u, so the scale is tanh(u).  The backward
  // then writes dL/dz to `out`, dL/dhpre to `dhpre` and dL/du to `dscale`.
  const float* hpre;
  float* dhpre;
  int rounds;
  int na;  // angles per token
};

// The per-token scale and input of the brick-wall kernels, plain or through the gated
// prologue (the RotationMinGRU / GivensMinGRU heads, reference src/mingru/min_gru.py:
// 2261-2262, 2719: scale = tanh(linear_u x), b = sigmoid(linear_z x) * linear_h x).
template <bool GP>
__device__ __forceinline__ float an_scale(const AnArgs& a, int64_t lane_tok) {
  return GP ? mg_tanh(a.scale[lane_tok]) : a.scale[lane_tok];
}

template <int K, bool GP>
__device__ __forceinline__ void an_input(const AnArgs& a, int64_t lane_tok, float (&bt)[K]) {
  if constexpr (GP) {
    float zz[K], hp[K];
    ld<K>(zz, a.b + lane_tok * K);
    ld<K>(hp, a.hpre + lane_tok * K);
#pragma unroll
    for (int i = 0; i < K; ++i) bt[i] = mg_sigmoid(zz[i]) * hp[i];
  } else {
    ld<K>(bt, a.b + lane_tok * K);
  }
}

// db_t = dL/dh_t (the token's adjoint) stored, or through the gated prologue dL/dz
// and dL/dhpre.
template <int K, bool GP>
__device__ __forceinline__ void an_store_db(const AnArgs& a, int64_t lane_tok,
                                            const float (&gt)[K]) {
  if constexpr (GP) {
    float zz[K], hp[K], dz[K], dh[K];
    ld<K>(zz, a.b + lane_tok * K);
    ld<K>(hp, a.hpre + lane_tok * K);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const float sg = mg_sigmoid(zz[i]);
      dh[i] = gt[i] * sg;
      dz[i] = dh[i] * hp[i] * (1.f - sg);
    }
    st<K>(a.out + lane_tok * K, dz);
    st<K>(a.dhpre + lane_tok * K, dh);
  } else {
    st<K>(a.out + lane_tok * K, gt);
  }
}

// an_input and an_store_db with the token's z, hpre (gated) or b already in registers.
template <int K, bool GP>
__device__ __forceinline__ void an_input_reg(const float (&v)[K], const float (&hq)[GP ? K : 1],
                                             float (&bt)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if constexpr (GP) bt[i] = mg_sigmoid(v[i]) * hq[i];
    else bt[i] = v[i];
  }
}

template <int K, bool GP>
__device__ __forceinline__ void an_store_db_reg(const AnArgs& a, int64_t lane_tok,
                                                const float (&gt)[K], const float (&zz)[GP ? K : 1],
                                                const float (&hp)[GP ? K : 1]) {
  if constexpr (GP) {
    float dz[K], dh[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const float sg = mg_sigmoid(zz[i]);
      dh[i] = gt[i] * sg;
      dz[i] = dh[i] * hp[i] * (1.f - sg);
    }
    st<K>(a.out + lane_tok * K, dz);
    st<K>(a.dhpre + lane_tok * K, dh);
  } else {
    st<K>(a.out + lane_tok * K, gt);
  }
}

// Per-token inputs of the lexicographic kernels, loaded one token ahead: at one
// wave per SIMD nothing else hides a load issued only when it is needed.
template <int K, bool HS, bool HD>
struct LexTok {
  static constexpr int R = K * (K - 1) / 2;
  float ang[R];
  float v[K];   // b_t (forward) or g_t (backward)
  float hp[K];  // h_{t-1} (backward final pass only)
  float d, gm;

  template <bool HP>
  __device__ __forceinline__ void load(const AnArgs& a, const float* vec, int64_t lane_tok,
                                       int64_t t, int64_t n, int64_t blk) {
    ld<R>(ang, a.theta + lane_tok * R);
    ld<K>(v, vec + lane_tok * K);
    d = HS ? a.scale[lane_tok] : 1.f;
    gm = HD ? a.gamma[lane_tok] : 1.f;
    if constexpr (HP) {
      if (t > 0) ld<K>(hp, a.h + lane_tok * K - n * K);
      else ld<K>(hp, a.h0 + blk * K);
    }
  }
};

// Per-token inputs of the brick-wall kernels with R rounds fixed at compile time (the
// mixers' R = 3, and RotationMinGRU's R = 1), loaded one token ahead as LexTok's are;
// other round counts take the per-token loop.  v: b_t, or z_t under the gated
// prologue (forward), or g_t (backward); hq: the gated prologue's hpre_t; zb: z_t in
// the gated backward final pass; hp: h_{t-1} (backward final pass).
template <int K, int R, bool HS, bool HD, bool HQ, bool ZB, bool HP>
struct BrickTok {
  static constexpr int H = K / 2;
  float ang[R][H];
  float v[K];
  float hq[HQ ? K : 1];
  float zb[ZB ? K : 1];
  float hp[HP ? K : 1];
  float d, gm;  // the scale input (u under the gated prologue) and the decay

  __device__ __forceinline__ void load(const AnArgs& a, const float* vec, int64_t lane_tok,
                                       int64_t t, int64_t n, int64_t blk) {
    const float* th = a.theta + lane_tok * (R * H);
#pragma unroll
    for (int r = 0; r < R; ++r) ld<H>(ang[r], th + r * H);
    ld<K>(v, vec + lane_tok * K);
    if constexpr (HQ) ld<K>(hq, a.hpre + lane_tok * K);
    if constexpr (ZB) ld<K>(zb, a.b + lane_tok * K);
    d = HS ? a.scale[lane_tok] : 1.f;
    gm = HD ? a.gamma[lane_tok] : 1.f;
    if constexpr (HP) {
      if (t > 0) ld<K>(hp, a.h + lane_tok * K - n * K);
      else ld<K>(hp, a.h0 + blk * K);
    }
  }
};

// The R brick-wall rounds of a token with its angles in registers: rounds 0 .. R-1,
// or (TRANSPOSE) their transposes from R-1 down to 0.
template <int K, int NC, bool TRANSPOSE, int R>
__device__ __forceinline__ void brick_rounds_reg(float (&X)[K][NC], const float (&ang)[R][K / 2]) {
  constexpr int H = K / 2;
  static_for(
      [&](auto rc) {
        constexpr int r = TRANSPOSE ? R - 1 - decltype(rc)::value : decltype(rc)::value;
        float cs[H], sn[H];
#pragma unroll
        for (int m = 0; m < H; ++m) mg_sincos(ang[r][m], sn[m], cs[m]);
        brick_planes<K, NC, TRANSPOSE, r & 1>(X, cs, sn, std::make_integer_sequence<int, H>{});
      },
      std::make_index_sequence<R>{});
}

// X <- M_t X and X <- M_t^T X (apply_M / apply_Mt) with the angles in registers.
template <int K, int R, bool HS, bool HD, int NC>
__device__ __forceinline__ void apply_M_brick(float (&X)[K][NC], const float (&ang)[R][K / 2],
                                              float d, float gm) {
  if (HS) {
#pragma unroll
    for (int q = 0; q < NC; ++q) X[1][q] *= d;
  }
  brick_rounds_reg<K, NC, false, R>(X, ang);
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
}

template <int K, int R, bool HS, bool HD, int NC>
__device__ __forceinline__ void apply_Mt_brick(float (&X)[K][NC], const float (&ang)[R][K / 2],
                                               float d, float gm) {
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int q = 0; q < NC; ++q) X[i][q] *= gm;
  }
  brick_rounds_reg<K, NC, true, R>(X, ang);
  if (HS) {
#pragma unroll
    for (int q = 0; q < NC; ++q) X[1][q] *= d;
  }
}

// Runs body(tok, t) over `count` tokens t = first, first + dir, ..., each token's
// inputs loaded one token ahead into two alternating buffers.  The next token's
// loads are issued unconditionally (the index clamped to the range) before the
// current token's body and in the same basic block, so they overlap it.  A
// conditional prefetch into a buffer copied at the loop's end let the compiler
// sink the loads down to the copy, next to their first use.
// Scheduling barriers keep the compiler from moving work across the prefetches.
// That bounds the registers of a body as large as the forward reduce pass's (some of
// its instances spilled without them), and the other token passes measured faster
// with them too (C4 backward 114.7 -> 111.5 us).
template <typename Tok, typename Load, typename Body>
__device__ __forceinline__ void token_pairs(int64_t first, int count, int dir, Load&& load,
                                            Body&& body) {
  Tok A, B;
  load(A, first);
  const int64_t last = first + (int64_t)(count - 1) * dir;
  int i = 0;
  for (; i + 2 <= count; i += 2) {
    const int64_t t = first + (int64_t)i * dir;
    load(B, t + dir);
    __builtin_amdgcn_sched_barrier(0);
    body(A, t);
    load(A, i + 2 < count ? t + 2 * dir : last);
    __builtin_amdgcn_sched_barrier(0);
    body(B, t + dir);
  }
  if (i < count) body(A, first + (int64_t)i * dir);
}

struct AnGeom {
  int64_t T, n, NB;  // tokens, blocks per batch row, blocks in total (B * n)
  int n_tiles, n_lg, n_chunks;
  int n_run, n_groups;  // runs of AN_RUN consecutive blocks, groups of AN_GROUP chunks
};

// Chunk-parallel passes: one wave per (lane group, chunk), one lane per block.
struct AnThread {
  int64_t bb, plane, blk;
  int c;
  bool ok;
};

__device__ __forceinline__ AnThread an_thread(const AnGeom& g) {
  AnThread th;
  const int64_t gw = (int64_t)blockIdx.x * AN_WAVES + threadIdx.x / MG_WAVE;
  const int lane = threadIdx.x & (MG_WAVE - 1);
  const int lg = (int)(gw % g.n_lg);
  th.c = (int)(gw / g.n_lg);
  th.bb = lg / g.n_tiles;
  th.plane = (int64_t)(lg % g.n_tiles) * MG_WAVE + lane;
  th.ok = th.c < g.n_chunks && th.plane < g.n;
  th.blk = th.bb * g.n + th.plane;
  return th;
}

// Forward reduce pass: one workgroup per (run of AN_RUN consecutive blocks, group of
// AN_GROUP consecutive chunks).  Thread 32 j + b of each half of the workgroup holds
// chunk j of the group for block b of the run -- the first half the chunk's first
// AN_CHUNK / 2 tokens, the second half the rest -- so wave w of a half holds chunks
// 2w and 2w + 1 (a token row of 32 consecutive blocks per chunk, 3.5 KB of angles at
// k = 8).  The two halves' maps are composed into the chunk maps through LDS, and
// the workgroup then holds every chunk map of its blocks' group, which it composes
// into the group maps of the two-level walk.  One thread per (block, chunk) gave
// one wave per SIMD at C4, too few to keep the rotations' VALU work issuing.
constexpr int AN_RUN = 32;
constexpr int AN_HALF = MG_WAVE * AN_WAVES;  // threads per half of a reduce workgroup
constexpr int AN_RED_THREADS = 2 * AN_HALF;
static_assert(AN_RUN * AN_GROUP == AN_HALF, "a workgroup half is one group of chunks");

struct AnRThread {
  int64_t bb, plane, blk;
  int c, grp, j, b, cnt;  // cnt: chunks in the group (uniform)
  bool live;              // the block exists: the thread joins the compose
  bool ok;                // ... and so does the chunk: the thread reduces it
  bool full;              // every lane of the wave is ok (wave-uniform)
};

// The reduce thread q = 32 j + b of a workgroup half (q < AN_HALF).
__device__ __forceinline__ AnRThread an_rthread(const AnGeom& g, int q) {
  AnRThread th;
  const int run = (int)(blockIdx.x % (unsigned)g.n_run);
  th.grp = (int)(blockIdx.x / (unsigned)g.n_run);
  th.j = q / AN_RUN;
  th.b = q % AN_RUN;
  th.blk = (int64_t)run * AN_RUN + th.b;
  th.c = th.grp * AN_GROUP + th.j;
  th.cnt = min(AN_GROUP, g.n_chunks - th.grp * AN_GROUP);
  th.live = th.blk < g.NB;
  th.ok = th.live && th.c < g.n_chunks;
  th.full = (int64_t)(run + 1) * AN_RUN <= g.NB && (th.c | 1) < g.n_chunks;
  th.bb = th.blk / g.n;
  th.plane = th.blk % g.n;
  return th;
}

// LDS row of one reduce thread: its chunk map [P | L] (K*K + K floats), padded so
// that the rows of 16 consecutive blocks of one chunk fall in distinct banks.
template <int K>
constexpr int an_row_stride() {
  return (K * K + K + 3) / 4 * 4 + 4;
}

// Index of field f of chunk c for block blk in a [chunk][block][field] array:
// a lane's fields are contiguous, and so are the k lanes of one block in the
// boundary walk.
__device__ __forceinline__ int64_t an_idx(const AnGeom& g, int c, int f, int nf, int64_t blk) {
  return ((int64_t)c * g.NB + blk) * nf + f;
}

// Orders the LDS accesses of one wave's lanes around it (no s_barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Stores one R-float row per lane when the 64 lanes' rows are consecutive in
// memory (lane l's row at dst0 + l R; the whole wave active).  The rows pass
// through LDS, so each store instruction writes 1 KiB of consecutive bytes (whole
// lines) instead of a 16-byte piece of each of 64 rows.  Called at the end of a
// token's work: its waits then find the next token's prefetched loads done.
template <int R>
__device__ __forceinline__ void wave_rows_store(float* __restrict__ dst0, const float (&row)[R],
                                                float* lds, int lane) {
  static_assert(R % 4 == 0, "rows of whole 16-byte pieces");
  wave_sync();  // the previous call's reads are done before this call's writes
#pragma unroll
  for (int k = 0; k < R; k += 4)
    *reinterpret_cast<float4*>(lds + lane * R + k) =
        make_float4(row[k], row[k + 1], row[k + 2], row[k + 3]);
  wave_sync();
#pragma unroll
  for (int k = 0; k < R / 4; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(lds + (k * MG_WAVE + lane) * 4);
    *reinterpret_cast<float4*>(dst0 + (k * MG_WAVE + lane) * 4) = v;
  }
}

// ---- forward pass 1: chunk aggregates h -> P_c h + L_c ------------------------
// Each half of the workgroup pushes [P | L] through its half of the chunk's tokens;
// the pair compose (P2 P1, P2 L1 + L2) is split between the pair's two threads by
// columns of P and rows of L.  With the two-level walk the workgroup then composes
// its group maps h -> Pg h + Lg over chunks c0 .. c1: thread (j < K, b) carries
// column j of block b's Pg (and, redundantly, its Lg) through the group's chunk
// maps read back from LDS.
template <int K, int SCHED, bool HS, bool HD, bool GP = false>
__global__ __launch_bounds__(AN_RED_THREADS) void angle_fwd_reduce(AnArgs a, AnGeom g) {
  static_assert(K % 2 == 0, "the pair compose splits the columns of P in two");
  mg_sincos_setup();
  const int q = threadIdx.x % AN_HALF, half = threadIdx.x / AN_HALF;
  const AnRThread th = an_rthread(g, q);
  // Push [P | L] through this half's tokens.
  float X[K][K + 1];
#pragma unroll
  for (int i = 0; i < K; ++i)
#pragma unroll
    for (int c = 0; c <= K; ++c) X[i][c] = (i == c) ? 1.f : 0.f;
  // The decay is a scalar per token, so it commutes with the rotations: P's K
  // columns take the product of the half's decays once at the end, and only the
  // offset column, which receives b_t every token, is decayed token by token.
  float gprod = 1.f;
  if (th.ok) {
    const int64_t t0 = (int64_t)th.c * AN_CHUNK + half * (AN_CHUNK / 2);
    const int64_t te = min(t0 + AN_CHUNK / 2, g.T);
    if (t0 < te) {
      if constexpr (SCHED == SCHED_LEX) {
        using Tok = LexTok<K, HS, HD>;
        token_pairs<Tok>(
            t0, (int)(te - t0), 1,
            [&](Tok& k, int64_t t) {
              k.template load<false>(a, a.b, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
            },
            [&](const Tok& cur, int64_t) {
              apply_M_lex<K, HS, false, K + 1>(X, cur.ang, cur.d, 1.f);
              if (HD) gprod *= cur.gm;
#pragma unroll
              for (int i = 0; i < K; ++i)
                X[i][K] = HD ? fmaf(cur.gm, X[i][K], cur.v[i]) : X[i][K] + cur.v[i];
            });
      } else {
        brick_dispatch(a.rounds, [&](auto rc) {
          constexpr int R = decltype(rc)::value;
          if constexpr (R > 0) {
            using Tok = BrickTok<K, R, HS, HD, GP, false, false>;
            token_pairs<Tok>(
                t0, (int)(te - t0), 1,
                [&](Tok& k, int64_t t) {
                  k.load(a, a.b, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
                },
                [&](const Tok& cur, int64_t) {
                  const float d = HS ? (GP ? mg_tanh(cur.d) : cur.d) : 1.f;
                  apply_M_brick<K, R, HS, false, K + 1>(X, cur.ang, d, 1.f);
                  if (HD) gprod *= cur.gm;
                  float bt[K];
                  an_input_reg<K, GP>(cur.v, cur.hq, bt);
#pragma unroll
                  for (int i = 0; i < K; ++i)
                    X[i][K] = HD ? fmaf(cur.gm, X[i][K], bt[i]) : X[i][K] + bt[i];
                });
          } else {
            for (int64_t t = t0; t < te; ++t) {
              const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
              const float d = HS ? an_scale<GP>(a, lane_tok) : 1.f;
              const float gm = HD ? a.gamma[lane_tok] : 1.f;
              apply_M<K, SCHED, HS, false, K + 1>(X, a.theta + lane_tok * a.na, a.rounds, d, 1.f);
              if (HD) gprod *= gm;
              float bt[K];
              an_input<K, GP>(a, lane_tok, bt);
#pragma unroll
              for (int i = 0; i < K; ++i)
                X[i][K] = HD ? fmaf(gm, X[i][K], bt[i]) : X[i][K] + bt[i];
            }
          }
        });
      }
    }
  }
  if (HD) {
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int c = 0; c < K; ++c) X[i][c] *= gprod;
  }
  // Rows of LDS: thread t's half map [P | L] in row t; the chunk maps then replace
  // the first half's rows (row q = 32 j + b: chunk j of block b).
  constexpr int RS = an_row_stride<K>();
  __shared__ __attribute__((aligned(16))) float s_rows[AN_RED_THREADS * RS];
  const int lane = threadIdx.x & (MG_WAVE - 1), w = threadIdx.x / MG_WAVE;
  {
    float* row = s_rows + threadIdx.x * RS;
    float Pf[K * K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
#pragma unroll
      for (int c = 0; c < K; ++c) Pf[i * K + c] = X[i][c];
      row[K * K + i] = X[i][K];
    }
#pragma unroll
    for (int k = 0; k < K * K; k += 4)
      *reinterpret_cast<float4*>(row + k) = make_float4(Pf[k], Pf[k + 1], Pf[k + 2], Pf[k + 3]);
  }
  __syncthreads();
  // Pair compose for chunk q: this thread forms columns H half .. of P = P2 P1 and
  // rows H half .. of L = P2 L1 + L2 (H = K / 2).
  constexpr int H = K / 2;
  float Pn[K][H], Ln[H];
  {
    const float* r1 = s_rows + q * RS;             // first half of the chunk
    const float* r2 = s_rows + (AN_HALF + q) * RS;  // second half
    float p1[K][H], l1[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
      for (int c = 0; c < H; ++c) p1[k][c] = r1[k * K + H * half + c];
      l1[k] = r1[K * K + k];
    }
#pragma unroll
    for (int i = 0; i < K; ++i) {
      float p2[K];
      if constexpr (K % 4 == 0) {
#pragma unroll
        for (int k = 0; k < K; k += 4) {
          const float4 v = *reinterpret_cast<const float4*>(r2 + i * K + k);
          p2[k] = v.x;
          p2[k + 1] = v.y;
          p2[k + 2] = v.z;
          p2[k + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int k = 0; k < K; ++k) p2[k] = r2[i * K + k];
      }
#pragma unroll
      for (int c = 0; c < H; ++c) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc = fmaf(p2[k], p1[k][c], acc);
        Pn[i][c] = acc;
      }
      if (i / H == half) {
        float acc = r2[K * K + i];
#pragma unroll
        for (int k = 0; k < K; ++k) acc = fmaf(p2[k], l1[k], acc);
        Ln[i % H] = acc;
      }
    }
  }
  __syncthreads();  // every pair has read both halves' rows
  {
    float* row = s_rows + q * RS;
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int c = 0; c < H; ++c) row[i * K + H * half + c] = Pn[i][c];
#pragma unroll
    for (int i = 0; i < H; ++i) row[K * K + H * half + i] = Ln[i];
  }
  __syncthreads();
  if (half) return;  // the first half stores the chunk maps and composes the groups
  if (th.full) {
    // Piece p: floats 4 (64 p + lane) .. of the wave's 64 rows; the rows of one
    // piece are consecutive blocks of one chunk.
    const int64_t blk0 = th.blk - th.b;
#pragma unroll
    for (int p = 0; p < K * K / 4; ++p) {
      const int o = (p * MG_WAVE + lane) * 4, r = o / (K * K), col = o % (K * K);
      const float4 v = *reinterpret_cast<const float4*>(s_rows + (w * MG_WAVE + r) * RS + col);
      *reinterpret_cast<float4*>(a.prod + an_idx(g, th.grp * AN_GROUP + 2 * w + r / AN_RUN, col,
                                                 K * K, blk0 + r % AN_RUN)) = v;
    }
  } else if (th.ok) {
    float Pf[K * K];
#pragma unroll
    for (int k = 0; k < K * K; ++k) Pf[k] = s_rows[q * RS + k];
    st<K * K>(a.prod + an_idx(g, th.c, 0, K * K, th.blk), Pf);
  }
  if (th.ok) {
    float Lf[K];
#pragma unroll
    for (int i = 0; i < K; ++i) Lf[i] = s_rows[q * RS + K * K + i];
    st<K>(a.lsum + an_idx(g, th.c, 0, K, th.blk), Lf);
  }
  if (g.n_chunks <= AN_GROUP_MIN) return;  // uniform
  if (!th.live || th.j >= K) return;
  float m[K], l[K];  // column j and offset of the maps composed so far (chunk c0's)
#pragma unroll
  for (int i = 0; i < K; ++i) {
    m[i] = s_rows[th.b * RS + i * K + th.j];
    l[i] = s_rows[th.b * RS + K * K + i];
  }
  for (int s = 1; s < th.cnt; ++s) {
    const float* row = s_rows + (s * AN_RUN + th.b) * RS;
    float P[K * K], L[K];
#pragma unroll
    for (int k = 0; k < K * K; k += 4) {
      const float4 v = *reinterpret_cast<const float4*>(row + k);
      P[k] = v.x;
      P[k + 1] = v.y;
      P[k + 2] = v.z;
      P[k + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < K; ++i) L[i] = row[K * K + i];
    float nm[K], nl[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      float am = 0.f, al = L[i];
#pragma unroll
      for (int c = 0; c < K; ++c) {
        am = fmaf(P[i * K + c], m[c], am);
        al = fmaf(P[i * K + c], l[c], al);
      }
      nm[i] = am;
      nl[i] = al;
    }
#pragma unroll
    for (int i = 0; i < K; ++i) {
      m[i] = nm[i];
      l[i] = nl[i];
    }
  }
  float* out = a.gprod + an_idx(g, th.grp, 0, K * K, th.blk);
#pragma unroll
  for (int i = 0; i < K; ++i) out[i * K + th.j] = m[i];
  if (th.j == 0) st<K>(a.gsum + an_idx(g, th.grp, 0, K, th.blk), l);
}

// ---- forward pass 2: states at chunk boundaries, h_{c+1} = P_c h_c + L_c -------
// Two lanes per block, lane p owning state rows K/2 p .. K/2 p + K/2 - 1.  Each
// lane loads columns K/2 p .. of every row of P_c (one 16-byte piece per row, so
// the two lanes of a block read each row's 32 bytes together), forms the partial
// sums of all K rows over its own half of h, and the pair exchanges the partials
// of each other's rows by DPP quad_perm moves (no LDS crossbar).  The loads are
// prefetched AN_WALK_AHEAD chunks ahead in a ring of registers.

// The partner lane's value (lane ^ 1), by DPP quad_perm [1, 0, 3, 2].
__device__ __forceinline__ float pair_swap(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
}

// Own-row results from partial sums over the lane's half: part[i] covers all K rows;
// out[i] = base[i] + own partial + the partner's partial for row H p + i.
template <int K>
__device__ __forceinline__ void pair_reduce(const float (&part)[K], int p, const float* base,
                                            float* out) {
  constexpr int H = K / 2;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float mine = p ? part[H + i] : part[i], theirs = p ? part[i] : part[H + i];
    out[i] = base[i] + mine + pair_swap(theirs);
  }
}

template <int K>
__global__ __launch_bounds__(AN_WALK_THREADS) void angle_fwd_scan(AnArgs a, AnGeom g) {
  constexpr int H = K / 2;
  const int64_t gt = (int64_t)blockIdx.x * AN_WALK_THREADS + threadIdx.x;
  const int64_t blk = gt >> 1;
  const int p = (int)(gt & 1);
  if (blk >= g.NB) return;  // the two lanes of a block leave together
  struct Op {
    float P[K * H];  // [i][jj]: row i of P_c, column H p + jj
    float L[H];
  };
  auto fetch = [&](Op& o, int c) {
    c = min(c, g.n_chunks - 1);  // clamped reads past the end are unused
    const float* pc = a.prod + an_idx(g, c, H * p, K * K, blk);
#pragma unroll
    for (int i = 0; i < K; ++i) ld<H>(o.P + i * H, pc + i * K);
    ld<H>(o.L, a.lsum + an_idx(g, c, H * p, K, blk));
  };
  float h[H];
  ld<H>(h, a.h0 + blk * K + H * p);
  auto step = [&](const Op& o, Op& fill, int c) {
    fetch(fill, c + AN_WALK_AHEAD);
    st<H>(a.bound + an_idx(g, c, H * p, K, blk), h);
    float part[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int jj = 0; jj < H; ++jj) acc = fmaf(o.P[i * H + jj], h[jj], acc);
      part[i] = acc;
    }
    pair_reduce<K>(part, p, o.L, h);
  };
  constexpr int R = AN_WALK_RING;  // ring: chunk c sits in slot c % R, the loop unrolled by R
  Op buf[R];
#pragma unroll
  for (int d = 0; d < R - 1; ++d) fetch(buf[d], d);
  int c = 0;
  for (; c + R <= g.n_chunks; c += R) {
#pragma unroll
    for (int d = 0; d < R; ++d) step(buf[d], buf[(d + R - 1) % R], c + d);
  }
#pragma unroll
  for (int d = 0; d < R - 1; ++d)
    if (c + d < g.n_chunks) step(buf[d], buf[(d + R - 1) % R], c + d);
}

// ---- forward pass 3: every token's state from its chunk-entry state ------------
template <int K, int SCHED, bool HS, bool HD, bool GP = false>
__global__ __launch_bounds__(MG_WAVE* AN_WAVES) void angle_fwd_final(AnArgs a, AnGeom g) {
  mg_sincos_setup();
  const AnThread th = an_thread(g);
  if (!th.ok) return;
  const int64_t t0 = (int64_t)th.c * AN_CHUNK;
  float v[K][1];
  {
    float b0[K];
    ld<K>(b0, a.bound + an_idx(g, th.c, 0, K, th.blk));
#pragma unroll
    for (int i = 0; i < K; ++i) v[i][0] = b0[i];
  }
  const int64_t te = min(t0 + AN_CHUNK, g.T);
  if constexpr (SCHED == SCHED_LEX) {
    using Tok = LexTok<K, HS, HD>;
    token_pairs<Tok>(
        t0, (int)(te - t0), 1,
        [&](Tok& k, int64_t t) {
          k.template load<false>(a, a.b, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
        },
        [&](const Tok& cur, int64_t t) {
          const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
          apply_M_lex<K, HS, HD, 1>(v, cur.ang, cur.d, cur.gm);
          float bt[K];
#pragma unroll
          for (int i = 0; i < K; ++i) {
            v[i][0] += cur.v[i];
            bt[i] = v[i][0];
          }
          st<K>(a.out + lane_tok * K, bt);  // k floats per lane: L2 merges the rows
        });
  } else {
    brick_dispatch(a.rounds, [&](auto rc) {
      constexpr int R = decltype(rc)::value;
      if constexpr (R > 0) {
        using Tok = BrickTok<K, R, HS, HD, GP, false, false>;
        token_pairs<Tok>(
            t0, (int)(te - t0), 1,
            [&](Tok& k, int64_t t) {
              k.load(a, a.b, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
            },
            [&](const Tok& cur, int64_t t) {
              const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
              const float d = HS ? (GP ? mg_tanh(cur.d) : cur.d) : 1.f;
              apply_M_brick<K, R, HS, HD, 1>(v, cur.ang, d, cur.gm);
              float bt[K];
              an_input_reg<K, GP>(cur.v, cur.hq, bt);
#pragma unroll
              for (int i = 0; i < K; ++i) {
                v[i][0] += bt[i];
                bt[i] = v[i][0];
              }
              st<K>(a.out + lane_tok * K, bt);  // k floats per lane: L2 merges the rows
            });
      } else {
        for (int64_t t = t0; t < te; ++t) {
          const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
          const float d = HS ? an_scale<GP>(a, lane_tok) : 1.f;
          const float gm = HD ? a.gamma[lane_tok] : 1.f;
          apply_M<K, SCHED, HS, HD, 1>(v, a.theta + lane_tok * a.na, a.rounds, d, gm);
          float bt[K];
          an_input<K, GP>(a, lane_tok, bt);
#pragma unroll
          for (int i = 0; i < K; ++i) {
            v[i][0] += bt[i];
            bt[i] = v[i][0];
          }
          st<K>(a.out + lane_tok * K, bt);  // k floats per lane: L2 merges the rows
        }
      }
    });
  }
}

// token_grad for the lexicographic schedule with the angles already loaded.
template <int K, bool HS, bool HD>
__device__ __forceinline__ void token_grad_lex(float (&x)[K][1], const float (&hp)[K],
                                               const float (&ang)[K * (K - 1) / 2],
                                               float (&gr)[K * (K - 1) / 2], float d, float gm,
                                               float& dd, float& dg) {
  constexpr int R = K * (K - 1) / 2;
  float v[K][1];
#pragma unroll
  for (int i = 0; i < K; ++i) v[i][0] = hp[i];
  if (HS) v[1][0] *= d;
  float cs[R], sn[R];
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
  if (HS) {
    dd = x[1][0] * hp[1];
    x[1][0] *= d;
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
    st<R>(dth, gr);  // partial-line rows: L2 merges them (no streaming hint)
  } else {
    constexpr int H = K / 2;
    brick_rounds<K, 1, false>(v, th, rounds);
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
      st<H>(dth + r * H, gr);  // partial-line rows: L2 merges them
    }
  }
  if (HS) {
    dd = x[1][0] * hp[1];
    x[1][0] *= d;
  }
}

// token_grad for the brick-wall schedule with the R rounds' angles in registers: each
// angle's sin and cos are evaluated once for both sweeps, and dtheta is returned in gr
// (round-major, as the angles are stored).
template <int K, int R, bool HS, bool HD>
__device__ __forceinline__ void token_grad_brick(float (&x)[K][1], const float (&hp)[K],
                                                 const float (&ang)[R][K / 2],
                                                 float (&gr)[R * (K / 2)], float d, float gm,
                                                 float& dd, float& dg) {
  constexpr int H = K / 2;
  float v[K][1];
#pragma unroll
  for (int i = 0; i < K; ++i) v[i][0] = hp[i];
  if (HS) v[1][0] *= d;
  float cs[R][H], sn[R][H];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < H; ++m) mg_sincos(ang[r][m], sn[r][m], cs[r][m]);
  static_for(
      [&](auto rc) {
        constexpr int r = decltype(rc)::value;
        brick_planes<K, 1, false, r & 1>(v, cs[r], sn[r], std::make_integer_sequence<int, H>{});
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
        static_for(
            [&](auto mc) {
              constexpr int m = decltype(mc)::value;
              constexpr int I = 2 * m + (r & 1), J = (I + 1) % K;
              gr[r * H + m] = rot_grad<K, I, J>(v, x, cs[r][m], sn[r][m]);
            },
            std::make_index_sequence<H>{});
      },
      std::make_index_sequence<R>{});
  if (HS) {
    dd = x[1][0] * hp[1];
    x[1][0] *= d;
  }
}

// Runs f with the brick-wall round count as a compile-time constant where a
// prefetching token loop exists for it (the mixers' 3 rounds, RotationMinGRU's 1),
// else with 0 (the per-token loop that reads any number of rounds).
constexpr int AN_BRICK_TOK_RMAX = 3;
template <typename F>
__device__ __forceinline__ void brick_dispatch(int rounds, F&& f) {
  if (rounds == 3) f(std::integral_constant<int, 3>{});
  else if (rounds == 1) f(std::integral_constant<int, 1>{});
  else f(std::integral_constant<int, 0>{});
}

// ---- backward pass 1: adjoint offsets of each chunk ---------------------------
// The adjoint flowing out of chunk c to the left is y_out = P_c^T y_in + Lb_c,
// with y_in the adjoint flowing in from the right, P_c the forward chunk
// product (saved by the forward) and Lb_c this pass's zero-start reverse sweep
// x <- M_t^T (x + g_t).
template <int K, int SCHED, bool HS, bool HD, bool GP = false>
__global__ __launch_bounds__(MG_WAVE* AN_WAVES) void angle_bwd_reduce(AnArgs a, AnGeom g) {
  mg_sincos_setup();
  const AnThread th = an_thread(g);
  if (!th.ok) return;
  const int64_t t0 = (int64_t)th.c * AN_CHUNK;
  float x[K][1];
#pragma unroll
  for (int i = 0; i < K; ++i) x[i][0] = 0.f;
  const int64_t te = min(t0 + AN_CHUNK, g.T);
  if constexpr (SCHED == SCHED_LEX) {
    using Tok = LexTok<K, HS, HD>;
    token_pairs<Tok>(
        te - 1, (int)(te - t0), -1,
        [&](Tok& k, int64_t t) {
          k.template load<false>(a, a.gh, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
        },
        [&](const Tok& cur, int64_t) {
#pragma unroll
          for (int i = 0; i < K; ++i) x[i][0] += cur.v[i];
          apply_Mt_lex<K, HS, HD, 1>(x, cur.ang, cur.d, cur.gm);
        });
  } else {
    brick_dispatch(a.rounds, [&](auto rc) {
      constexpr int R = decltype(rc)::value;
      if constexpr (R > 0) {
        using Tok = BrickTok<K, R, HS, HD, false, false, false>;
        token_pairs<Tok>(
            te - 1, (int)(te - t0), -1,
            [&](Tok& k, int64_t t) {
              k.load(a, a.gh, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
            },
            [&](const Tok& cur, int64_t) {
              const float d = HS ? (GP ? mg_tanh(cur.d) : cur.d) : 1.f;
#pragma unroll
              for (int i = 0; i < K; ++i) x[i][0] += cur.v[i];
              apply_Mt_brick<K, R, HS, HD, 1>(x, cur.ang, d, cur.gm);
            });
      } else {
        for (int64_t t = te - 1; t >= t0; --t) {
          const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
          const float d = HS ? an_scale<GP>(a, lane_tok) : 1.f;
          const float gm = HD ? a.gamma[lane_tok] : 1.f;
          float gt[K];
          ld<K>(gt, a.gh + lane_tok * K);
#pragma unroll
          for (int i = 0; i < K; ++i) x[i][0] += gt[i];
          apply_Mt<K, SCHED, HS, HD, 1>(x, a.theta + lane_tok * a.na, a.rounds, d, gm);
        }
      }
    });
  }
  float xf[K];
#pragma unroll
  for (int i = 0; i < K; ++i) xf[i] = x[i][0];
  st<K>(a.lsum + an_idx(g, th.c, 0, K, th.blk), xf);
}

// The whole state from the lane's half: lo = rows 0 .. K/2 - 1, hi = the rest.
template <int H>
__device__ __forceinline__ void pair_state(const float (&own)[H], int p, float (&lo)[H],
                                           float (&hi)[H]) {
#pragma unroll
  for (int j = 0; j < H; ++j) {
    const float o = pair_swap(own[j]);
    lo[j] = p ? o : own[j];
    hi[j] = p ? own[j] : o;
  }
}

// ---- backward pass 2: adjoints at chunk boundaries, right to left --------------
// y_out = P_c^T y_in + Lb_c; two lanes per block as in the forward walk, lane p
// loading columns K/2 p .. K/2 p + K/2 - 1 of P_c (one 16-byte piece per row).
template <int K>
__global__ __launch_bounds__(AN_WALK_THREADS) void angle_bwd_scan(AnArgs a, AnGeom g) {
  constexpr int H = K / 2;
  const int64_t gt = (int64_t)blockIdx.x * AN_WALK_THREADS + threadIdx.x;
  const int64_t blk = gt >> 1;
  const int p = (int)(gt & 1);
  if (blk >= g.NB) return;  // the two lanes of a block leave together
  struct Op {
    float P[K * H];  // [j][i]: columns H p .. H p + H - 1 of P_c, row j
    float L[H];
  };
  auto fetch = [&](Op& o, int c) {
    c = max(c, 0);  // clamped reads past the start are unused
    const float* pc = a.prod + an_idx(g, c, H * p, K * K, blk);
#pragma unroll
    for (int j = 0; j < K; ++j) ld<H>(o.P + j * H, pc + j * K);
    ld<H>(o.L, a.lsum + an_idx(g, c, H * p, K, blk));
  };
  float y[H];
#pragma unroll
  for (int i = 0; i < H; ++i) y[i] = 0.f;
  // y <- P_c^T y + Lb_c, rows H p + i of the result from column H p + i of P_c.
  auto step = [&](const Op& o, Op& fill, int c) {
    fetch(fill, c - AN_WALK_AHEAD);
    st<H>(a.bound + an_idx(g, c, H * p, K, blk), y);
    float lo[H], hi[H];
    pair_state<H>(y, p, lo, hi);
#pragma unroll
    for (int i = 0; i < H; ++i) {
      float acc = o.L[i];
#pragma unroll
      for (int j = 0; j < H; ++j) acc = fmaf(o.P[j * H + i], lo[j], acc);
#pragma unroll
      for (int j = 0; j < H; ++j) acc = fmaf(o.P[(H + j) * H + i], hi[j], acc);
      y[i] = acc;
    }
  };
  const int last = g.n_chunks - 1;
  constexpr int R = AN_WALK_RING;  // ring, as in the forward walk, in reverse chunk order
  Op buf[R];
#pragma unroll
  for (int d = 0; d < R - 1; ++d) fetch(buf[d], last - d);
  int c = last;
  for (; c - (R - 1) >= 0; c -= R) {
#pragma unroll
    for (int d = 0; d < R; ++d) step(buf[d], buf[(d + R - 1) % R], c - d);
  }
#pragma unroll
  for (int d = 0; d < R - 1; ++d)
    if (c - d >= 0) step(buf[d], buf[(d + R - 1) % R], c - d);
  st<H>(a.dh0 + blk * K + H * p, y);  // the adjoint leaving chunk 0 is dL/dh0
}

// ---- two-level walk: the chunk states inside each group ------------------------
// Forward group map over chunks c0 .. c1 (applied in order): h -> Pg h + Lg.
// Backward group map over the same chunks applied from c1 down to c0:
// y -> Qg y + lg with Qg = P_c0^T ... P_c1^T = Pg^T.  The forward reduce pass
// composes Pg and Lg, angle_group_offsets the backward's lg; Pg is stored row-major
// ([group][block][K*K]) after the chunk products and read by both directions, the
// backward walk reading its columns as it reads a chunk product's.

// Chunk-entry states (forward) / adjoints (backward) of every chunk of a group
// from the group's entry value `gb` [group][block][K].  K lanes per (block,
// group), lane i owning coordinate i: all of the group's rows i of P_c (columns,
// backward) and offsets are loaded up front, and a chunk step is one partner read
// per coordinate and K multiply-adds.
template <int K, bool BWD>
__global__ __launch_bounds__(AN_WALK_THREADS) void angle_group_fill(AnArgs a, AnGeom g,
                                                                    const float* gb,
                                                                    int n_groups) {
  const int64_t gt = (int64_t)blockIdx.x * AN_WALK_THREADS + threadIdx.x;
  const int i = (int)(gt % K);
  const int64_t gbk = gt / K;
  const int64_t blk = gbk % g.NB;
  const int grp = (int)(gbk / g.NB);
  const bool ok = grp < n_groups;  // every lane stays for the partner reads
  const int lane = threadIdx.x & (MG_WAVE - 1), base = lane - i;
  const int c0 = ok ? grp * AN_GROUP : 0;
  const int c1 = ok ? min(c0 + AN_GROUP, g.n_chunks) - 1 : 0;
  const int cnt = c1 - c0 + 1;
  float P[AN_GROUP][K], L[AN_GROUP];
#pragma unroll
  for (int s = 0; s < AN_GROUP; ++s) {
    const int c = BWD ? c1 - min(s, cnt - 1) : c0 + min(s, cnt - 1);
    const float* pc = a.prod + an_idx(g, c, 0, K * K, blk);
    if (ok) {
      if (BWD) {
#pragma unroll
        for (int q = 0; q < K; ++q) P[s][q] = pc[q * K + i];
      } else {
        ld<K>(P[s], pc + i * K);
      }
      L[s] = a.lsum[an_idx(g, c, i, K, blk)];
    } else {
#pragma unroll
      for (int q = 0; q < K; ++q) P[s][q] = 0.f;
      L[s] = 0.f;
    }
  }
  float h = ok ? gb[an_idx(g, grp, i, K, blk)] : 0.f;
#pragma unroll
  for (int s = 0; s < AN_GROUP; ++s) {
    if (ok && s < cnt) a.bound[an_idx(g, BWD ? c1 - s : c0 + s, i, K, blk)] = h;
    float acc = L[s];
#pragma unroll
    for (int q = 0; q < K; ++q) acc = fmaf(P[s][q], __shfl(h, base + q), acc);
    h = acc;
  }
}

// Backward group offsets lg of the maps y -> Qg y + lg (chunks applied from c1 down
// to c0) from the chunk maps y -> P_c^T y + Lb_c: K lanes per (block, group), lane i
// owning coordinate i, with all of the group's columns i of P_c and offsets loaded up
// front; a chunk step is one partner read per coordinate and K multiply-adds.  The
// linear parts Qg = Pg^T are the forward's group maps, which the walk reads as they
// are.
template <int K>
__global__ __launch_bounds__(AN_WALK_THREADS) void angle_group_offsets(AnArgs a, AnGeom g,
                                                                       int n_groups) {
  const int64_t gt = (int64_t)blockIdx.x * AN_WALK_THREADS + threadIdx.x;
  const int i = (int)(gt % K);
  const int64_t gbk = gt / K;
  const int64_t blk = gbk % g.NB;
  const int grp = (int)(gbk / g.NB);
  const bool ok = grp < n_groups;  // every lane stays for the partner reads
  const int lane = threadIdx.x & (MG_WAVE - 1), base = lane - i;
  const int c0 = ok ? grp * AN_GROUP : 0;
  const int c1 = ok ? min(c0 + AN_GROUP, g.n_chunks) - 1 : 0;
  const int cnt = c1 - c0 + 1;
  float P[AN_GROUP][K], L[AN_GROUP];
#pragma unroll
  for (int s = 0; s < AN_GROUP; ++s) {
    const int c = c1 - min(s, cnt - 1);
    const float* pc = a.prod + an_idx(g, c, 0, K * K, blk);
    if (ok) {
#pragma unroll
      for (int q = 0; q < K; ++q) P[s][q] = pc[q * K + i];
      L[s] = a.lsum[an_idx(g, c, i, K, blk)];
    } else {
#pragma unroll
      for (int q = 0; q < K; ++q) P[s][q] = 0.f;
      L[s] = 0.f;
    }
  }
  float y = 0.f;
#pragma unroll
  for (int s = 0; s < AN_GROUP; ++s) {
    float acc = L[s];
#pragma unroll
    for (int q = 0; q < K; ++q) acc = fmaf(P[s][q], __shfl(y, base + q), acc);
    y = s < cnt ? acc : y;
  }
  if (ok) a.gsum[an_idx(g, grp, i, K, blk)] = y;
}

// Group walk and fill in one launch, for at most AN_WALKFILL_GROUPS groups: each
// team of K lanes (one per (block, group), lane i holding row i) forms its group's
// entry value itself by applying every preceding group map -- forward from h0 over
// groups 0 .. grp-1, backward from zero over groups n_groups-1 .. grp+1 -- with all
// those maps loaded at once, then fills the group's chunk-entry values as
// angle_group_fill does.  Group 0's backward team also writes dL/dh0.  The
// redundant walks cost at most AN_WALKFILL_GROUPS - 1 matrix-vector steps per team
// and save the separate group walk's launch.
template <int K, bool BWD>
__global__ __launch_bounds__(AN_WALK_THREADS) void angle_group_walk_fill(AnArgs a, AnGeom g,
                                                                         const float* gp,
                                                                         const float* gl,
                                                                         int n_groups) {
  constexpr int NP = AN_WALKFILL_GROUPS - 1;  // predecessor groups, at most
  const int64_t gt = (int64_t)blockIdx.x * AN_WALK_THREADS + threadIdx.x;
  const int i = (int)(gt % K);
  const int64_t gbk = gt / K;
  const int64_t blk = gbk % g.NB;
  const int grp = (int)(gbk / g.NB);
  const bool ok = grp < n_groups;  // every lane stays for the partner reads
  const int lane = threadIdx.x & (MG_WAVE - 1), base = lane - i;
  const int npred = ok ? (BWD ? n_groups - 1 - grp : grp) : 0;
  // Row i of each predecessor's map (backward: column i of the stored transposed
  // map) and its offset, in the order they apply.
  float GP[NP][K], GL[NP];
#pragma unroll
  for (int s = 0; s < NP; ++s) {
    const int gq = BWD ? n_groups - 1 - s : s;
    if (s < npred) {
      const float* pg = gp + an_idx(g, gq, 0, K * K, blk);
      if (BWD) {
#pragma unroll
        for (int q = 0; q < K; ++q) GP[s][q] = pg[q * K + i];
      } else {
        ld<K>(GP[s], pg + i * K);
      }
      GL[s] = gl[an_idx(g, gq, i, K, blk)];
    } else {
#pragma unroll
      for (int q = 0; q < K; ++q) GP[s][q] = 0.f;
      GL[s] = 0.f;
    }
  }
  const int c0 = ok ? grp * AN_GROUP : 0;
  const int c1 = ok ? min(c0 + AN_GROUP, g.n_chunks) - 1 : 0;
  const int cnt = c1 - c0 + 1;
  float P[AN_GROUP][K], L[AN_GROUP];
#pragma unroll
  for (int s = 0; s < AN_GROUP; ++s) {
    const int c = BWD ? c1 - min(s, cnt - 1) : c0 + min(s, cnt - 1);
    const float* pc = a.prod + an_idx(g, c, 0, K * K, blk);
    if (ok) {
      if (BWD) {
#pragma unroll
        for (int q = 0; q < K; ++q) P[s][q] = pc[q * K + i];
      } else {
        ld<K>(P[s], pc + i * K);
      }
      L[s] = a.lsum[an_idx(g, c, i, K, blk)];
    } else {
#pragma unroll
      for (int q = 0; q < K; ++q) P[s][q] = 0.f;
      L[s] = 0.f;
    }
  }
  float h = (ok && !BWD) ? a.h0[blk * K + i] : 0.f;
#pragma unroll
  for (int s = 0; s < NP; ++s) {
    if (s < npred) {  // uniform across the team
      float acc = GL[s];
#pragma unroll
      for (int q = 0; q < K; ++q) acc = fmaf(GP[s][q], __shfl(h, base + q), acc);
      h = acc;
    }
  }
#pragma unroll
  for (int s = 0; s < AN_GROUP; ++s) {
    if (ok && s < cnt) a.bound[an_idx(g, BWD ? c1 - s : c0 + s, i, K, blk)] = h;
    float acc = L[s];
#pragma unroll
    for (int q = 0; q < K; ++q) acc = fmaf(P[s][q], __shfl(h, base + q), acc);
    h = acc;
  }
  if (BWD && ok && grp == 0) a.dh0[blk * K + i] = h;  // the adjoint leaving chunk 0
}

// ---- backward pass 3: every token's gradients from its chunk-entry adjoint ------
template <int K, int SCHED, bool HS, bool HD, bool GP = false>
__global__ __launch_bounds__(MG_WAVE* AN_WAVES) void angle_bwd_final(AnArgs a, AnGeom g) {
  mg_sincos_setup();
  const AnThread th = an_thread(g);
  if (!th.ok) return;
  const int64_t t0 = (int64_t)th.c * AN_CHUNK;
  float y[K][1];
  {
    float b0[K];
    ld<K>(b0, a.bound + an_idx(g, th.c, 0, K, th.blk));
#pragma unroll
    for (int i = 0; i < K; ++i) y[i][0] = b0[i];
  }
  const int64_t te = min(t0 + AN_CHUNK, g.T);
  if constexpr (SCHED == SCHED_LEX) {
    using Tok = LexTok<K, HS, HD>;
    constexpr int R = K * (K - 1) / 2;
    // With every lane of the wave active, the lanes' dtheta rows of one token are
    // consecutive and leave through LDS as whole lines (C4: backward 144 -> 132 us).
    constexpr bool ROWS = R % 4 == 0;
    __shared__ __attribute__((aligned(16))) float s_rows[ROWS ? AN_WAVES : 1][MG_WAVE * R];
    const int lane = threadIdx.x & (MG_WAVE - 1);
    const bool whole = ROWS && __builtin_amdgcn_read_exec() == ~0ull;
    float* rows = s_rows[ROWS ? threadIdx.x / MG_WAVE : 0];
    token_pairs<Tok>(
        te - 1, (int)(te - t0), -1,
        [&](Tok& k, int64_t t) {
          k.template load<true>(a, a.gh, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
        },
        [&](const Tok& cur, int64_t t) {
          const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
          float gt[K];
#pragma unroll
          for (int i = 0; i < K; ++i) {
            y[i][0] += cur.v[i];
            gt[i] = y[i][0];
          }
          st<K>(a.out + lane_tok * K, gt);  // db_t = dL/dh_t
          float dd = 0.f, dg = 0.f, gr[R];
          token_grad_lex<K, HS, HD>(y, cur.hp, cur.ang, gr, cur.d, cur.gm, dd, dg);
          if constexpr (ROWS) {
            if (whole) wave_rows_store<R>(a.dtheta + (lane_tok - lane) * R, gr, rows, lane);
            else st<R>(a.dtheta + lane_tok * R, gr);
          } else {
            st<R>(a.dtheta + lane_tok * R, gr);  // partial-line rows: the L2 merges them
          }
          if (HS) a.dscale[lane_tok] = dd;
          if (HD) a.dgamma[lane_tok] = dg;
        });
  } else {
    // dtheta rows of the prefetching form (R K/2 floats per lane) leave through LDS as
    // whole lines when they are whole 16-byte pieces and the wave is complete.
    constexpr int BR = AN_BRICK_TOK_RMAX * (K / 2);
    __shared__ __attribute__((aligned(16))) float s_brows[AN_WAVES][MG_WAVE * BR];
    const int lane = threadIdx.x & (MG_WAVE - 1);
    const bool whole = __builtin_amdgcn_read_exec() == ~0ull;
    float* rows = s_brows[threadIdx.x / MG_WAVE];
    brick_dispatch(a.rounds, [&](auto rc) {
      constexpr int R = decltype(rc)::value;
      if constexpr (R > 0) {
        constexpr int NA = R * (K / 2);
        using Tok = BrickTok<K, R, HS, HD, GP, GP, true>;
        token_pairs<Tok>(
            te - 1, (int)(te - t0), -1,
            [&](Tok& k, int64_t t) {
              k.load(a, a.gh, (th.bb * g.T + t) * g.n + th.plane, t, g.n, th.blk);
            },
            [&](const Tok& cur, int64_t t) {
              const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
              const float d = HS ? (GP ? mg_tanh(cur.d) : cur.d) : 1.f;
              float gt[K];
#pragma unroll
              for (int i = 0; i < K; ++i) {
                y[i][0] += cur.v[i];
                gt[i] = y[i][0];
              }
              an_store_db_reg<K, GP>(a, lane_tok, gt, cur.zb, cur.hq);  // db_t (or dz, dhpre)
              float dd = 0.f, dg = 0.f, gr[NA];
              token_grad_brick<K, R, HS, HD>(y, cur.hp, cur.ang, gr, d, cur.gm, dd, dg);
              if constexpr (NA % 4 == 0) {
                if (whole) wave_rows_store<NA>(a.dtheta + (lane_tok - lane) * NA, gr, rows, lane);
                else st<NA>(a.dtheta + lane_tok * NA, gr);
              } else {
                st<NA>(a.dtheta + lane_tok * NA, gr);  // partial-line rows: the L2 merges them
              }
              if (HS) a.dscale[lane_tok] = GP ? dd * (1.f - d * d) : dd;  // GP: dL/du, d = tanh(u)
              if (HD) a.dgamma[lane_tok] = dg;
            });
      } else {
        for (int64_t t = te - 1; t >= t0; --t) {
          const int64_t lane_tok = (th.bb * g.T + t) * g.n + th.plane;
          const float d = HS ? an_scale<GP>(a, lane_tok) : 1.f;
          const float gm = HD ? a.gamma[lane_tok] : 1.f;
          float gt[K], hp[K];
          ld<K>(gt, a.gh + lane_tok * K);
          if (t > 0) ld<K>(hp, a.h + lane_tok * K - g.n * K);
          else ld<K>(hp, a.h0 + th.blk * K);
#pragma unroll
          for (int i = 0; i < K; ++i) {
            y[i][0] += gt[i];
            gt[i] = y[i][0];
          }
          an_store_db<K, GP>(a, lane_tok, gt);  // db_t = dL/dh_t (or dz, dhpre)
          float dd = 0.f, dg = 0.f;
          token_grad<K, SCHED, HS, HD>(y, hp, a.theta + lane_tok * a.na,
                                       a.dtheta + lane_tok * a.na, a.rounds, d, gm, dd, dg);
          if (HS) a.dscale[lane_tok] = GP ? dd * (1.f - d * d) : dd;  // GP: dL/du, d = tanh(u)
          if (HD) a.dgamma[lane_tok] = dg;
        }
      }
    });
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

AnGeom an_geom(int64_t B, int64_t T, int64_t n) {
  AnGeom g;
  g.T = T;
  g.n = n;
  g.NB = B * n;
  g.n_tiles = (int)((n + MG_WAVE - 1) / MG_WAVE);
  g.n_lg = (int)(B * g.n_tiles);
  g.n_chunks = (int)((T + AN_CHUNK - 1) / AN_CHUNK);
  g.n_run = (int)((g.NB + AN_RUN - 1) / AN_RUN);
  g.n_groups = (g.n_chunks + AN_GROUP - 1) / AN_GROUP;
  return g;
}

bool an_two_level(const AnGeom& g) { return g.n_chunks > AN_GROUP_MIN; }

// Workspace: header, chunk offsets and chunk-entry values ([chunk][block][k] each),
// then the two-level walk's group offsets and group-entry values ([group][block][k]
// each).
size_t an_ws_bytes(int64_t B, int64_t T, int64_t n, int k) {
  const AnGeom g = an_geom(B, T, n);
  const size_t one = mg_align_up((size_t)g.n_chunks * k * g.NB * sizeof(float), 256);
  const size_t gv = mg_align_up((size_t)g.n_groups * k * g.NB * sizeof(float), 256);
  return MG_HEADER_BYTES + 2 * one + 2 * gv;
}

// Saved by the forward for the backward: the chunk products, K*K floats per
// (chunk, block), and with the two-level walk the group maps, K*K floats per
// (group, block).
size_t an_state_bytes(int64_t B, int64_t T, int64_t n, int k) {
  const AnGeom g = an_geom(B, T, n);
  const int64_t maps = g.n_chunks + (an_two_level(g) ? g.n_groups : 0);
  return (size_t)maps * k * k * g.NB * sizeof(float);
}

template <int K, int SCHED, bool HS, bool HD, bool BWD, bool GP = false>
int an_launch(AnArgs a, int64_t B, int64_t T, int64_t n, void* ws, size_t ws_bytes,
              hipStream_t stream) {
  const AnGeom g = an_geom(B, T, n);
  if (ws_bytes < an_ws_bytes(B, T, n, K)) return MG_ERR_WORKSPACE;
  const size_t one = mg_align_up((size_t)g.n_chunks * K * g.NB * sizeof(float), 256);
  a.lsum = (float*)((char*)ws + MG_HEADER_BYTES);
  a.bound = (float*)((char*)ws + MG_HEADER_BYTES + one);
  const int ng = g.n_groups;
  const size_t gv = mg_align_up((size_t)ng * K * g.NB * sizeof(float), 256);
  a.gsum = (float*)((char*)ws + MG_HEADER_BYTES + 2 * one);
  float* gb = (float*)((char*)ws + MG_HEADER_BYTES + 2 * one + gv);
  a.gprod = a.prod + (size_t)g.n_chunks * K * K * g.NB;  // after the chunk products
  const int64_t waves = (int64_t)g.n_lg * g.n_chunks;
  const dim3 grid((unsigned)((waves + AN_WAVES - 1) / AN_WAVES)), block(MG_WAVE * AN_WAVES);
  const dim3 rgrid((unsigned)((int64_t)g.n_run * ng));
  const dim3 sgrid((unsigned)((g.NB * 2 + AN_WALK_THREADS - 1) / AN_WALK_THREADS)),
      sblock(AN_WALK_THREADS);
  // Boundary walk: direct over the chunks, or over the groups of AN_GROUP chunks
  // whose maps the reduce pass composed.
  auto walk = [&]() {
    if (!an_two_level(g)) {
      if (BWD) hipLaunchKernelGGL((angle_bwd_scan<K>), sgrid, sblock, 0, stream, a, g);
      else hipLaunchKernelGGL((angle_fwd_scan<K>), sgrid, sblock, 0, stream, a, g);
      return;
    }
    const float* gp = a.gprod;
    const float* gl = a.gsum;
    const dim3 cgrid((unsigned)((g.NB * ng * K + AN_WALK_THREADS - 1) / AN_WALK_THREADS));
    if (BWD) hipLaunchKernelGGL((angle_group_offsets<K>), cgrid, sblock, 0, stream, a, g, ng);
    if (ng <= AN_WALKFILL_GROUPS) {
      hipLaunchKernelGGL((angle_group_walk_fill<K, BWD>), cgrid, sblock, 0, stream, a, g, gp, gl,
                         ng);
      return;
    }
    // The walk kernels over the group maps: chunks -> groups.
    AnArgs ag = a;
    AnGeom gg = g;
    ag.prod = a.gprod;
    ag.lsum = a.gsum;
    ag.bound = gb;
    gg.n_chunks = ng;
    if (BWD) hipLaunchKernelGGL((angle_bwd_scan<K>), sgrid, sblock, 0, stream, ag, gg);
    else hipLaunchKernelGGL((angle_fwd_scan<K>), sgrid, sblock, 0, stream, ag, gg);
    hipLaunchKernelGGL((angle_group_fill<K, BWD>), cgrid, sblock, 0, stream, a, g,
                       (const float*)gb, ng);
  };
  if (BWD) {
    hipLaunchKernelGGL((angle_bwd_reduce<K, SCHED, HS, HD, GP>), grid, block, 0, stream, a, g);
    walk();
    hipLaunchKernelGGL((angle_bwd_final<K, SCHED, HS, HD, GP>), grid, block, 0, stream, a, g);
  } else {
    hipLaunchKernelGGL((angle_fwd_reduce<K, SCHED, HS, HD, GP>), rgrid, dim3(AN_RED_THREADS), 0, stream,
                       a, g);
    walk();
    hipLaunchKernelGGL((angle_fwd_final<K, SCHED, HS, HD, GP>), grid, block, 0, stream, a, g);
  }
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

template <bool BWD>
int an_dispatch(const AnArgs& a, int64_t B, int64_t T, int64_t n, int k, int sched, int flags,
                void* ws, size_t ws_bytes, hipStream_t stream) {
  const bool hs = flags & 1, hd = flags & 2;
  if (flags & AN_FLAG_GATED) {  // the gated prologue: brick-wall schedules only
#define MG_AN_GCASE(KK)                                                                         \
  if (k == KK && sched == SCHED_BRICK) {                                                        \
    if (hs && hd)                                                                               \
      return an_launch<KK, SCHED_BRICK, true, true, BWD, true>(a, B, T, n, ws, ws_bytes, stream); \
    if (hs)                                                                                     \
      return an_launch<KK, SCHED_BRICK, true, false, BWD, true>(a, B, T, n, ws, ws_bytes,        \
                                                                stream);                        \
    if (hd)                                                                                     \
      return an_launch<KK, SCHED_BRICK, false, true, BWD, true>(a, B, T, n, ws, ws_bytes,        \
                                                                stream);                        \
    return an_launch<KK, SCHED_BRICK, false, false, BWD, true>(a, B, T, n, ws, ws_bytes, stream); \
  }
    MG_AN_GCASE(2)
    MG_AN_GCASE(4)
    MG_AN_GCASE(8)
#undef MG_AN_GCASE
    return MG_ERR_ARG;
  }
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
  const AnGeom g = an_geom(B, T, n);
  return (int64_t)g.n_lg * g.n_chunks < (1ll << 31) - AN_WAVES &&
         (int64_t)g.n_run * g.n_groups < (1ll << 31) && g.NB * 8 < (1ll << 31);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

size_t mg_angle_scan_workspace_bytes(int64_t B, int64_t T, int64_t n, int k) {
  if (B <= 0 || T <= 0 || n <= 0 || k <= 0 || k > 8) return 256;
  return an_ws_bytes(B, T, n, k);
}

size_t mg_angle_scan_state_bytes(int64_t B, int64_t T, int64_t n, int k) {
  if (B <= 0 || T <= 0 || n <= 0 || k <= 0 || k > 8) return 0;
  return an_state_bytes(B, T, n, k);
}

int mg_angle_scan_fwd(const float* theta, const float* scale, const float* gamma, const float* b,
                      const float* h0, float* h, float* chunk_prod, int64_t B, int64_t T,
                      int64_t n, int k, int sched, int rounds, int flags, void* ws,
                      size_t ws_bytes, hipStream_t stream) {
  if (!theta || !b || !h0 || !h || !chunk_prod || !ws || (flags & ~3) ||
      !an_args_ok(B, T, n, k, sched, rounds) || !an_geometry_ok(B, T, n))
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
  a.prod = chunk_prod;
  a.rounds = rounds;
  a.na = sched == SCHED_LEX ? k * (k - 1) / 2 : rounds * (k / 2);
  return an_dispatch<false>(a, B, T, n, k, sched, flags, ws, ws_bytes, stream);
}

int mg_angle_scan_bwd(const float* theta, const float* scale, const float* gamma, const float* h0,
                      const float* h, const float* chunk_prod, const float* gh, float* dtheta,
                      float* dscale, float* dgamma, float* db, float* dh0, int64_t B, int64_t T,
                      int64_t n, int k, int sched, int rounds, int flags, void* ws,
                      size_t ws_bytes, hipStream_t stream) {
  if (!theta || !h0 || !h || !chunk_prod || !gh || !dtheta || !db || !dh0 || !ws ||
      (flags & ~3) || !an_args_ok(B, T, n, k, sched, rounds) || !an_geometry_ok(B, T, n))
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
  a.prod = const_cast<float*>(chunk_prod);
  a.rounds = rounds;
  a.na = sched == SCHED_LEX ? k * (k - 1) / 2 : rounds * (k / 2);
  return an_dispatch<true>(a, B, T, n, k, sched, flags, ws, ws_bytes, stream);
}

int mg_angle_scan_gated_fwd(const float* theta, const float* u, const float* gamma,
                            const float* z, const float* hpre, const float* h0, float* h,
                            float* chunk_prod, int64_t B, int64_t T, int64_t n, int k, int rounds,
                            int flags, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!theta || !z || !hpre || !h0 || !h || !chunk_prod || !ws || (flags & ~3) ||
      !an_args_ok(B, T, n, k, SCHED_BRICK, rounds) || !an_geometry_ok(B, T, n))
    return MG_ERR_ARG;
  if (((flags & 1) && !u) || ((flags & 2) && !gamma)) return MG_ERR_ARG;
  if (!aligned16(theta) || !aligned16(z) || !aligned16(hpre) || !aligned16(h0) || !aligned16(h))
    return MG_ERR_ARG;
  AnArgs a{};
  a.theta = theta;
  a.scale = u;
  a.gamma = gamma;
  a.b = z;
  a.hpre = hpre;
  a.h0 = h0;
  a.out = h;
  a.prod = chunk_prod;
  a.rounds = rounds;
  a.na = rounds * (k / 2);
  return an_dispatch<false>(a, B, T, n, k, SCHED_BRICK, flags | AN_FLAG_GATED, ws, ws_bytes,
                            stream);
}

int mg_angle_scan_gated_bwd(const float* theta, const float* u, const float* gamma,
                            const float* z, const float* hpre, const float* h0, const float* h,
                            const float* chunk_prod, const float* gh, float* dtheta, float* du,
                            float* dgamma, float* dz, float* dhpre, float* dh0, int64_t B,
                            int64_t T, int64_t n, int k, int rounds, int flags, void* ws,
                            size_t ws_bytes, hipStream_t stream) {
  if (!theta || !z || !hpre || !h0 || !h || !chunk_prod || !gh || !dtheta || !dz || !dhpre ||
      !dh0 || !ws || (flags & ~3) || !an_args_ok(B, T, n, k, SCHED_BRICK, rounds) ||
      !an_geometry_ok(B, T, n))
    return MG_ERR_ARG;
  if (((flags & 1) && (!u || !du)) || ((flags & 2) && (!gamma || !dgamma))) return MG_ERR_ARG;
  if (!aligned16(theta) || !aligned16(z) || !aligned16(hpre) || !aligned16(h0) ||
      !aligned16(h) || !aligned16(gh) || !aligned16(dtheta) || !aligned16(dz) ||
      !aligned16(dhpre) || !aligned16(dh0))
    return MG_ERR_ARG;
  AnArgs a{};
  a.theta = theta;
  a.scale = u;
  a.gamma = gamma;
  a.b = z;
  a.hpre = hpre;
  a.h0 = h0;
  a.h = h;
  a.gh = gh;
  a.out = dz;
  a.dhpre = dhpre;
  a.dtheta = dtheta;
  a.dscale = du;
  a.dgamma = dgamma;
  a.dh0 = dh0;
  a.prod = const_cast<float*>(chunk_prod);
  a.rounds = rounds;
  a.na = rounds * (k / 2);
  return an_dispatch<true>(a, B, T, n, k, SCHED_BRICK, flags | AN_FLAG_GATED, ws, ws_bytes,
                           stream);
}

}  // extern "C"

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
// involution, partners sharing one angle that no other plane of the round uses,
// opposite unit signs), so every round is orthogonal and its inverse is its
// transpose.
//
// This is the general path: k in {2, 4, 8, 16}, any such tables, up to
// AT_MAX_ROUNDS rounds.  The compiled-schedule kernels in scan_angle.hip cover
// the brick-wall and lexicographic schedules of k <= 8.
//
// Work layout: k consecutive lanes per block, lane p owning coordinate p, so a
// round reads the partner coordinate with one ds_bpermute and h, b and the
// gradients move as contiguous rows.  The tables sit in LDS, one packed word
// per (round, coordinate).  Time is split into AT_CHUNK-token chunks, scanned
// reduce-then-scan like the compiled kernels (no workgroup waits on another):
//   forward  1. per (block, chunk): lane p pushes row p of the chunk map
//               [P_c | L_c] through the chunk's rounds (k + 1 partner reads
//               per round);
//            2. per block: walk the chunk boundaries, h <- P_c h + L_c;
//            3. per (block, chunk): re-apply the rounds from the chunk-entry
//               state and write every h_t.
//   backward 1. per (block, chunk): the zero-start reverse sweep of the adjoint,
//               Lb_c (the linear part is P_c^T, saved by the forward);
//            2. per block: walk y <- P_c^T y + Lb_c from the end, writing dh0;
//            3. per (block, chunk): from the adjoint entering each chunk,
//               recompute each token's rounds from h_{t-1} (read from the
//               forward output), sweep them backwards recovering each round's
//               input by the transposed rotation, and write dtheta, dscale,
//               dgamma and db.
#include "mg_common.h"
#include "mg_sincos.h"

#include <algorithm>

namespace {

using mg::mg_sincos;
using mg::mg_sincos_setup;

constexpr int AT_THREADS = 256;
constexpr int AT_CHUNK = 16;        // tokens per chunk
constexpr int AT_MAX_HALF = 64;     // angles per round
constexpr int AT_MAX_ROUNDS = 128;  // rounds held in LDS

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
  float* prod;   // chunk products [chunk][block][k][k]: forward writes, backward reads
  float* lsum;   // chunk offsets [chunk][block][k]
  float* bound;  // chunk-entry states / adjoints [chunk][block][k]
  int64_t B, T, n, NB;
  int k, R, half, n_chunks;
  int has_scale, has_decay;
};

// Packed table word of (round, coordinate): partner | angle << 8 | negative << 16 | active << 17.
__device__ __forceinline__ void at_load_tables(const AtArgs& a, int* s_tab) {
  for (int i = threadIdx.x; i < a.R * a.k; i += blockDim.x) {
    const int p = i % a.k;
    const int pp = min(max(a.perm[i], 0), a.k - 1);
    const int an = min(max(a.p2p[i], 0), a.half - 1);
    s_tab[i] = pp | (an << 8) | ((a.sgn[i] < 0.f ? 1 : 0) << 16) | ((pp != p ? 1 : 0) << 17);
  }
  mg_sincos_setup();  // ends in the barrier that also publishes s_tab
}

struct AtRound {
  int partner;  // lane of the partner coordinate
  int ang;      // angle index within the round
  float sg;     // sign of this coordinate (+1 / -1)
  bool act;     // false when the partner is the coordinate itself
};

__device__ __forceinline__ AtRound at_round(const int* s_tab, int k, int r, int p, int base) {
  const int w = s_tab[r * k + p];
  AtRound q;
  q.partner = base + (w & 0xff);
  q.ang = (w >> 8) & 0xff;
  q.sg = (w >> 16) & 1 ? -1.f : 1.f;
  q.act = (w >> 17) & 1;
  return q;
}

// A lane of the chunk passes: coordinate p of block blk in chunk c.
struct AtLane {
  int64_t blk, bb, plane;
  int c, p, lane, base;
  bool ok;
};

__device__ __forceinline__ AtLane at_chunk_lane(const AtArgs& a) {
  AtLane L;
  const int64_t gid = (int64_t)blockIdx.x * AT_THREADS + threadIdx.x;
  L.lane = threadIdx.x & (MG_WAVE - 1);
  L.p = (int)(gid % a.k);
  L.base = L.lane - L.p;
  const int64_t cb = gid / a.k;  // chunk * NB + block
  L.ok = cb < (int64_t)a.n_chunks * a.NB;
  const int64_t cbs = L.ok ? cb : 0;
  L.c = (int)(cbs / a.NB);
  L.blk = cbs - (int64_t)L.c * a.NB;
  L.bb = L.blk / a.n;
  L.plane = L.blk - L.bb * a.n;
  return L;
}

// A lane of the boundary walks: coordinate p of block blk.
__device__ __forceinline__ AtLane at_walk_lane(const AtArgs& a) {
  AtLane L;
  const int64_t gid = (int64_t)blockIdx.x * AT_THREADS + threadIdx.x;
  L.lane = threadIdx.x & (MG_WAVE - 1);
  L.p = (int)(gid % a.k);
  L.base = L.lane - L.p;
  L.ok = gid / a.k < a.NB;
  L.blk = L.ok ? gid / a.k : 0;
  L.bb = L.blk / a.n;
  L.plane = L.blk - L.bb * a.n;
  L.c = 0;
  return L;
}

__device__ __forceinline__ int64_t at_tok(const AtArgs& a, const AtLane& L, int64_t t) {
  return (L.bb * a.T + t) * a.n + L.plane;
}
__device__ __forceinline__ int64_t at_cidx(const AtArgs& a, int c, int64_t blk) {
  return (int64_t)c * a.NB + blk;
}

// v <- rounds of token tk (forward direction) applied to coordinate p's value.
__device__ __forceinline__ float at_rounds_fwd(const AtArgs& a, const int* s_tab,
                                               const AtLane& L, int64_t tk, float v) {
  for (int r = 0; r < a.R; ++r) {
    const AtRound q = at_round(s_tab, a.k, r, L.p, L.base);
    float s = 0.f, c = 1.f;
    if (L.ok) mg_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
    const float vp = at_shfl(v, q.partner);
    if (q.act) v = fmaf(c, v, q.sg * s * vp);
  }
  return v;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(AT_THREADS) void angle_tables_fwd_reduce(AtArgs a) {
  __shared__ int s_tab[AT_MAX_ROUNDS * 16];
  at_load_tables(a, s_tab);
  const AtLane L = at_chunk_lane(a);
  // Row p of [P | L]: X[j] = P[p][j], X[K] = L[p].
  float X[K + 1];
#pragma unroll
  for (int j = 0; j <= K; ++j) X[j] = (j == L.p) ? 1.f : 0.f;
  const int64_t t0 = (int64_t)L.c * AT_CHUNK;
  const int64_t te = min(t0 + AT_CHUNK, a.T);
  float gprod = 1.f;
  for (int64_t t = t0; t < te; ++t) {
    const int64_t tk = at_tok(a, L, t);
    if (a.has_scale && L.p == 1 && L.ok) {
      const float d = a.scale[tk];
#pragma unroll
      for (int j = 0; j <= K; ++j) X[j] *= d;
    }
    for (int r = 0; r < a.R; ++r) {
      const AtRound q = at_round(s_tab, K, r, L.p, L.base);
      float s = 0.f, c = 1.f;
      if (L.ok) mg_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
      const float cs = q.sg * s;
#pragma unroll
      for (int j = 0; j <= K; ++j) {
        const float xp = at_shfl(X[j], q.partner);
        if (q.act) X[j] = fmaf(c, X[j], cs * xp);
      }
    }
    // The decay is a scalar per token: P takes the chunk's product of decays once at
    // the end, the offset column (which receives b_t every token) per token.
    const float gm = (a.has_decay && L.ok) ? a.gamma[tk] : 1.f;
    gprod *= gm;
    X[K] = fmaf(gm, X[K], L.ok ? a.b[tk * K + L.p] : 0.f);
  }
  if (!L.ok) return;
  float* pr = a.prod + (at_cidx(a, L.c, L.blk) * K + L.p) * K;
#pragma unroll
  for (int j = 0; j < K; j += 2)
    *reinterpret_cast<float2*>(pr + j) = make_float2(X[j] * gprod, X[j + 1] * gprod);
  a.lsum[at_cidx(a, L.c, L.blk) * K + L.p] = X[K];
}

// h_{c+1} = P_c h_c + L_c over the chunks of each block; bound[c] = h_c.
template <int K>
__global__ __launch_bounds__(AT_THREADS) void angle_tables_fwd_walk(AtArgs a) {
  const AtLane L = at_walk_lane(a);
  float h = L.ok ? a.h0[L.blk * K + L.p] : 0.f;
  float P[K], Pn[K], l = 0.f, ln = 0.f;
  auto fetch = [&](float (&dst)[K], float& dl, int c) {
    c = min(c, a.n_chunks - 1);
    if (L.ok) {
      const float* pr = a.prod + (at_cidx(a, c, L.blk) * K + L.p) * K;
#pragma unroll
      for (int j = 0; j < K; j += 2) {
        const float2 v = *reinterpret_cast<const float2*>(pr + j);
        dst[j] = v.x;
        dst[j + 1] = v.y;
      }
      dl = a.lsum[at_cidx(a, c, L.blk) * K + L.p];
    } else {
#pragma unroll
      for (int j = 0; j < K; ++j) dst[j] = 0.f;
      dl = 0.f;
    }
  };
  fetch(P, l, 0);
  for (int c = 0; c < a.n_chunks; ++c) {
    fetch(Pn, ln, c + 1);
    if (L.ok) a.bound[at_cidx(a, c, L.blk) * K + L.p] = h;
    float acc = l;
#pragma unroll
    for (int j = 0; j < K; ++j) acc = fmaf(P[j], at_shfl(h, L.base + j), acc);
    h = acc;
#pragma unroll
    for (int j = 0; j < K; ++j) P[j] = Pn[j];
    l = ln;
  }
}

template <int K>
__global__ __launch_bounds__(AT_THREADS) void angle_tables_fwd_final(AtArgs a) {
  __shared__ int s_tab[AT_MAX_ROUNDS * 16];
  at_load_tables(a, s_tab);
  const AtLane L = at_chunk_lane(a);
  float v = L.ok ? a.bound[at_cidx(a, L.c, L.blk) * K + L.p] : 0.f;
  const int64_t t0 = (int64_t)L.c * AT_CHUNK;
  const int64_t te = min(t0 + AT_CHUNK, a.T);
  for (int64_t t = t0; t < te; ++t) {
    const int64_t tk = at_tok(a, L, t);
    if (a.has_scale && L.p == 1 && L.ok) v *= a.scale[tk];
    v = at_rounds_fwd(a, s_tab, L, tk, v);
    if (L.ok) {
      if (a.has_decay) v *= a.gamma[tk];
      v += a.b[tk * K + L.p];
      a.out[tk * K + L.p] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
// y <- M_t^T (g_t + y) over the chunk from its end, from y = 0: Lb_c.
template <int K>
__global__ __launch_bounds__(AT_THREADS) void angle_tables_bwd_reduce(AtArgs a) {
  __shared__ int s_tab[AT_MAX_ROUNDS * 16];
  at_load_tables(a, s_tab);
  const AtLane L = at_chunk_lane(a);
  const int64_t t0 = (int64_t)L.c * AT_CHUNK;
  const int64_t te = min(t0 + AT_CHUNK, a.T);
  float y = 0.f;
  for (int64_t t = te - 1; t >= t0; --t) {
    const int64_t tk = at_tok(a, L, t);
    y += L.ok ? a.gh[tk * K + L.p] : 0.f;
    if (a.has_decay && L.ok) y *= a.gamma[tk];
    for (int r = a.R - 1; r >= 0; --r) {
      const AtRound q = at_round(s_tab, K, r, L.p, L.base);
      float s = 0.f, c = 1.f;
      if (L.ok) mg_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
      const float yp = at_shfl(y, q.partner);
      if (q.act) y = fmaf(c, y, -q.sg * s * yp);
    }
    if (a.has_scale && L.p == 1 && L.ok) y *= a.scale[tk];
  }
  if (L.ok) a.lsum[at_cidx(a, L.c, L.blk) * K + L.p] = y;
}

// From the end: bound[c] = adjoint entering chunk c from the right,
// y <- P_c^T y + Lb_c; the adjoint leaving chunk 0 is dh0.
template <int K>
__global__ __launch_bounds__(AT_THREADS) void angle_tables_bwd_walk(AtArgs a) {
  const AtLane L = at_walk_lane(a);
  float y = 0.f;
  float P[K], Pn[K], l = 0.f, ln = 0.f;  // column p of P_c
  auto fetch = [&](float (&dst)[K], float& dl, int c) {
    c = max(c, 0);
    if (L.ok) {
      const float* pc = a.prod + at_cidx(a, c, L.blk) * K * K + L.p;
#pragma unroll
      for (int j = 0; j < K; ++j) dst[j] = pc[j * K];
      dl = a.lsum[at_cidx(a, c, L.blk) * K + L.p];
    } else {
#pragma unroll
      for (int j = 0; j < K; ++j) dst[j] = 0.f;
      dl = 0.f;
    }
  };
  fetch(P, l, a.n_chunks - 1);
  for (int c = a.n_chunks - 1; c >= 0; --c) {
    fetch(Pn, ln, c - 1);
    if (L.ok) a.bound[at_cidx(a, c, L.blk) * K + L.p] = y;
    float acc = l;
#pragma unroll
    for (int j = 0; j < K; ++j) acc = fmaf(P[j], at_shfl(y, L.base + j), acc);
    y = acc;
#pragma unroll
    for (int j = 0; j < K; ++j) P[j] = Pn[j];
    l = ln;
  }
  if (L.ok) a.dh0[L.blk * K + L.p] = y;
}

template <int K>
__global__ __launch_bounds__(AT_THREADS) void angle_tables_bwd_final(AtArgs a) {
  __shared__ int s_tab[AT_MAX_ROUNDS * 16];
  at_load_tables(a, s_tab);
  const AtLane L = at_chunk_lane(a);
  const int64_t t0 = (int64_t)L.c * AT_CHUNK;
  const int64_t te = min(t0 + AT_CHUNK, a.T);
  float y = L.ok ? a.bound[at_cidx(a, L.c, L.blk) * K + L.p] : 0.f;  // adjoint from t+1
  for (int64_t t = te - 1; t >= t0; --t) {
    const int64_t tk = at_tok(a, L, t);
    const float x = y + (L.ok ? a.gh[tk * K + L.p] : 0.f);  // dL/dh_t in total
    float hp = 0.f, d = 1.f, gm = 1.f;
    if (L.ok) {
      hp = t > 0 ? a.h[(tk - a.n) * K + L.p] : a.h0[L.blk * K + L.p];
      if (a.has_scale) d = a.scale[tk];
      if (a.has_decay) gm = a.gamma[tk];
      a.out[tk * K + L.p] = x;  // db
    }
    // Forward through the token's rounds: u_R.
    float u = (a.has_scale && L.p == 1) ? hp * d : hp;
    u = at_rounds_fwd(a, s_tab, L, tk, u);
    // dgamma = <x, u_R> over the block's K lanes (aligned groups of K lanes).
    if (a.has_decay) {
      float dg = x * u;
#pragma unroll
      for (int off = K >> 1; off > 0; off >>= 1) dg += at_shfl(dg, L.lane ^ off);
      if (L.ok && L.p == 0) a.dgamma[tk] = dg;
    }
    float adj = gm * x;  // adjoint on u_R
    for (int r = a.R - 1; r >= 0; --r) {
      const AtRound q = at_round(s_tab, K, r, L.p, L.base);
      float s = 0.f, c = 1.f;
      if (L.ok) mg_sincos(a.theta[(tk * a.R + r) * a.half + q.ang], s, c);
      // u holds u_r (after the rotation); recover u_{r-1} by the transposed rotation.
      const float up = at_shfl(u, q.partner);
      const float u_prev = q.act ? fmaf(c, u, -q.sg * s * up) : u;
      const float u_prev_p = at_shfl(u_prev, q.partner);
      const float ap = at_shfl(adj, q.partner);
      // d u_r[p] / d theta = -s u[p] + sgn c u[partner]  (u = u_{r-1})
      const float e = q.act ? adj * fmaf(-s, u_prev, q.sg * c * u_prev_p) : 0.f;
      const float e_pair = e + at_shfl(e, q.partner);
      // The plane's first member (negative sign) writes the angle's gradient; the
      // host checked that no other plane of the round shares the angle.
      if (L.ok && q.act && q.sg < 0.f) a.dtheta[(tk * a.R + r) * a.half + q.ang] = e_pair;
      if (q.act) adj = fmaf(c, adj, -q.sg * s * ap);  // adjoint on u_{r-1}
      u = u_prev;
    }
    // adj is the adjoint on u_0 = S h_{t-1}.
    if (a.has_scale && L.p == 1) {
      if (L.ok) a.dscale[tk] = adj * hp;
      adj *= d;
    }
    y = adj;
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
int at_chunks(int64_t T) { return (int)((T + AT_CHUNK - 1) / AT_CHUNK); }

bool at_args_ok(int64_t B, int64_t T, int64_t n, int k, int R, int half) {
  if (B <= 0 || T <= 0 || n <= 0 || R <= 0 || R > AT_MAX_ROUNDS || half <= 0 ||
      half > AT_MAX_HALF)
    return false;
  if (!(k == 2 || k == 4 || k == 8 || k == 16)) return false;
  const int64_t lanes = (int64_t)at_chunks(T) * B * n * k;
  return lanes < (1ll << 31);
}

template <int K, typename Kern>
int at_launch(Kern kern, const AtArgs& a, int64_t lanes, hipStream_t stream) {
  hipLaunchKernelGGL(kern, dim3((unsigned)((lanes + AT_THREADS - 1) / AT_THREADS)),
                     dim3(AT_THREADS), 0, stream, a);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

template <int K>
int at_fwd(AtArgs a, hipStream_t stream) {
  const int64_t chunk_lanes = (int64_t)a.n_chunks * a.NB * K, walk_lanes = a.NB * K;
  int rc = at_launch<K>(angle_tables_fwd_reduce<K>, a, chunk_lanes, stream);
  if (rc == MG_OK) rc = at_launch<K>(angle_tables_fwd_walk<K>, a, walk_lanes, stream);
  if (rc == MG_OK) rc = at_launch<K>(angle_tables_fwd_final<K>, a, chunk_lanes, stream);
  return rc;
}

template <int K>
int at_bwd(AtArgs a, hipStream_t stream) {
  const int64_t chunk_lanes = (int64_t)a.n_chunks * a.NB * K, walk_lanes = a.NB * K;
  int rc = at_launch<K>(angle_tables_bwd_reduce<K>, a, chunk_lanes, stream);
  if (rc == MG_OK) rc = at_launch<K>(angle_tables_bwd_walk<K>, a, walk_lanes, stream);
  if (rc == MG_OK) rc = at_launch<K>(angle_tables_bwd_final<K>, a, chunk_lanes, stream);
  return rc;
}

int at_by_k(int k, AtArgs& a, bool bwd, hipStream_t stream) {
  switch (k) {
    case 2: return bwd ? at_bwd<2>(a, stream) : at_fwd<2>(a, stream);
    case 4: return bwd ? at_bwd<4>(a, stream) : at_fwd<4>(a, stream);
    case 8: return bwd ? at_bwd<8>(a, stream) : at_fwd<8>(a, stream);
    default: return bwd ? at_bwd<16>(a, stream) : at_fwd<16>(a, stream);
  }
}

// Workspace: lsum and bound, [chunk][block][k] floats each.
size_t at_ws_bytes(int64_t B, int64_t T, int64_t n, int k) {
  return 2 * mg_align_up((size_t)at_chunks(T) * B * n * k * sizeof(float), 256);
}

}  // namespace

extern "C" {

size_t mg_angle_scan_tables_state_bytes(int64_t B, int64_t T, int64_t n, int k) {
  if (B <= 0 || T <= 0 || n <= 0 || k <= 0 || k > 16) return 0;
  return (size_t)at_chunks(T) * B * n * k * k * sizeof(float);
}

size_t mg_angle_scan_tables_workspace_bytes(int64_t B, int64_t T, int64_t n, int k) {
  if (B <= 0 || T <= 0 || n <= 0 || k <= 0 || k > 16) return 256;
  return at_ws_bytes(B, T, n, k);
}

int mg_angle_scan_tables_fwd(const float* theta, const float* scale, const float* gamma,
                             const float* b, const float* h0, const int* perm, const float* sgn,
                             const int* p2p, float* h, float* chunk_prod, int64_t B, int64_t T,
                             int64_t n, int k, int R, int half, int flags, void* ws,
                             size_t ws_bytes, hipStream_t stream) {
  if (!theta || !b || !h0 || !perm || !sgn || !p2p || !h || !chunk_prod || !ws) return MG_ERR_ARG;
  if (!at_args_ok(B, T, n, k, R, half)) return MG_ERR_ARG;
  if (((flags & 1) && !scale) || ((flags & 2) && !gamma) || (flags & ~3)) return MG_ERR_ARG;
  if (ws_bytes < at_ws_bytes(B, T, n, k)) return MG_ERR_WORKSPACE;
  const size_t half_ws = at_ws_bytes(B, T, n, k) / 2;
  AtArgs a{theta, scale, gamma, b, h0, perm, sgn, p2p, nullptr, nullptr, h, nullptr, nullptr,
           nullptr, nullptr, chunk_prod, (float*)ws, (float*)((char*)ws + half_ws),
           B, T, n, B * n, k, R, half, at_chunks(T), flags & 1, (flags >> 1) & 1};
  return at_by_k(k, a, false, stream);
}

int mg_angle_scan_tables_bwd(const float* theta, const float* scale, const float* gamma,
                             const float* h0, const float* h, const float* chunk_prod,
                             const float* gh, const int* perm, const float* sgn, const int* p2p,
                             float* dtheta, float* dscale, float* dgamma, float* db, float* dh0,
                             int64_t B, int64_t T, int64_t n, int k, int R, int half, int flags,
                             void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!theta || !h0 || !h || !chunk_prod || !gh || !perm || !sgn || !p2p || !dtheta || !db ||
      !dh0 || !ws)
    return MG_ERR_ARG;
  if (!at_args_ok(B, T, n, k, R, half)) return MG_ERR_ARG;
  if (((flags & 1) && (!scale || !dscale)) || ((flags & 2) && (!gamma || !dgamma)) ||
      (flags & ~3))
    return MG_ERR_ARG;
  if (ws_bytes < at_ws_bytes(B, T, n, k)) return MG_ERR_WORKSPACE;
  const size_t half_ws = at_ws_bytes(B, T, n, k) / 2;
  AtArgs a{theta, scale, gamma, nullptr, h0, perm, sgn, p2p, h, gh, db, dtheta, dscale, dgamma,
           dh0, const_cast<float*>(chunk_prod), (float*)ws, (float*)((char*)ws + half_ws),
           B, T, n, B * n, k, R, half, at_chunks(T), flags & 1, (flags >> 1) & 1};
  return at_by_k(k, a, true, stream);
}

}  // extern "C"

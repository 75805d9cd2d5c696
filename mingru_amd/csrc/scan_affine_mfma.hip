// Block-matrix affine scans with 8x8 and 16x16 blocks on the matrix cores
// (matrix_affine_scan / matrix_scan, reference src/mingru/min_gru.py:1513-1655;
// the reference kernel's envelope k in {1, 2, 4, 8, 16},
// src/mingru/triton_scans.py:183), fwd + bwd.
//
// Recurrence and adjoint as in scan_affine.hip:
//   Abar_t = A_t Abar_{t-1},  Bbar_t = A_t Bbar_{t-1} + B_t
//   X_t = G_t + A_{t+1}^T X_{t+1},  dA_t = XA_t Abar_{t-1}^T + XB_t Bbar_{t-1}^T,  dB_t = XB_t.
//
// One wave owns one 16x16 block: a 16x16 plane, or two 8x8 planes placed on the
// block diagonal (their products stay block diagonal; the zero blocks cost MFMA
// work but no memory traffic).  The k x v offsets of the block's planes are
// stacked into a 16 x 16 matrix whose columns beyond v are zero.  Every product
// of two 16x16 matrices is four v_mfma_f32_16x16x4f32, so a step holds its
// state in 4 + 4 registers per lane instead of the k*k + k*v floats a
// thread-per-plane kernel needs (256 + 256 for k = 16).
//
// Register layouts of a 16x16 matrix M over a wave, lane l = 16 g + c:
//   col layout (the MFMA accumulator): register i holds M[4g + i][c]
//   row layout:                       register q holds M[c][4g + q]
// mm(X_row, Z_col, C_col) returns C + X Z in col layout: the q-th MFMA contracts
// k = 4g + q, whose Z entries are exactly register q of the col layout, so the
// state (right factor) feeds the next product without any data movement.  The
// row layout of M is the col layout of M^T; a transposed copy goes through LDS.
//
// Time is split into chunks of WAVES * TSUB steps per workgroup (one block),
// chained by the decoupled look-back of the other scans; the carried map is
// (P, L) for the forward and (P, LA, LB) for the backward.  A look-back walk
// accumulates the transposed prefix E^T = X^T E^T: a predecessor's published
// col-layout registers are the row layout of its transpose, so the walk needs
// no transposes either.
#include "mg_affm.h"

#include <algorithm>

namespace {

using namespace mg;

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int AM_WAVES = 4;
constexpr int AM_TSUB = 8;
constexpr int AM_LDS_STRIDE = 20;  // floats per LDS row: 16 + 4 keeps 16-byte row reads aligned
constexpr int AM_LDS_MAT = 16 * AM_LDS_STRIDE;

__device__ __forceinline__ v4f mm(v4f xr, v4f zc, v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xr[0], zc[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xr[1], zc[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xr[2], zc[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xr[3], zc[3], acc, 0, 0, 0);
  return acc;
}

__device__ __forceinline__ v4f v4zero() { return v4f{0.f, 0.f, 0.f, 0.f}; }

// The identity in col layout (equally in row layout): entry (4g + i, c).
__device__ __forceinline__ v4f v4eye(int g, int c) {
  v4f r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (4 * g + i == c) ? 1.f : 0.f;
  return r;
}

// Orders the LDS accesses of one wave's lanes around it (no s_barrier).
__device__ __forceinline__ void am_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// LDS matrices: row-major 16 x 16 with AM_LDS_STRIDE floats per row.
__device__ __forceinline__ void lds_put_col(float* s, v4f m, int g, int c) {
#pragma unroll
  for (int i = 0; i < 4; ++i) s[(4 * g + i) * AM_LDS_STRIDE + c] = m[i];
}
__device__ __forceinline__ v4f lds_get_col(const float* s, int g, int c) {
  v4f r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = s[(4 * g + i) * AM_LDS_STRIDE + c];
  return r;
}
__device__ __forceinline__ v4f lds_get_row(const float* s, int g, int c) {
  const float4 v = *reinterpret_cast<const float4*>(s + c * AM_LDS_STRIDE + 4 * g);
  return v4f{v.x, v.y, v.z, v.w};
}

// Row layout of a matrix held in col layout, through this wave's scratch matrix.
__device__ __forceinline__ v4f col_to_row(v4f m, float* s, int g, int c) {
  am_wave_sync();  // earlier reads of the scratch are done
  lds_put_col(s, m, g, c);
  am_wave_sync();
  return lds_get_row(s, g, c);
}

struct AmGeom {
  int64_t T, n;
  int ng, n_lg, n_chunks;  // 16x16 blocks per batch row, blocks in total, chunks
};

struct AmThread {
  int lane, g, c, w, chunk, bb, gi;
  unsigned epoch;
  bool valid;
};

template <bool REVERSE>
__device__ __forceinline__ AmThread am_thread(const AmGeom& geo, unsigned* header) {
  AmThread th;
  const MgTicket tk = mg_take_ticket(header);
  th.valid = tk.ticket < gridDim.x;
  const unsigned ticket = th.valid ? tk.ticket : 0u;
  th.epoch = tk.epoch;
  th.lane = threadIdx.x & (MG_WAVE - 1);
  th.g = th.lane >> 4;
  th.c = th.lane & 15;
  th.w = threadIdx.x / MG_WAVE;
  const int kk = (int)(ticket / (unsigned)geo.n_lg);
  const int lg = (int)(ticket - (unsigned)kk * (unsigned)geo.n_lg);
  th.chunk = REVERSE ? geo.n_chunks - 1 - kk : kk;
  th.bb = lg / geo.ng;
  th.gi = lg - th.bb * geo.ng;
  return th;
}

// Memory access of one block at one time step.  PPW = 16 / K planes per block.
template <int K, int V>
struct AmIo {
  static constexpr int PPW = 16 / K;
  int64_t T, n, bb;
  int gi, g, c;

  // plane of block row r, or -1 outside the problem
  __device__ __forceinline__ int64_t plane(int r) const {
    const int64_t p = (int64_t)gi * PPW + r / K;
    return p < n ? p : -1;
  }
  __device__ __forceinline__ int64_t tok(int64_t t, int64_t p) const { return (bb * T + t) * n + p; }

  // Row layout of the k x k matrix X_t (A_t, or Abar_t for the transposed reads):
  // row c, columns 4g..4g+3; identity outside the problem and off the diagonal blocks.
  __device__ __forceinline__ v4f ld_row_kk(const float* __restrict__ X, int64_t t) const {
    const int64_t p = plane(c);
    if (t >= 0 && t < T && p >= 0 && (4 * g) / K == c / K) {
      const float4 v = *reinterpret_cast<const float4*>(X + tok(t, p) * (K * K) + (c % K) * K +
                                                        (4 * g) % K);
      return v4f{v.x, v.y, v.z, v.w};
    }
    return (t >= 0 && t < T && p >= 0) ? v4zero() : v4eye(g, c);
  }
  // Row layout of X_t^T (col layout of X_t): entry (4g + q, c) of X_t.
  __device__ __forceinline__ v4f ld_col_kk(const float* __restrict__ X, int64_t t,
                                           bool eye_outside) const {
    v4f r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 4 * g + q;
      const int64_t p = plane(row);
      if (t < T && p >= 0 && row / K == c / K)
        r[q] = X[tok(t, p) * (K * K) + (row % K) * K + c % K];
      else
        r[q] = (eye_outside && (t >= T || p < 0) && row == c) ? 1.f : 0.f;
    }
    return r;
  }
  __device__ __forceinline__ void st_col_kk(float* __restrict__ X, int64_t t, v4f m) const {
    if (t >= T) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * g + i;
      const int64_t p = plane(row);
      if (p >= 0 && row / K == c / K) X[tok(t, p) * (K * K) + (row % K) * K + c % K] = m[i];
    }
  }
  // Col layout of the stacked k x v offsets (zero columns beyond v).
  __device__ __forceinline__ v4f ld_col_kv(const float* __restrict__ X, int64_t t) const {
    v4f r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * g + i;
      const int64_t p = plane(row);
      r[i] = (t < T && c < V && p >= 0) ? X[tok(t, p) * (K * V) + (row % K) * V + c] : 0.f;
    }
    return r;
  }
  __device__ __forceinline__ void st_col_kv(float* __restrict__ X, int64_t t, v4f m) const {
    if (t >= T || c >= V) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * g + i;
      const int64_t p = plane(row);
      if (p >= 0) X[tok(t, p) * (K * V) + (row % K) * V + c] = m[i];
    }
  }
  // Col layout of Bbar_t^T: entry (4g + q, c) = Bbar_t[c][4g + q] (zero beyond v).
  __device__ __forceinline__ v4f ld_colT_kv(const float* __restrict__ X, int64_t t) const {
    v4f r = v4zero();
    const int64_t p = plane(c);
    if (t < 0 || t >= T || p < 0) return r;
    const float* row = X + tok(t, p) * (K * V) + (c % K) * V;
    if constexpr (V % 4 == 0) {
      if (4 * g < V) {
        const float4 v = *reinterpret_cast<const float4*>(row + 4 * g);
        r = v4f{v.x, v.y, v.z, v.w};
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * g + q < V) r[q] = row[4 * g + q];
    }
    return r;
  }
};

// Look-back slots: [block][chunk][field][64 lanes] tagged words.
template <int NF>
__device__ __forceinline__ void am_put(mg_slot_t* base, const AmGeom& geo, int lg, int chunk,
                                       int lane, const v4f (&x)[NF / 4], unsigned epoch) {
  mg_slot_t* p = base + ((int64_t)lg * geo.n_chunks + chunk) * NF * MG_WAVE + lane;
#pragma unroll
  for (int m = 0; m < NF / 4; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) mg_slot_put(p + (4 * m + i) * MG_WAVE, x[m][i], epoch);
}

template <int NF>
__device__ __forceinline__ bool am_try(const mg_slot_t* base, const AmGeom& geo, int lg, int chunk,
                                       int lane, v4f (&x)[NF / 4], unsigned epoch) {
  const mg_slot_t* p = base + ((int64_t)lg * geo.n_chunks + chunk) * NF * MG_WAVE + lane;
  bool ok = true;
#pragma unroll
  for (int m = 0; m < NF / 4; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v;
      ok &= mg_slot_get(p + (4 * m + i) * MG_WAVE, v, epoch);
      x[m][i] = v;
    }
  return ok;
}

// Maps with NM matrices: m[0] = P (linear part), m[1..] = offsets; all col layout.
// Look-back for one workgroup (run by its wave 0).  `G` is the workgroup
// aggregate; returns E, the composition of every earlier (forward) / later
// (REVERSE) chunk's map, in col layout.  `scr` is this wave's LDS scratch.
template <int NM, bool REVERSE>
__device__ void am_lookback(const v4f (&G)[NM], const AmGeom& geo, const AmThread& th, int lg,
                            unsigned* header, mg_slot_t* agg, mg_slot_t* incl, float* scr,
                            v4f (&E)[NM]) {
  constexpr int NF = 4 * NM;
  const int first = REVERSE ? geo.n_chunks - 1 : 0;
  const int dir = REVERSE ? 1 : -1;
  // E^T accumulated in col layout (= E in row layout)
  v4f Et[NM];
  Et[0] = v4eye(th.g, th.c);
#pragma unroll
  for (int m = 1; m < NM; ++m) Et[m] = v4zero();
  if (th.chunk != first) {
    am_put<NF>(agg, geo, lg, th.chunk, th.lane, G, th.epoch);
    int j = th.chunk + dir;
    unsigned spins = 0;
    bool done = false;
    while (!done) {
      // A map is spread over the whole wave, so a predecessor's words are used only
      // once every lane has seen its own part published (wave-uniform decisions).
      v4f X[NM];
      bool have = __all(am_try<NF>(incl, geo, lg, j, th.lane, X, th.epoch));
      const bool inclusive = have;
      if (!have && j != first) have = __all(am_try<NF>(agg, geo, lg, j, th.lane, X, th.epoch));
      if (have) {
        // (E o X)^T: offsets L^T <- L_X^T P_E^T + L_E^T first, then P^T <- P_X^T P_E^T.
#pragma unroll
        for (int m = 1; m < NM; ++m) Et[m] = mm(X[m], Et[0], Et[m]);
        Et[0] = mm(X[0], Et[0], v4zero());
        if (inclusive) done = true;
        else j += dir;
      } else {
        __builtin_amdgcn_s_sleep(1);
        if (++spins >= MG_SPIN_LIMIT) {
          mg_count_error(header);
          done = true;
        }
      }
    }
  }
  // E in col layout (transpose back), then the inclusive map G o E.
#pragma unroll
  for (int m = 0; m < NM; ++m) E[m] = col_to_row(Et[m], scr, th.g, th.c);
  const v4f Gr = col_to_row(G[0], scr, th.g, th.c);
  v4f I[NM];
  I[0] = mm(Gr, E[0], v4zero());
#pragma unroll
  for (int m = 1; m < NM; ++m) I[m] = mm(Gr, E[m], G[m]);
  am_put<NF>(incl, geo, lg, th.chunk, th.lane, I, th.epoch);
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int K, int V, int TSUB, int WAVES>
__global__ __launch_bounds__(MG_WAVE* WAVES) void affine_mfma_fwd(
    const float* __restrict__ A, const float* __restrict__ Bm, float* __restrict__ Abar,
    float* __restrict__ Bbar, AmGeom geo, unsigned* header, mg_slot_t* agg, mg_slot_t* incl) {
  __shared__ __align__(16) float s_loc[WAVES][2][AM_LDS_MAT];
  __shared__ __align__(16) float s_ew[WAVES][2][AM_LDS_MAT];
  __shared__ __align__(16) float s_E[2][AM_LDS_MAT];
  __shared__ __align__(16) float s_scr[AM_LDS_MAT];
  const AmThread th = am_thread<false>(geo, header);
  if (!th.valid) return;
  const int lg = th.bb * geo.ng + th.gi;
  const AmIo<K, V> io{geo.T, geo.n, th.bb, th.gi, th.g, th.c};
  const int64_t t0 = (int64_t)th.chunk * (WAVES * TSUB) + th.w * TSUB;

  v4f a[TSUB], b[TSUB];
#pragma unroll
  for (int s = 0; s < TSUB; ++s) {
    a[s] = io.ld_row_kk(A, t0 + s);
    b[s] = io.ld_col_kv(Bm, t0 + s);
  }
  // This wave's sub-chunk map S -> P S + L.
  v4f P = v4eye(th.g, th.c), L = v4zero();
#pragma unroll
  for (int s = 0; s < TSUB; ++s) {
    L = mm(a[s], L, b[s]);
    P = mm(a[s], P, v4zero());
  }
  lds_put_col(s_loc[th.w][0], P, th.g, th.c);
  lds_put_col(s_loc[th.w][1], L, th.g, th.c);
  __syncthreads();
  if (th.w == 0) {
    // Exclusive prefixes ew_j = loc_{j-1} o ... o loc_0 and the aggregate G.
    v4f S[2] = {P, L};
    for (int j = 1; j < WAVES; ++j) {
      lds_put_col(s_ew[j][0], S[0], th.g, th.c);
      lds_put_col(s_ew[j][1], S[1], th.g, th.c);
      const v4f Xr = lds_get_row(s_loc[j][0], th.g, th.c);
      const v4f Xl = lds_get_col(s_loc[j][1], th.g, th.c);
      S[1] = mm(Xr, S[1], Xl);
      S[0] = mm(Xr, S[0], v4zero());
    }
    v4f E[2];
    am_lookback<2, false>(S, geo, th, lg, header, agg, incl, s_scr, E);
    lds_put_col(s_E[0], E[0], th.g, th.c);
    lds_put_col(s_E[1], E[1], th.g, th.c);
  }
  __syncthreads();
  v4f CP = lds_get_col(s_E[0], th.g, th.c), CL = lds_get_col(s_E[1], th.g, th.c);
  if (th.w > 0) {
    const v4f Xr = lds_get_row(s_ew[th.w][0], th.g, th.c);
    CL = mm(Xr, CL, lds_get_col(s_ew[th.w][1], th.g, th.c));
    CP = mm(Xr, CP, v4zero());
  }
  // Replay from (Abar_{t0-1}, Bbar_{t0-1}).
#pragma unroll
  for (int s = 0; s < TSUB; ++s) {
    CL = mm(a[s], CL, b[s]);
    CP = mm(a[s], CP, v4zero());
    io.st_col_kk(Abar, t0 + s, CP);
    io.st_col_kv(Bbar, t0 + s, CL);
  }
}

// ---------------------------------------------------------------------------
// backward: maps Y -> A_t^T (G_t + Y) on [YA | YB], composed in reverse time
// ---------------------------------------------------------------------------
template <int K, int V, int TSUB, int WAVES>
__global__ __launch_bounds__(MG_WAVE* WAVES) void affine_mfma_bwd(
    const float* __restrict__ A, const float* __restrict__ Abar, const float* __restrict__ Bbar,
    const float* __restrict__ GA, const float* __restrict__ GB, float* __restrict__ dA,
    float* __restrict__ dB, AmGeom geo, unsigned* header, mg_slot_t* agg, mg_slot_t* incl) {
  __shared__ __align__(16) float s_loc[WAVES][3][AM_LDS_MAT];
  __shared__ __align__(16) float s_ew[WAVES][3][AM_LDS_MAT];
  __shared__ __align__(16) float s_E[3][AM_LDS_MAT];
  __shared__ __align__(16) float s_scr[WAVES][AM_LDS_MAT];
  const AmThread th = am_thread<true>(geo, header);
  if (!th.valid) return;
  const int lg = th.bb * geo.ng + th.gi;
  const AmIo<K, V> io{geo.T, geo.n, th.bb, th.gi, th.g, th.c};
  const int64_t t0 = (int64_t)th.chunk * (WAVES * TSUB) + th.w * TSUB;
  float* scr = s_scr[th.w];

  v4f at[TSUB], ga[TSUB], gb[TSUB];
#pragma unroll
  for (int s = 0; s < TSUB; ++s) {
    at[s] = io.ld_col_kk(A, t0 + s, true);  // row layout of A_t^T
    ga[s] = io.ld_col_kk(GA, t0 + s, false);
    gb[s] = io.ld_col_kv(GB, t0 + s);
  }
  v4f M[3] = {v4eye(th.g, th.c), v4zero(), v4zero()};
#pragma unroll
  for (int s = TSUB - 1; s >= 0; --s) {
    M[1] = mm(at[s], ga[s] + M[1], v4zero());
    M[2] = mm(at[s], gb[s] + M[2], v4zero());
    M[0] = mm(at[s], M[0], v4zero());
  }
#pragma unroll
  for (int m = 0; m < 3; ++m) lds_put_col(s_loc[th.w][m], M[m], th.g, th.c);
  __syncthreads();
  if (th.w == 0) {
    // ew_j = loc_{j+1} o ... o loc_{W-1}; G = loc_0 o ... o loc_{W-1}.
    v4f S[3];
#pragma unroll
    for (int m = 0; m < 3; ++m) S[m] = lds_get_col(s_loc[WAVES - 1][m], th.g, th.c);
    for (int j = WAVES - 2; j >= 0; --j) {
#pragma unroll
      for (int m = 0; m < 3; ++m) lds_put_col(s_ew[j][m], S[m], th.g, th.c);
      const v4f Xr = lds_get_row(s_loc[j][0], th.g, th.c);
#pragma unroll
      for (int m = 1; m < 3; ++m) S[m] = mm(Xr, S[m], lds_get_col(s_loc[j][m], th.g, th.c));
      S[0] = mm(Xr, S[0], v4zero());
    }
    v4f E[3];
    am_lookback<3, true>(S, geo, th, lg, header, agg, incl, scr, E);
#pragma unroll
    for (int m = 0; m < 3; ++m) lds_put_col(s_E[m], E[m], th.g, th.c);
  }
  __syncthreads();
  // Adjoint entering this sub-chunk from the right: offsets of ew_w o E.
  v4f YA = lds_get_col(s_E[1], th.g, th.c), YB = lds_get_col(s_E[2], th.g, th.c);
  if (th.w < WAVES - 1) {
    const v4f Xr = lds_get_row(s_ew[th.w][0], th.g, th.c);
    YA = mm(Xr, YA, lds_get_col(s_ew[th.w][1], th.g, th.c));
    YB = mm(Xr, YB, lds_get_col(s_ew[th.w][2], th.g, th.c));
  }
#pragma unroll
  for (int s = TSUB - 1; s >= 0; --s) {
    const int64_t t = t0 + s;
    const v4f XA = ga[s] + YA, XB = gb[s] + YB;
    if (t < geo.T) {
      const v4f XAr = col_to_row(XA, scr, th.g, th.c);
      const v4f XBr = col_to_row(XB, scr, th.g, th.c);
      // Abar_{t-1}^T in col layout is Abar_{t-1} in row layout (identity before t = 0).
      v4f d = mm(XAr, io.ld_row_kk(Abar, t - 1), v4zero());
      d = mm(XBr, io.ld_colT_kv(Bbar, t - 1), d);
      io.st_col_kk(dA, t, d);
      io.st_col_kv(dB, t, XB);
    }
    YA = mm(at[s], XA, v4zero());
    YB = mm(at[s], XB, v4zero());
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
struct AmPlan {
  AmGeom g;
  size_t agg_off, incl_off, total;
};

AmPlan am_plan(int64_t B, int64_t T, int64_t n, int k, int nf) {
  AmPlan p;
  const int ppw = 16 / k;
  p.g.T = T;
  p.g.n = n;
  p.g.ng = (int)((n + ppw - 1) / ppw);
  p.g.n_lg = (int)(B * p.g.ng);
  const int64_t cl = (int64_t)AM_WAVES * AM_TSUB;
  p.g.n_chunks = (int)((T + cl - 1) / cl);
  const size_t data = (size_t)p.g.n_lg * p.g.n_chunks * nf * MG_WAVE * sizeof(mg_slot_t);
  p.agg_off = MG_HEADER_BYTES;
  p.incl_off = p.agg_off + mg_align_up(data, 256);
  p.total = p.incl_off + mg_align_up(data, 256);
  return p;
}

template <int K, int V>
int am_fwd(const float* A, const float* Bm, float* Abar, float* Bbar, int64_t B, int64_t T,
           int64_t n, void* ws, size_t ws_bytes, hipStream_t stream) {
  const AmPlan p = am_plan(B, T, n, K, 8);
  if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
  hipLaunchKernelGGL((affine_mfma_fwd<K, V, AM_TSUB, AM_WAVES>),
                     dim3((unsigned)(p.g.n_lg * p.g.n_chunks)), dim3(MG_WAVE * AM_WAVES), 0,
                     stream, A, Bm, Abar, Bbar, p.g, (unsigned*)ws,
                     (mg_slot_t*)((char*)ws + p.agg_off), (mg_slot_t*)((char*)ws + p.incl_off));
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

template <int K, int V>
int am_bwd(const float* A, const float* Abar, const float* Bbar, const float* GA, const float* GB,
           float* dA, float* dB, int64_t B, int64_t T, int64_t n, void* ws, size_t ws_bytes,
           hipStream_t stream) {
  const AmPlan p = am_plan(B, T, n, K, 12);
  if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
  hipLaunchKernelGGL((affine_mfma_bwd<K, V, AM_TSUB, AM_WAVES>),
                     dim3((unsigned)(p.g.n_lg * p.g.n_chunks)), dim3(MG_WAVE * AM_WAVES), 0,
                     stream, A, Abar, Bbar, GA, GB, dA, dB, p.g, (unsigned*)ws,
                     (mg_slot_t*)((char*)ws + p.agg_off), (mg_slot_t*)((char*)ws + p.incl_off));
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

#define MG_AM_DISPATCH(FN, ...)              \
  switch (k * 100 + v) {                     \
    case 801: return FN<8, 1>(__VA_ARGS__);  \
    case 802: return FN<8, 2>(__VA_ARGS__);  \
    case 804: return FN<8, 4>(__VA_ARGS__);  \
    case 808: return FN<8, 8>(__VA_ARGS__);  \
    case 816: return FN<8, 16>(__VA_ARGS__); \
    case 1601: return FN<16, 1>(__VA_ARGS__);  \
    case 1602: return FN<16, 2>(__VA_ARGS__);  \
    case 1604: return FN<16, 4>(__VA_ARGS__);  \
    case 1608: return FN<16, 8>(__VA_ARGS__);  \
    case 1616: return FN<16, 16>(__VA_ARGS__); \
    default: return MG_ERR_ARG;              \
  }

}  // namespace

namespace mg {

size_t affine_mfma_workspace_bytes(int64_t B, int64_t T, int64_t n, int k) {
  return std::max(am_plan(B, T, n, k, 8).total, am_plan(B, T, n, k, 12).total);
}

bool affine_mfma_geometry_ok(int64_t B, int64_t T, int64_t n, int k) {
  const int64_t blocks = B * ((n + 16 / k - 1) / (16 / k));
  const int64_t chunks = (T + AM_WAVES * AM_TSUB - 1) / (AM_WAVES * AM_TSUB);
  return blocks * chunks < (1ll << 31);
}

int affine_mfma_fwd(const float* A, const float* Bm, float* Abar, float* Bbar, int64_t B,
                    int64_t T, int64_t n, int k, int v, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
  MG_AM_DISPATCH(am_fwd, A, Bm, Abar, Bbar, B, T, n, ws, ws_bytes, stream)
}

int affine_mfma_bwd(const float* A, const float* Abar, const float* Bbar, const float* GA,
                    const float* GB, float* dA, float* dB, int64_t B, int64_t T, int64_t n, int k,
                    int v, void* ws, size_t ws_bytes, hipStream_t stream) {
  MG_AM_DISPATCH(am_bwd, A, Abar, Bbar, GA, GB, dA, dB, B, T, n, ws, ws_bytes, stream)
}

}  // namespace mg

// DeltaMinGRU chunked-WY delta rule, forward and backward (gfx950, MFMA).
//
// Recurrence per head (reference src/mingru/min_gru.py:3103-3255, 3611-3688):
// for every micro-step m (token-major, nh per token)
//     H <- H - beta_m k_m (k_m^T H) + beta_m k_m v_m^T,       y_t = H_t^T q_t.
// Chunked-WY form over a chunk of C tokens (M = nh C micro-rows), with Hc the
// state entering the chunk:
//     KK = K K^T,  L = strict_lower(KK) * beta_col,  Tm = I + L
//     U  = Tm^-1 (V - K Hc) = U0 - W Hc,   U0 = Tm^-1 V,  W = Tm^-1 K
//     P  = (Q K^T) * beta_col * read,  read[t][m] = (m < (t+1) nh)
//     y  = Q Hc + P U,   H_next = Hc + K^T (beta_row * U).
// Backward (reference src/mingru/triton_scans.py:473-605), with dHn the
// gradient of the state leaving the chunk:
//     G  = Tm^-T (P^T dy + beta_row * (K dHn)) = G0 + E dHn,
//          G0 = Tm^-T P^T dy,  E = Tm^-T diag(beta) K
//     dHc = dHn + Q^T dy - K^T G,   dV = G
//     dQ = dy Hc^T + dS K,          dS = (dy U^T) * beta_col * read
//     dK = dS^T Q + (beta_row U) dHn^T - G Hc^T + dKK K + dKK^T K,
//          dKK = (-G U^T) * beta_col * strict
//     dbeta_m = sum_j U[m][j] (K dHn)[m][j] + sum_t dP[t][m] S[t][m] read[t][m]
//             + sum_i dT[i][m] KK[i][m] strict[i][m].
//
// Kernels (every matrix is zero-padded to 64 x 64; d_k, d_v <= 64, M <= 64):
//   fwd_prep   grid (chunk, head): KK, blocked inverse Tm^-1, W, U0, P
//   fwd_chain  grid (head * d_v slice): serial over chunks, H slice (64 x 16)
//              resident; U = U0 - W H, y = Q H + P U, H += K^T (beta U);
//              stores the chunk-entry states (saved for the backward)
//   bwd_prep   grid (chunk, head): Tm^-1 again, U, P, E, G0, Q^T dy
//   bwd_chain  grid (head * d_v slice): reverse serial pass, G = G0 + E dH,
//              dH += Q^T dy - K^T G; stores G and the chunk-exit state grads
//   bwd_grads  grid (chunk, head): dQ, dK, dV, dbeta from Hc, dHn, U, G.
// The serial passes are split over d_v because both recurrences act on the
// columns of H independently.  These kernels serve fp32 inputs: products run
// on v_mfma_f32_16x16x4_f32 with fp32 operands (gfx950 has no reduced-precision
// fp32 MFMA).  bf16 inputs go to the bf16-MFMA kernels of delta_wy_bf16.hip;
// the entry points below pick the path from the dtype tag.
#include "mg_delta.h"

namespace {

using namespace mgd;

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename TI>
__global__ __launch_bounds__(NT) void dw_fwd_prep(const TI* __restrict__ Q, const TI* __restrict__ K,
                                                  const TI* __restrict__ V, const TI* __restrict__ beta,
                                                  float* __restrict__ Wo, float* __restrict__ U0o,
                                                  float* __restrict__ Po, float* __restrict__ To,
                                                  DwGeom g) {
  __shared__ float sK[DN * LD], sV[DN * LD], sL[DN * LD], sT[DN * LD];
  __shared__ float sY[2 * 32 * LDS16];
  __shared__ float sb[DN];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;  // first micro-row of the chunk
  Tile<TI> tk, tv, tq;
  tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
  tv.load(V + row0 * g.dv, ch.M, g.dv, g.dv);
  tq.load(Q + (bh * g.T + ch.t0) * g.dk, ch.Ct, g.dk, g.dk);
  const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
  tk.store(sK);
  tv.store(sV);
  sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
  __syncthreads();
  build_L(sK, sb, sL);
  __syncthreads();
  unit_lower_inverse(sL, sT, sY);  // ends with a barrier
  // sL is free: Q goes there for P.
  tq.store(sL);
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  store_inv_packed<NT>(To + mat, sT);  // for the backward preparation kernel
  {
    floatx4 wa[4], ua[4];
    zero_row4(wa);
    zero_row4(ua);
    mma_row4<64>(wa, sT + 16 * w * LD, LD, 1, sK, LD, 1, 16);
    mma_row4<64>(ua, sT + 16 * w * LD, LD, 1, sV, LD, 1, 16);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      acc_store_ws(wa[J], Wo + mat + 16 * w * DN + 16 * J);
      acc_store_ws(ua[J], U0o + mat + 16 * w * DN + 16 * J);
    }
  }
  __syncthreads();
  {
    floatx4 sp[4];
    zero_row4(sp);
    mma_row4<64>(sp, sL + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, m = 16 * J + r;
        const float v = sp[J][i] * sb[m];  // formed first: the mask then picks a local
        sp[J][i] = (m < (t + 1) * g.nh) ? v : 0.f;
      }
      acc_store_ws(sp[J], Po + mat + 16 * w * DN + 16 * J);
    }
  }
}

// Loads 16 consecutive floats (a lane's A-fragment row segment for KD = 64).
__device__ __forceinline__ void load16(float (&a)[16], const float* p) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float4 x = q[v];
    a[4 * v] = x.x;
    a[4 * v + 1] = x.y;
    a[4 * v + 2] = x.z;
    a[4 * v + 3] = x.w;
  }
}

// acc += sign * A B with A's row segment held in registers (KD = 64) and B in LDS.
__device__ __forceinline__ floatx4 mma_reg(floatx4 acc, const float (&a)[16], const float* b,
                                           int brs, float sa) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 16; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sa * a[s], b[(16 * g + s) * brs + r], acc, 0, 0, 0);
  return acc;
}

template <typename TI>
__global__ __launch_bounds__(NT) void dw_fwd_chain(const TI* __restrict__ Q, const TI* __restrict__ K,
                                                   const TI* __restrict__ beta,
                                                   const float* __restrict__ H0,
                                                   const float* __restrict__ Wm,
                                                   const float* __restrict__ U0m,
                                                   const float* __restrict__ Pm, TI* __restrict__ y,
                                                   float* __restrict__ HT, float* __restrict__ Hb,
                                                   DwGeom g, int64_t BH) {
  __shared__ float sK[2][DN * LD], sQ[2][DN * LD];
  __shared__ float sb[2][DN];
  __shared__ float sH[DN * LDS16], sU[DN * LDS16];
  int64_t bh;
  int col0;
  if (!chain_slot(g, BH, bh, col0)) return;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int col = col0 + r;
  // H slice rows 16w..16w+15 (d_k), columns col0..col0+15 (d_v), accumulator layout.
  floatx4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    h[i] = ldf_or0(H0, (bh * g.dk + d) * g.dv + col, d < g.dk && col < g.dv);
  }
  // Operands of chunk c + 1 are fetched into registers while chunk c computes.
  Tile<TI> tk, tq;
  float bv, wa[16], pa[16];
  floatx4 u0;
  auto fetch = [&](int c) {
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tq.load(Q + (bh * g.T + ch.t0) * g.dk, ch.Ct, g.dk, g.dk);
    bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    load16(wa, Wm + mat + (16 * w + r) * DN + 16 * gg);
    load16(pa, Pm + mat + (16 * w + r) * DN + 16 * gg);
    u0 = acc_load_ws(U0m + mat + 16 * w * DN + col0);
  };
  fetch(0);
  for (int c = 0; c < g.nc; ++c) {
    const int buf = c & 1;
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    tk.store(sK[buf]);
    tq.store(sQ[buf]);
    sb[buf][threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values
    float wc[16], pc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      wc[i] = wa[i];
      pc[i] = pa[i];
    }
    floatx4 u = u0;
    if (c + 1 < g.nc) fetch(c + 1);
    acc_store_lds(h, sH + 16 * w * LDS16, LDS16);
    acc_store_ws(h, Hb + mat + 16 * w * DN + col0);
    __syncthreads();
    u = mma_reg(u, wc, sH, LDS16, -1.f);  // U = U0 - W H (rows 16w.. of the micro-steps)
    acc_store_lds(u, sU + 16 * w * LDS16, LDS16);
    floatx4 yy = mma<64>(zero4(), sQ[buf] + 16 * w * LD, LD, 1, sH, LDS16, 1);
    __syncthreads();
    yy = mma_reg(yy, pc, sU, LDS16, 1.f);  // + P U
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * gg + i;
      if (t < ch.Ct && col < g.dv) stf(y, (bh * g.T + ch.t0 + t) * g.dv + col, yy[i]);
    }
    // H += K^T (beta U): A[i][m] = beta_m K[m][16w + i].
    {
      const float* kb = sK[buf];
      const float* bb = sb[buf];
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const int m = 16 * gg + s;
        h = __builtin_amdgcn_mfma_f32_16x16x4f32(bb[m] * kb[m * LD + 16 * w + r],
                                                 sU[m * LDS16 + r], h, 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    if (d < g.dk && col < g.dv) HT[(bh * g.dk + d) * g.dv + col] = h[i];
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
template <typename TI>
__global__ __launch_bounds__(NT) void dw_bwd_prep(const TI* __restrict__ Q, const TI* __restrict__ K,
                                                  const TI* __restrict__ V, const TI* __restrict__ beta,
                                                  const TI* __restrict__ dy,
                                                  const float* __restrict__ Hb,
                                                  const float* __restrict__ Tin,
                                                  float* __restrict__ Uo, float* __restrict__ Eo,
                                                  float* __restrict__ G0o, float* __restrict__ QdYo,
                                                  DwGeom g) {
  __shared__ float sK[DN * LD], sV[DN * LD], sL[DN * LD], sT[DN * LD], sX[DN * LD];
  __shared__ float sQ[DN * LD], sD[DN * LD];
  __shared__ float sb[DN];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  {
    Tile<TI> tk, tv, tq, td;
    Tile<float> th;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tv.load(V + row0 * g.dv, ch.M, g.dv, g.dv);
    th.load(Hb + mat, g.dk, g.dv, DN);
    tq.load(Q + (bh * g.T + ch.t0) * g.dk, ch.Ct, g.dk, g.dk);
    td.load(dy + (bh * g.T + ch.t0) * g.dv, ch.Ct, g.dv, g.dv);
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    tk.store(sK);
    tv.store(sV);
    th.store(sX);
    tq.store(sQ);
    td.store(sD);
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
    load_inv_packed<NT>(sT, Tin + mat);  // T = (I + L)^-1 as the forward formed it
  }
  __syncthreads();
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  // R = V - K Hc in place in sV (tile (w, J) read and written by wave w only).
  {
    floatx4 acc[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) acc[J] = acc_load_lds(sV + 16 * w * LD + 16 * J, LD);
    mma_row4<64>(acc, sK + 16 * w * LD, LD, 1, sX, LD, 1, 16, -1.f);
#pragma unroll
    for (int J = 0; J < 4; ++J) acc_store_lds(acc[J], sV + 16 * w * LD + 16 * J, LD);
  }
  __syncthreads();
  // U = Tm^-1 R; P = (Q K^T) * beta_col * read into sL (free).
  {
    floatx4 u[4], sp[4];
    zero_row4(u);
    zero_row4(sp);
    mma_row4<64>(u, sT + 16 * w * LD, LD, 1, sV, LD, 1, 16);
    mma_row4<64>(sp, sQ + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      acc_store_ws(u[J], Uo + mat + 16 * w * DN + 16 * J);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, m = 16 * J + r;
        const float v = sp[J][i] * sb[m];  // formed first: the mask then picks a local
        sp[J][i] = (m < (t + 1) * g.nh) ? v : 0.f;
      }
      acc_store_lds(sp[J], sL + 16 * w * LD + 16 * J, LD);
    }
  }
  __syncthreads();
  // D1 = P^T dy into sX (Hc no longer needed); Q^T dy and E = Tm^-T diag(beta) K out.
  {
    floatx4 d1[4], qd[4];
    zero_row4(d1);
    zero_row4(qd);
    mma_row4<64>(d1, sL + 16 * w, 1, LD, sD, LD, 1, 16);
    mma_row4<64>(qd, sQ + 16 * w, 1, LD, sD, LD, 1, 16);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      acc_store_lds(d1[J], sX + 16 * w * LD + 16 * J, LD);
      acc_store_ws(qd[J], QdYo + mat + 16 * w * DN + 16 * J);
    }
  }
  // sK := diag(beta) K for E, once every wave is done with the unscaled K.
  __syncthreads();
  for (int e = threadIdx.x; e < DN * DN; e += NT) {
    const int i = e >> 6, j = e & 63;
    sK[i * LD + j] *= sb[i];
  }
  __syncthreads();
  {
    floatx4 ea[4], g0[4];
    zero_row4(ea);
    zero_row4(g0);
    mma_row4<64>(ea, sT + 16 * w, 1, LD, sK, LD, 1, 16);
    mma_row4<64>(g0, sT + 16 * w, 1, LD, sX, LD, 1, 16);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      acc_store_ws(ea[J], Eo + mat + 16 * w * DN + 16 * J);
      acc_store_ws(g0[J], G0o + mat + 16 * w * DN + 16 * J);
    }
  }
}

template <typename TI>
__global__ __launch_bounds__(NT) void dw_bwd_chain(const TI* __restrict__ K,
                                                   const float* __restrict__ dHT,
                                                   const float* __restrict__ Em,
                                                   const float* __restrict__ G0m,
                                                   const float* __restrict__ QdYm,
                                                   float* __restrict__ Gm, float* __restrict__ dHn,
                                                   float* __restrict__ dH0, DwGeom g, int64_t BH) {
  __shared__ float sK[2][DN * LD];
  __shared__ float sH[DN * LDS16], sG[DN * LDS16];
  int64_t bh;
  int col0;
  if (!chain_slot(g, BH, bh, col0)) return;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int col = col0 + r;
  floatx4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    h[i] = ldf_or0(dHT, (bh * g.dk + d) * g.dv + col, d < g.dk && col < g.dv);
  }
  Tile<TI> tk;
  float ea[16];
  floatx4 g0, qd0;
  auto fetch = [&](int c) {
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    tk.load(K + (bh * g.T + ch.t0) * g.nh * g.dk, ch.M, g.dk, g.dk);
    load16(ea, Em + mat + (16 * w + r) * DN + 16 * gg);
    g0 = acc_load_ws(G0m + mat + 16 * w * DN + col0);
    qd0 = acc_load_ws(QdYm + mat + 16 * w * DN + col0);
  };
  fetch(g.nc - 1);
  for (int c = g.nc - 1; c >= 0; --c) {
    const int buf = c & 1;
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    tk.store(sK[buf]);
    float ec[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) ec[i] = ea[i];
    floatx4 gacc = g0;
    const floatx4 qd = qd0;
    if (c > 0) fetch(c - 1);
    acc_store_lds(h, sH + 16 * w * LDS16, LDS16);
    acc_store_ws(h, dHn + mat + 16 * w * DN + col0);
    __syncthreads();
    gacc = mma_reg(gacc, ec, sH, LDS16, 1.f);  // G = G0 + E dH
    acc_store_ws(gacc, Gm + mat + 16 * w * DN + col0);
    acc_store_lds(gacc, sG + 16 * w * LDS16, LDS16);
    __syncthreads();
    // dH += Q^T dy - K^T G: A[i][m] = K[m][16w + i].
    h += qd;
    const float* kb = sK[buf];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int m = 16 * gg + s;
      h = __builtin_amdgcn_mfma_f32_16x16x4f32(-kb[m * LD + 16 * w + r], sG[m * LDS16 + r], h, 0,
                                               0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    if (d < g.dk && col < g.dv) dH0[(bh * g.dk + d) * g.dv + col] = h[i];
  }
}

template <typename TI>
__global__ __launch_bounds__(NT) void dw_bwd_grads(
    const TI* __restrict__ Q, const TI* __restrict__ K, const TI* __restrict__ beta,
    const TI* __restrict__ dy, const float* __restrict__ Hb, const float* __restrict__ dHn,
    const float* __restrict__ Um, const float* __restrict__ Gm, TI* __restrict__ dQ,
    TI* __restrict__ dK, TI* __restrict__ dV, TI* __restrict__ dbeta, DwGeom g) {
  __shared__ float sK[DN * LD], sQ[DN * LD], sD[DN * LD], sU[DN * LD], sG[DN * LD],
      sH[DN * LD], sX[DN * LD];
  __shared__ float sb[DN];
  // dbeta partials: [0..3] read-term column sums per wave, [4..7] strict-term
  // column sums per wave, [8] row sums of U * (K dHn).
  __shared__ float sdb[9][DN];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const int64_t trow0 = bh * g.T + ch.t0;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  Tile<float> tn;  // dHn, stored once Hc is no longer needed
  {
    Tile<TI> tk, tq, td;
    Tile<float> tu, tg, th;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tq.load(Q + trow0 * g.dk, ch.Ct, g.dk, g.dk);
    td.load(dy + trow0 * g.dv, ch.Ct, g.dv, g.dv);
    tu.load(Um + mat, ch.M, g.dv, DN);
    tg.load(Gm + mat, ch.M, g.dv, DN);
    th.load(Hb + mat, g.dk, g.dv, DN);
    tn.load(dHn + mat, g.dk, g.dv, DN);
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    tk.store(sK);
    tq.store(sQ);
    td.store(sD);
    tu.store(sU);
    tg.store(sG);
    th.store(sH);
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
  }
  __syncthreads();
  // S = Q K^T, dP = dy U^T (rows = tokens of block w, cols = micro-rows of block J).
  floatx4 s4[4], dp4[4];
  zero_row4(s4);
  zero_row4(dp4);
  mma_row4<64>(s4, sQ + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
  mma_row4<64>(dp4, sD + 16 * w * LD, LD, 1, sU, 1, LD, 16 * LD);
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    const floatx4 s = s4[J], dp = dp4[J];
    floatx4 ds, db;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * gg + i, m = 16 * J + r;
      const bool rd = m < (t + 1) * g.nh;
      const float dv = dp[i] * sb[m], bv = dp[i] * s[i];  // formed first, then picked
      ds[i] = rd ? dv : 0.f;
      db[i] = rd ? bv : 0.f;
    }
    acc_store_lds(ds, sX + 16 * w * LD + 16 * J, LD);
    put_colsum(db, sdb[w], 16 * J + r);
  }
  __syncthreads();
  // dQ = dy Hc^T + dS K; dK (kept in registers) = dS^T Q - G Hc^T.
  floatx4 dk[4];
  {
    floatx4 q[4];
    zero_row4(q);
    mma_row4<64>(q, sD + 16 * w * LD, LD, 1, sH, 1, LD, 16 * LD);
    mma_row4<64>(q, sX + 16 * w * LD, LD, 1, sK, LD, 1, 16);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, d = 16 * J + r;
        if (t < ch.Ct && d < g.dk) stf(dQ, (trow0 + t) * g.dk + d, q[J][i]);
      }
    }
    zero_row4(dk);
    mma_row4<64>(dk, sX + 16 * w, 1, LD, sQ, LD, 1, 16);
    mma_row4<64>(dk, sG + 16 * w * LD, LD, 1, sH, 1, LD, 16 * LD, -1.f);
  }
  __syncthreads();
  // dT = -G U^T, KK = K K^T; dKK = dT * beta_col * strict into sX.  dHn into sH.
  floatx4 dt4[4], kk4[4];
  zero_row4(dt4);
  zero_row4(kk4);
  mma_row4<64>(dt4, sG + 16 * w * LD, LD, 1, sU, 1, LD, 16 * LD, -1.f);
  mma_row4<64>(kk4, sK + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    const floatx4 dt = dt4[J], kk = kk4[J];
    floatx4 dkk, db;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * w + 4 * gg + i, j = 16 * J + r;
      const bool st = j < m;
      const float kv = dt[i] * sb[j], bv = dt[i] * kk[i];  // formed first, then picked
      dkk[i] = st ? kv : 0.f;
      db[i] = st ? bv : 0.f;
    }
    acc_store_lds(dkk, sX + 16 * w * LD + 16 * J, LD);
    put_colsum(db, sdb[4 + w], 16 * J + r);
  }
  tn.store(sH);
  __syncthreads();
  // dK += dKK K + dKK^T K + (beta_row U) dHn^T; dbeta += rowsum(U * (K dHn)).
  float rowp[4] = {0.f, 0.f, 0.f, 0.f};
  floatx4 bu4[4], x4[4];
  mma_row4<64>(dk, sX + 16 * w * LD, LD, 1, sK, LD, 1, 16);
  mma_row4<64>(dk, sX + 16 * w, 1, LD, sK, LD, 1, 16);
  zero_row4(bu4);
  zero_row4(x4);
  mma_row4<64>(bu4, sU + 16 * w * LD, LD, 1, sH, 1, LD, 16 * LD);
  mma_row4<64>(x4, sK + 16 * w * LD, LD, 1, sH, LD, 1, 16);
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    floatx4 a = dk[J];
    const floatx4 bu = bu4[J], x = x4[J];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * w + 4 * gg + i, d = 16 * J + r;
      a[i] += sb[m] * bu[i];
      if (m < ch.M && d < g.dk) stf(dK, (row0 + m) * g.dk + d, a[i]);
      // row sum over the 16 columns of this tile
      rowp[i] += mg_group_sum<16>(sU[m * LD + 16 * J + r] * x[i]);
    }
  }
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sdb[8][16 * w + 4 * gg + i] = rowp[i];
  }
  // dV = G.
  for (int e = threadIdx.x; e < DN * DN; e += NT) {
    const int m = e >> 6, j = e & 63;
    if (m < ch.M && j < g.dv) stf(dV, (row0 + m) * g.dv + j, sG[m * LD + j]);
  }
  __syncthreads();
  if (threadIdx.x < ch.M) {
    const int m = threadIdx.x;
    float acc = sdb[8][m];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc += sdb[q][m];
    stf(dbeta, row0 + m, acc);
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
template <typename TI>
int dw_fwd(const void* Q, const void* K, const void* V, const void* beta, const float* H0, void* y,
           float* HT, float* Hb, int64_t BH, const DwGeom& g, void* ws, size_t ws_bytes,
           hipStream_t stream) {
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 3 * mb) return MG_ERR_WORKSPACE;
  float* Wm = (float*)ws;
  float* U0m = (float*)((char*)ws + mb);
  float* Pm = (float*)((char*)ws + 2 * mb);
  hipLaunchKernelGGL(dw_fwd_prep<TI>, dim3(g.nc, (unsigned)BH), dim3(NT), 0, stream,
                     (const TI*)Q, (const TI*)K, (const TI*)V, (const TI*)beta, Wm, U0m, Pm,
                     dw_inv_slots(Hb, BH, g), g);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dw_fwd_chain<TI>, dim3(chain_grid(BH, g)), dim3(NT), 0, stream,
                     (const TI*)Q, (const TI*)K, (const TI*)beta, H0, Wm, U0m, Pm, (TI*)y, HT, Hb,
                     g, BH);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

template <typename TI>
int dw_bwd(const void* Q, const void* K, const void* V, const void* beta, const float* Hb,
           const void* dy, const float* dHT, void* dQ, void* dK, void* dV, void* dbeta,
           float* dH0, int64_t BH, const DwGeom& g, void* ws, size_t ws_bytes,
           hipStream_t stream) {
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 6 * mb) return MG_ERR_WORKSPACE;
  float* Um = (float*)ws;
  float* Em = (float*)((char*)ws + mb);
  float* G0m = (float*)((char*)ws + 2 * mb);
  float* QdYm = (float*)((char*)ws + 3 * mb);
  float* Gm = (float*)((char*)ws + 4 * mb);
  float* dHn = (float*)((char*)ws + 5 * mb);
  hipLaunchKernelGGL(dw_bwd_prep<TI>, dim3(g.nc, (unsigned)BH), dim3(NT), 0, stream,
                     (const TI*)Q, (const TI*)K, (const TI*)V, (const TI*)beta, (const TI*)dy, Hb,
                     dw_inv_slots(Hb, BH, g), Um, Em, G0m, QdYm, g);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dw_bwd_chain<TI>, dim3(chain_grid(BH, g)), dim3(NT), 0, stream,
                     (const TI*)K, dHT, Em, G0m, QdYm, Gm, dHn, dH0, g, BH);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dw_bwd_grads<TI>, dim3(g.nc, (unsigned)BH), dim3(NT), 0, stream,
                     (const TI*)Q, (const TI*)K, (const TI*)beta, (const TI*)dy, Hb, dHn, Um, Gm,
                     (TI*)dQ, (TI*)dK, (TI*)dV, (TI*)dbeta, g);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

size_t mg_delta_workspace_bytes(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv,
                                int chunk) {
  DwGeom g;
  int64_t BH;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return 256;
  return 6 * dw_mat_bytes(BH, g);
}

size_t mg_delta_state_bytes(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv, int chunk) {
  DwGeom g;
  int64_t BH;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return 0;
  return dw_state_bytes(BH, g);
}

int mg_delta_fwd(const void* Q, const void* K, const void* V, const void* beta, const float* H0,
                 void* y, float* HT, float* Hbound, int64_t B, int64_t H, int64_t T, int nh, int dk,
                 int dv, int chunk, int dtype, void* ws, size_t ws_bytes, hipStream_t stream) {
  DwGeom g;
  int64_t BH;
  if (!Q || !K || !V || !beta || !H0 || !y || !HT || !Hbound || !ws) return MG_ERR_ARG;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return MG_ERR_ARG;
  if (!al16(ws) || !al16(Hbound)) return MG_ERR_ARG;
  if (dtype == 0)
    return dw_fwd<float>(Q, K, V, beta, H0, y, HT, Hbound, BH, g, ws, ws_bytes, stream);
  if (dtype == 1)
    return dw_fwd_bf16(Q, K, V, beta, H0, y, HT, Hbound, BH, g, ws, ws_bytes, stream);
  return MG_ERR_ARG;
}

int mg_delta_bwd(const void* Q, const void* K, const void* V, const void* beta,
                 const float* Hbound, const void* dy, const float* dHT, void* dQ, void* dK,
                 void* dV, void* dbeta, float* dH0, int64_t B, int64_t H, int64_t T, int nh,
                 int dk, int dv, int chunk, int dtype, void* ws, size_t ws_bytes,
                 hipStream_t stream) {
  DwGeom g;
  int64_t BH;
  if (!Q || !K || !V || !beta || !Hbound || !dy || !dHT || !dQ || !dK || !dV || !dbeta || !dH0 ||
      !ws)
    return MG_ERR_ARG;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return MG_ERR_ARG;
  if (!al16(ws) || !al16(Hbound)) return MG_ERR_ARG;
  if (dtype == 0)
    return dw_bwd<float>(Q, K, V, beta, Hbound, dy, dHT, dQ, dK, dV, dbeta, dH0, BH, g, ws,
                         ws_bytes, stream);
  if (dtype == 1)
    return dw_bwd_bf16(Q, K, V, beta, Hbound, dy, dHT, dQ, dK, dV, dbeta, dH0, BH, g, ws,
                       ws_bytes, stream);
  return MG_ERR_ARG;
}

}  // extern "C"

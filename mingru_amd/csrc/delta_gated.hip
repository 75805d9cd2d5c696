// DeltaMinGRU decay-gated chunked-WY delta rule, forward and backward (gfx950, MFMA).
//
// Recurrence per head (reference src/mingru/min_gru.py:3611-3688, step): each
// token t first decays the state, then runs its nh micro-steps undecayed,
//     H <- gamma_t H;   H <- H - beta_m k_m (k_m^T H) + beta_m k_m v_m^T;   y_t = H_t^T q_t,
// with l_t = log gamma_t <= 0 given per (head, token).  Chunked form (reference
// _forward_chunked_gated, :3257-3448, which has no kernel there): within a chunk
// of C tokens every decay factor is exp of a span sum
//     span(t, t') = sum_{s=t'+1..t} l_s,   E[t][t'] = exp(span(t, t')) (t' <= t, else 0),
//     Lc_t = sum_{s<=t} l_s,  p_m = exp(Lc_tau(m)),  ptok_t = exp(Lc_t),
//     a_m = E[C-1][tau(m)],   PC = exp(Lc_{C-1}),     tau(m) = m / nh,
// each a sum of its own terms (never a difference of running sums).
// With Hc the state entering the chunk:
//     L  = strict_lower(K K^T) * beta_col * E[tau(i)][tau(j)],  Tm = I + L
//     U  = Tm^-1 (V - diag(p) K Hc) = U0 - W Hc,   U0 = Tm^-1 V,  W = Tm^-1 diag(p) K
//     P  = (Q K^T) * beta_col * E[t][tau(m)]
//     y  = diag(ptok) Q Hc + P U,     H_next = PC Hc + K^T diag(a beta) U.
// Backward, with dHn the gradient of the state leaving the chunk:
//     G   = Tm^-T (P^T dy + diag(a beta) K dHn) = G0 + E_ dHn   (E_ = Tm^-T diag(a beta) K)
//     dHc = PC dHn + (diag(ptok) Q)^T dy - (diag(p) K)^T G,      dV = G
//     dQ  = diag(ptok) dy Hc^T + dS K,          dS = (dy U^T) * beta_col * E_read
//     dK  = dS^T Q - diag(p) G Hc^T + dKK K + dKK^T K + diag(a beta) U dHn^T,
//           dKK = (-G U^T) * beta_col * E_mm (strict)
//     dbeta_m = sum_t dP S E_read + sum_i dT KK E_mm + a_m sum_j U (K dHn)
// and the decay gradient through every factor's log: with F[t][t'] the summed
// d/d span(t, t') and f[t] the summed d/d Lc_t,
//     dl_s = sum_{t >= s} ( f[t] + sum_{t' < s} F[t][t'] ),
// taken as wave-level prefix scans along the rows of F and per-wave column sums
// added in a fixed order.
//
// These kernels mirror delta_wy.hip (fp32 operands on v_mfma_f32_16x16x4_f32) and
// serve fp32 inputs; bf16 inputs (any nh) run the gated instantiations of the
// bf16-MFMA kernels (mg_delta_bf16.h), chosen by the dtype tag of the entry points.  The per-chunk decay vectors (a beta, ptok, p,
// PC) travel in a small vector region after the workspace matrices.
#include "mg_delta_bf16.h"

namespace {

using namespace mgd;

// L = strict_lower(K K^T) * beta_col * E[tau(i)][tau(j)] into sL; wave w builds block-row w.
__device__ __forceinline__ void build_L_gated(const float* sK, const float* sb, const float* sE,
                                              int nh, float* sL) {
  const int w = wave_id(), lane = lane_id(), r = lane & 15, g = lane >> 4;
  floatx4 acc[4];
  zero_row4(acc);
  mma_row4<64>(acc, sK + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
  for (int J = 0; J < 4; ++J) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * w + 4 * g + i, col = 16 * J + r;
      // formed first, then picked: a masked arm that reads LDS becomes a branch that
      // waits for the read on its own
      const float v = acc[J][i] * sb[col] * sE[(row / nh) * LD + col / nh];
      sL[row * LD + col] = col < row ? v : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void dg_fwd_prep(const float* __restrict__ Q,
                                                  const float* __restrict__ K,
                                                  const float* __restrict__ V,
                                                  const float* __restrict__ beta,
                                                  const float* __restrict__ lg,
                                                  float* __restrict__ Wo, float* __restrict__ U0o,
                                                  float* __restrict__ Po, float* __restrict__ vo,
                                                  float* __restrict__ To, DwGeom g) {
  __shared__ float sK[DN * LD], sV[DN * LD], sL[DN * LD], sT[DN * LD], sE[DN * LD];
  __shared__ float sY[2 * 32 * LDS16];
  __shared__ float sb[DN], sl[DN], sLc[DN], sp[DN], sab[DN];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  Tile<float> tk, tv, tq;
  tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
  tv.load(V + row0 * g.dv, ch.M, g.dv, g.dv);
  tq.load(Q + (bh * g.T + ch.t0) * g.dk, ch.Ct, g.dk, g.dk);
  const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
  const float lv = ld_l(lg, bh, g, ch);
  tk.store(sK);
  tv.store(sV);
  sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
  sl[threadIdx.x & (DN - 1)] = lv;
  __syncthreads();
  decay_tables<NT>(sl, sE);
  decay_vectors(sl, sb, ch, g.nh, sLc, sp, sab);
  __syncthreads();
  build_L_gated(sK, sb, sE, g.nh, sL);
  __syncthreads();
  unit_lower_inverse(sL, sT, sY);  // ends with a barrier
  tq.store(sL);  // sL is free: Q goes there for P
  write_vectors(vo + ((size_t)bh * g.nc + c) * VECN, sLc, sp, sab, ch);
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  store_inv_packed<NT>(To + mat, sT);  // for the backward preparation kernel
  __syncthreads();
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  {
    floatx4 sp4[4];
    zero_row4(sp4);
    mma_row4<64>(sp4, sL + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, m = 16 * J + r;
        const float v = sp4[J][i] * sb[m] * sE[t * LD + m / g.nh];  // formed first, then picked
        sp4[J][i] = (m < (t + 1) * g.nh) ? v : 0.f;
      }
      acc_store_ws(sp4[J], Po + mat + 16 * w * DN + 16 * J);
    }
  }
  __syncthreads();  // every wave is done with the unscaled K
  for (int e = threadIdx.x; e < DN * DN; e += NT) {
    const int i = e >> 6, j = e & 63;
    sK[i * LD + j] *= sp[i];
  }
  __syncthreads();
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
}

__device__ __forceinline__ void load16g(float (&a)[16], const float* p) {
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
__device__ __forceinline__ floatx4 mma_regg(floatx4 acc, const float (&a)[16], const float* b,
                                            int brs, float sa) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 16; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sa * a[s], b[(16 * g + s) * brs + r], acc, 0, 0, 0);
  return acc;
}

__global__ __launch_bounds__(NT) void dg_fwd_chain(const float* __restrict__ Q,
                                                   const float* __restrict__ K,
                                                   const float* __restrict__ H0,
                                                   const float* __restrict__ Wm,
                                                   const float* __restrict__ U0m,
                                                   const float* __restrict__ Pm,
                                                   const float* __restrict__ vm,
                                                   float* __restrict__ y, float* __restrict__ HT,
                                                   float* __restrict__ Hb, DwGeom g, int64_t BH) {
  __shared__ float sK[2][DN * LD], sQ[2][DN * LD];
  __shared__ float sab[2][DN];
  __shared__ float sH[DN * LDS16], sU[DN * LDS16];
  int64_t bh;
  int col0;
  if (!chain_slot(g, BH, bh, col0)) return;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int col = col0 + r;
  floatx4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    h[i] = ldf_or0(H0, (bh * g.dk + d) * g.dv + col, d < g.dk && col < g.dv);
  }
  Tile<float> tk, tq;
  float abv, pcv, wa[16], pa[16];
  floatx4 u0, ptv;
  auto fetch = [&](int c) {
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    const float* vv = vm + ((size_t)bh * g.nc + c) * VECN;
    const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tq.load(Q + (bh * g.T + ch.t0) * g.dk, ch.Ct, g.dk, g.dk);
    abv = vv[V_AB + (threadIdx.x & (DN - 1))];  // every wave loads the same 64 values
    pcv = ld_uniform_v(vv + V_PC);
#pragma unroll
    for (int i = 0; i < 4; ++i) ptv[i] = vv[V_PT + 16 * w + 4 * gg + i];
    load16g(wa, Wm + mat + (16 * w + r) * DN + 16 * gg);
    load16g(pa, Pm + mat + (16 * w + r) * DN + 16 * gg);
    u0 = acc_load_ws(U0m + mat + 16 * w * DN + col0);
  };
  fetch(0);
  for (int c = 0; c < g.nc; ++c) {
    const int buf = c & 1;
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    tk.store(sK[buf]);
    tq.store(sQ[buf]);
    sab[buf][threadIdx.x & (DN - 1)] = abv;  // and stores them: no branch to wait in
    float wc[16], pc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      wc[i] = wa[i];
      pc[i] = pa[i];
    }
    floatx4 u = u0;
    const floatx4 pt = ptv;
    const float PC = pcv;
    if (c + 1 < g.nc) fetch(c + 1);
    acc_store_lds(h, sH + 16 * w * LDS16, LDS16);
    acc_store_ws(h, Hb + mat + 16 * w * DN + col0);
    __syncthreads();
    u = mma_regg(u, wc, sH, LDS16, -1.f);  // U = U0 - W H
    acc_store_lds(u, sU + 16 * w * LDS16, LDS16);
    floatx4 yy = mma<64>(zero4(), sQ[buf] + 16 * w * LD, LD, 1, sH, LDS16, 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) yy[i] *= pt[i];  // diag(ptok) Q H
    __syncthreads();
    yy = mma_regg(yy, pc, sU, LDS16, 1.f);  // + P U
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * gg + i;
      if (t < ch.Ct && col < g.dv) y[(bh * g.T + ch.t0 + t) * g.dv + col] = yy[i];
    }
    // H = PC H + K^T (a beta U): A[i][m] = a_m beta_m K[m][16w + i].
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] *= PC;
    {
      const float* kb = sK[buf];
      const float* ab = sab[buf];
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const int m = 16 * gg + s;
        h = __builtin_amdgcn_mfma_f32_16x16x4f32(ab[m] * kb[m * LD + 16 * w + r],
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
__global__ __launch_bounds__(NT) void dg_bwd_prep(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ beta, const float* __restrict__ lg, const float* __restrict__ dy,
    const float* __restrict__ Hb, const float* __restrict__ Tin, float* __restrict__ Uo,
    float* __restrict__ Eo, float* __restrict__ G0o, float* __restrict__ QdYo,
    float* __restrict__ vo, DwGeom g) {
  __shared__ float sK[DN * LD], sV[DN * LD], sL[DN * LD], sT[DN * LD], sX[DN * LD];
  __shared__ float sQ[DN * LD], sD[DN * LD], sE[DN * LD];
  __shared__ float sb[DN], sl[DN], sLc[DN], sp[DN], sab[DN], spt[DN];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  {
    Tile<float> tk, tv, tq, td, th;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tv.load(V + row0 * g.dv, ch.M, g.dv, g.dv);
    th.load(Hb + mat, g.dk, g.dv, DN);
    tq.load(Q + (bh * g.T + ch.t0) * g.dk, ch.Ct, g.dk, g.dk);
    td.load(dy + (bh * g.T + ch.t0) * g.dv, ch.Ct, g.dv, g.dv);
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    const float lv = ld_l(lg, bh, g, ch);
    tk.store(sK);
    tv.store(sV);
    th.store(sX);
    tq.store(sQ);
    td.store(sD);
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
    sl[threadIdx.x & (DN - 1)] = lv;
    load_inv_packed<NT>(sT, Tin + mat);  // T = (I + L)^-1 as the forward formed it
  }
  __syncthreads();
  decay_tables<NT>(sl, sE);
  decay_vectors(sl, sb, ch, g.nh, sLc, sp, sab, spt);
  __syncthreads();
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  // R = V - diag(p) K Hc in place in sV (tile (w, J) read and written by wave w only).
  {
    floatx4 kh[4];
    zero_row4(kh);
    mma_row4<64>(kh, sK + 16 * w * LD, LD, 1, sX, LD, 1, 16);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      floatx4 acc = acc_load_lds(sV + 16 * w * LD + 16 * J, LD);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(-sp[16 * w + 4 * gg + i], kh[J][i], acc[i]);
      acc_store_lds(acc, sV + 16 * w * LD + 16 * J, LD);
    }
  }
  write_vectors(vo + ((size_t)bh * g.nc + c) * VECN, sLc, sp, sab, ch);
  __syncthreads();
  // U = Tm^-1 R; P = (Q K^T) * beta_col * E_read into sL (free).
  {
    floatx4 u[4], sp4[4];
    zero_row4(u);
    zero_row4(sp4);
    mma_row4<64>(u, sT + 16 * w * LD, LD, 1, sV, LD, 1, 16);
    mma_row4<64>(sp4, sQ + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      acc_store_ws(u[J], Uo + mat + 16 * w * DN + 16 * J);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, m = 16 * J + r;
        const float v = sp4[J][i] * sb[m] * sE[t * LD + m / g.nh];  // formed first, then picked
        sp4[J][i] = (m < (t + 1) * g.nh) ? v : 0.f;
      }
      acc_store_lds(sp4[J], sL + 16 * w * LD + 16 * J, LD);
    }
  }
  __syncthreads();
  // Q rows by ptok (for Q^T diag(ptok) dy) and K rows by a beta (for E_), once every
  // wave is done with the unscaled operands.
  for (int e = threadIdx.x; e < DN * DN; e += NT) {
    const int i = e >> 6, j = e & 63;
    sQ[i * LD + j] *= spt[i];
    sK[i * LD + j] *= sab[i];
  }
  __syncthreads();
  // D1 = P^T dy into sX (Hc no longer needed); (diag(ptok) Q)^T dy out.
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

__global__ __launch_bounds__(NT) void dg_bwd_chain(const float* __restrict__ K,
                                                   const float* __restrict__ dHT,
                                                   const float* __restrict__ Em,
                                                   const float* __restrict__ G0m,
                                                   const float* __restrict__ QdYm,
                                                   const float* __restrict__ vm,
                                                   float* __restrict__ Gm, float* __restrict__ dHn,
                                                   float* __restrict__ dH0, DwGeom g, int64_t BH) {
  __shared__ float sK[2][DN * LD];
  __shared__ float sp[2][DN];
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
  Tile<float> tk;
  float ea[16], pv, pcv;
  floatx4 g0, qd0;
  auto fetch = [&](int c) {
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    const float* vv = vm + ((size_t)bh * g.nc + c) * VECN;
    tk.load(K + (bh * g.T + ch.t0) * g.nh * g.dk, ch.M, g.dk, g.dk);
    load16g(ea, Em + mat + (16 * w + r) * DN + 16 * gg);
    g0 = acc_load_ws(G0m + mat + 16 * w * DN + col0);
    qd0 = acc_load_ws(QdYm + mat + 16 * w * DN + col0);
    pv = vv[V_P + (threadIdx.x & (DN - 1))];  // every wave loads the same 64 values
    pcv = ld_uniform_v(vv + V_PC);
  };
  fetch(g.nc - 1);
  for (int c = g.nc - 1; c >= 0; --c) {
    const int buf = c & 1;
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    tk.store(sK[buf]);
    sp[buf][threadIdx.x & (DN - 1)] = pv;  // and stores them: no branch to wait in
    float ec[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) ec[i] = ea[i];
    floatx4 gacc = g0;
    const floatx4 qd = qd0;
    const float PC = pcv;
    if (c > 0) fetch(c - 1);
    acc_store_lds(h, sH + 16 * w * LDS16, LDS16);
    acc_store_ws(h, dHn + mat + 16 * w * DN + col0);
    __syncthreads();
    gacc = mma_regg(gacc, ec, sH, LDS16, 1.f);  // G = G0 + E_ dH
    acc_store_ws(gacc, Gm + mat + 16 * w * DN + col0);
    acc_store_lds(gacc, sG + 16 * w * LDS16, LDS16);
    __syncthreads();
    // dH = PC dH + Q^T diag(ptok) dy - (diag(p) K)^T G: A[i][m] = p_m K[m][16w + i].
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = fmaf(PC, h[i], qd[i]);
    const float* kb = sK[buf];
    const float* pb = sp[buf];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int m = 16 * gg + s;
      h = __builtin_amdgcn_mfma_f32_16x16x4f32(-pb[m] * kb[m * LD + 16 * w + r], sG[m * LDS16 + r],
                                               h, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    if (d < g.dk && col < g.dv) dH0[(bh * g.dk + d) * g.dv + col] = h[i];
  }
}

// Row sums over the 16 lanes of a lane group (the 16 columns of a tile).
__device__ __forceinline__ float rowsum16(float p) { return mg_group_sum<16>(p); }

__global__ __launch_bounds__(NT) void dg_bwd_grads(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ beta,
    const float* __restrict__ lg, const float* __restrict__ dy, const float* __restrict__ Hb,
    const float* __restrict__ dHn, const float* __restrict__ Um, const float* __restrict__ Gm,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV,
    float* __restrict__ dbeta, float* __restrict__ dlg, DwGeom g) {
  __shared__ float sK[DN * LD], sQ[DN * LD], sD[DN * LD], sU[DN * LD], sG[DN * LD],
      sH[DN * LD], sX[DN * LD], sE[DN * LD], sF[DN * LD];
  __shared__ float sb[DN], sl[DN], sLc[DN], sp[DN], sab[DN], spt[DN];
  // Log-gradient vectors: [0] d/dLc_t from ptok, [1] d/dLc from p per micro-row,
  // [2] d/dspan(C-1, tau(m)) from a per micro-row, [3] f[t].
  __shared__ float sfv[4][DN];
  // dbeta partials: [0..3] read-term column sums per wave, [4..7] strict-term
  // column sums per wave, [8] a_m * row sums of U * (K dHn).
  __shared__ float sdb[9][DN];
  __shared__ float sred[NT / 64];
  __shared__ float sdl[NT / 64][DN];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const int64_t trow0 = bh * g.T + ch.t0;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  Tile<float> tn;  // dHn, stored once Hc is no longer needed
  {
    Tile<float> tk, tq, td, tu, tg, th;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tq.load(Q + trow0 * g.dk, ch.Ct, g.dk, g.dk);
    td.load(dy + trow0 * g.dv, ch.Ct, g.dv, g.dv);
    tu.load(Um + mat, ch.M, g.dv, DN);
    tg.load(Gm + mat, ch.M, g.dv, DN);
    th.load(Hb + mat, g.dk, g.dv, DN);
    tn.load(dHn + mat, g.dk, g.dv, DN);
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    const float lv = ld_l(lg, bh, g, ch);
    tk.store(sK);
    tq.store(sQ);
    td.store(sD);
    tu.store(sU);
    tg.store(sG);
    th.store(sH);
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
    sl[threadIdx.x & (DN - 1)] = lv;
  }
  __syncthreads();
  decay_tables<NT>(sl, sE);
  decay_vectors(sl, sb, ch, g.nh, sLc, sp, sab, spt);
  // PC term: <dHn, Hc>, with dHn in this thread's tile registers and Hc in sH.
  {
    const float part = mg_group_sum<64>(tn.dot(sH));
    if (lane == 0) sred[w] = part;
  }
  __syncthreads();
  // Phase 1.  S = Q K^T, dP = dy U^T (rows tokens, cols micro-rows); Q Hc, K Hc for
  // the ptok and p log-gradients.
  {
    floatx4 s4[4], dp4[4];
    zero_row4(s4);
    zero_row4(dp4);
    mma_row4<64>(s4, sQ + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
    mma_row4<64>(dp4, sD + 16 * w * LD, LD, 1, sU, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const floatx4 s = s4[J], dp = dp4[J];
      floatx4 ds, db, fr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, m = 16 * J + r;
        const bool rd = m < (t + 1) * g.nh;
        const float e = sE[t * LD + m / g.nh];  // read first, then picked
        const float er = rd ? e : 0.f;
        ds[i] = dp[i] * sb[m] * er;
        db[i] = dp[i] * s[i] * er;
        fr[i] = db[i] * sb[m];
      }
      acc_store_lds(ds, sX + 16 * w * LD + 16 * J, LD);
      acc_store_lds(fr, sF + 16 * w * LD + 16 * J, LD);
      put_colsum(db, sdb[w], 16 * J + r);
    }
  }
  {
    floatx4 qh4[4], kh4[4];
    zero_row4(qh4);
    zero_row4(kh4);
    mma_row4<64>(qh4, sQ + 16 * w * LD, LD, 1, sH, LD, 1, 16);
    mma_row4<64>(kh4, sK + 16 * w * LD, LD, 1, sH, LD, 1, 16);
    float fq[4] = {0.f, 0.f, 0.f, 0.f}, fp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int J = 0; J < 4; ++J) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * w + 4 * gg + i, cl = 16 * J + r;
        fq[i] += rowsum16(sD[row * LD + cl] * qh4[J][i]);
        fp[i] += rowsum16(sG[row * LD + cl] * kh4[J][i]);
      }
    }
    if (r == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * w + 4 * gg + i;
        sfv[0][row] = spt[row] * fq[i];
        sfv[1][row] = -sp[row] * fp[i];
      }
    }
  }
  __syncthreads();
  // Phase 2.  dQ = diag(ptok) dy Hc^T + dS K; dK (registers) = dS^T Q - diag(p) G Hc^T.
  floatx4 dk[4];
  {
    floatx4 q[4];
    zero_row4(q);
    mma_row4<64>(q, sD + 16 * w * LD, LD, 1, sH, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int i = 0; i < 4; ++i) q[J][i] *= spt[16 * w + 4 * gg + i];
    mma_row4<64>(q, sX + 16 * w * LD, LD, 1, sK, LD, 1, 16);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * gg + i, d = 16 * J + r;
        if (t < ch.Ct && d < g.dk) dQ[(trow0 + t) * g.dk + d] = q[J][i];
      }
    }
    floatx4 gh[4];
    zero_row4(dk);
    zero_row4(gh);
    mma_row4<64>(dk, sX + 16 * w, 1, LD, sQ, LD, 1, 16);
    mma_row4<64>(gh, sG + 16 * w * LD, LD, 1, sH, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int i = 0; i < 4; ++i) dk[J][i] = fmaf(-sp[16 * w + 4 * gg + i], gh[J][i], dk[J][i]);
  }
  __syncthreads();
  // Phase 3.  dT = -G U^T, KK = K K^T; dKK = dT * beta_col * E_mm (strict) into sX, the
  // micro-level span gradients dT * L into sD (dy is no longer needed).  dHn into sH.
  {
    floatx4 dt4[4], kk4[4];
    zero_row4(dt4);
    zero_row4(kk4);
    mma_row4<64>(dt4, sG + 16 * w * LD, LD, 1, sU, 1, LD, 16 * LD, -1.f);
    mma_row4<64>(kk4, sK + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const floatx4 dt = dt4[J], kk = kk4[J];
      floatx4 dkk, db, ft;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * w + 4 * gg + i, j = 16 * J + r;
        const float e = sE[(m / g.nh) * LD + j / g.nh];  // read first, then picked
        const float em = j < m ? e : 0.f;
        dkk[i] = dt[i] * sb[j] * em;
        db[i] = dt[i] * kk[i] * em;
        ft[i] = db[i] * sb[j];
      }
      acc_store_lds(dkk, sX + 16 * w * LD + 16 * J, LD);
      acc_store_lds(ft, sD + 16 * w * LD + 16 * J, LD);
      put_colsum(db, sdb[4 + w], 16 * J + r);
    }
  }
  tn.store(sH);
  __syncthreads();
  // Phase 4.  dK += dKK K + dKK^T K + diag(a beta) U dHn^T; rows of U * (K dHn) give
  // the Hn terms of dbeta (times a) and of the decay gradient (times a beta).
  {
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
        a[i] = fmaf(sab[m], bu[i], a[i]);
        if (m < ch.M && d < g.dk) dK[(row0 + m) * g.dk + d] = a[i];
        rowp[i] += rowsum16(sU[m * LD + 16 * J + r] * x[i]);
      }
    }
    if (r == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * w + 4 * gg + i;
        const float v = sE[(ch.Ct - 1) * LD + m / g.nh] * rowp[i];  // formed first, then picked
        sdb[8][m] = m < ch.M ? v : 0.f;
        sfv[2][m] = sab[m] * rowp[i];
      }
    }
  }
  // dV = G.
  for (int e = threadIdx.x; e < DN * DN; e += NT) {
    const int m = e >> 6, j = e & 63;
    if (m < ch.M && j < g.dv) dV[(row0 + m) * g.dv + j] = sG[m * LD + j];
  }
  __syncthreads();
  // Phase 5.  dbeta; token-level span gradients F[t][t'] (t' < t) into sQ and f[t].
  if (threadIdx.x < ch.M) {
    const int m = threadIdx.x;
    float acc = sdb[8][m];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc += sdb[q][m];
    dbeta[row0 + m] = acc;
  }
  const int nh = g.nh;
  for (int e = threadIdx.x; e < DN * DN; e += NT) {
    const int t = e >> 6, tp = e & 63;
    float v = 0.f;
    if (t < ch.Ct && tp < t) {
      for (int j = 0; j < nh; ++j) v += sF[t * LD + tp * nh + j];
      for (int a = 0; a < nh; ++a)
        for (int b = 0; b < nh; ++b) v += sD[(t * nh + a) * LD + tp * nh + b];
      if (t == ch.Ct - 1)
        for (int j = 0; j < nh; ++j) v += sfv[2][tp * nh + j];
    }
    sQ[t * LD + tp] = v;
  }
  if (threadIdx.x < DN) {
    const int t = threadIdx.x;
    float f = 0.f;
    if (t < ch.Ct) {
      f = sfv[0][t];
      for (int a = 0; a < nh; ++a) f += sfv[1][t * nh + a];
      if (t == ch.Ct - 1) {
        float pcs = 0.f;
#pragma unroll
        for (int q = 0; q < NT / 64; ++q) pcs += sred[q];
        f = fmaf(expf(sLc[t]), pcs, f);
      }
    }
    sfv[3][t] = f;
  }
  __syncthreads();
  // dl_s = sum_{t >= s} (f[t] + sum_{t' < s} F[t][t']).  Wave w scans rows
  // 16w..16w+15 of F: an exclusive prefix scan along each row (lane s), then each
  // lane adds the rows t >= s; the four wave partials are summed in a fixed order.
  {
    float acc = 0.f;
    for (int rr = 0; rr < DN / (NT / 64); ++rr) {
      const int t = (DN / (NT / 64)) * w + rr;
      const float ex = mg_wave_prev(mg_wave_prefix_sum(sQ[t * LD + lane]));
      if (t >= lane && t < ch.Ct) acc += sfv[3][t] + ex;
    }
    sdl[w][lane] = acc;
  }
  __syncthreads();
  if (threadIdx.x < ch.Ct) {
    const int s = threadIdx.x;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < NT / 64; ++q) acc += sdl[q][s];
    dlg[trow0 + s] = acc;
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
size_t dg_vec_bytes(int64_t BH, const DwGeom& g) {
  return (size_t)BH * g.nc * VECN * sizeof(float);
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// ---------------------------------------------------------------------------
// bf16 inputs: the gated instantiations of the bf16-MFMA kernels
// ---------------------------------------------------------------------------
namespace mgd {

int dw_fwd_bf16_gated(const void* Q, const void* K, const void* V, const void* beta,
                      const float* lg, const float* H0, void* y, float* HT, float* Hb, int64_t BH,
                      const DwGeom& g, void* ws, size_t ws_bytes, hipStream_t stream) {
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 4 * mb + (size_t)BH * g.nc * VECN * sizeof(float)) return MG_ERR_WORKSPACE;
  float* Am = (float*)ws;  // split pair
  float* Bm = (float*)((char*)ws + mb);
  float* Qem = (float*)((char*)ws + 2 * mb);  // split pair
  float* Pum = (float*)((char*)ws + 3 * mb);
  float* vm = (float*)((char*)ws + 4 * mb);
  hipLaunchKernelGGL(dwb_fwd_prep<true>, dim3(g.nc, (unsigned)BH), dim3(NTB), 0, stream,
                     (const u16*)Q, (const u16*)K, (const u16*)V, (const u16*)beta, lg, Am, Bm,
                     Qem, Pum, vm, dw_inv_slots(Hb, BH, g), g);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dwb_fwd_chain<true>, dim3(chain_grid(BH, g)), dim3(NT), 0, stream, H0, Am, Bm,
                     Qem, Pum, vm, (u16*)y, HT, Hb, g, BH);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

int dw_bwd_bf16_gated(const void* Q, const void* K, const void* V, const void* beta,
                      const float* lg, const float* Hb, const void* dy, const float* dHT, void* dQ,
                      void* dK, void* dV, void* dbeta, float* dlg, float* dH0, int64_t BH,
                      const DwGeom& g, void* ws, size_t ws_bytes, hipStream_t stream) {
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 6 * mb + (size_t)BH * g.nc * VECN * sizeof(float)) return MG_ERR_WORKSPACE;
  float* Um = (float*)ws;
  float* Em = (float*)((char*)ws + mb);  // split pair
  float* G0m = (float*)((char*)ws + 2 * mb);
  float* Apm = (float*)((char*)ws + 3 * mb);  // split pair
  float* bpm = (float*)((char*)ws + 4 * mb);
  float* dHn = (float*)((char*)ws + 5 * mb);
  float* vm = (float*)((char*)ws + 6 * mb);
  const dim3 pgrid(g.nc, (unsigned)BH);
  const u16 *q = (const u16*)Q, *k = (const u16*)K, *b = (const u16*)beta, *d = (const u16*)dy;
  const int rc = dwb_bwd_prep_launch(true, Q, K, V, beta, lg, dy, Hb, Um, Em, G0m, Apm, bpm, vm, BH,
                                     g, stream);
  if (rc != MG_OK) return rc;
  hipLaunchKernelGGL(dwb_bwd_chain<true>, dim3(chain_grid(BH, g)), dim3(NT), 0, stream, dHT, Apm,
                     bpm, vm, dHn, dH0, g, BH);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dwb_bwd_grads<true>, pgrid, dim3(NTB), 0, stream, q, k, b, lg, d, Hb, dHn, Um,
                     Em, G0m, (u16*)dQ, (u16*)dK, (u16*)dV, (u16*)dbeta, dlg, g);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

}  // namespace mgd

extern "C" {

size_t mg_delta_gated_workspace_bytes(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv,
                                      int chunk) {
  DwGeom g;
  int64_t BH;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return 256;
  return 6 * dw_mat_bytes(BH, g) + dg_vec_bytes(BH, g);
}

int mg_delta_gated_fwd(const void* Q, const void* K, const void* V, const void* beta,
                       const float* log_gamma, const float* H0, void* y, float* HT,
                       float* Hbound, int64_t B, int64_t H, int64_t T, int nh, int dk, int dv,
                       int chunk, int dtype, void* ws, size_t ws_bytes, hipStream_t stream) {
  DwGeom g;
  int64_t BH;
  if (!Q || !K || !V || !beta || !log_gamma || !H0 || !y || !HT || !Hbound || !ws)
    return MG_ERR_ARG;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return MG_ERR_ARG;
  if (!al16(ws) || !al16(Hbound)) return MG_ERR_ARG;
  if (dtype == 1) {
    return dw_fwd_bf16_gated(Q, K, V, beta, log_gamma, H0, y, HT, Hbound, BH, g, ws, ws_bytes,
                             stream);
  }
  if (dtype != 0) return MG_ERR_ARG;
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 3 * mb + dg_vec_bytes(BH, g)) return MG_ERR_WORKSPACE;
  float* Wm = (float*)ws;
  float* U0m = (float*)((char*)ws + mb);
  float* Pm = (float*)((char*)ws + 2 * mb);
  float* vm = (float*)((char*)ws + 3 * mb);
  const float *q = (const float*)Q, *k = (const float*)K, *v = (const float*)V,
              *b = (const float*)beta;
  hipLaunchKernelGGL(dg_fwd_prep, dim3(g.nc, (unsigned)BH), dim3(NT), 0, stream, q, k, v, b,
                     log_gamma, Wm, U0m, Pm, vm, dw_inv_slots(Hbound, BH, g), g);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dg_fwd_chain, dim3(chain_grid(BH, g)), dim3(NT), 0, stream, q, k, H0, Wm,
                     U0m, Pm, vm, (float*)y, HT, Hbound, g, BH);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

int mg_delta_gated_bwd(const void* Q, const void* K, const void* V, const void* beta,
                       const float* log_gamma, const float* Hbound, const void* dy,
                       const float* dHT, void* dQ, void* dK, void* dV, void* dbeta,
                       float* dlog_gamma, float* dH0, int64_t B, int64_t H, int64_t T, int nh,
                       int dk, int dv, int chunk, int dtype, void* ws, size_t ws_bytes,
                       hipStream_t stream) {
  DwGeom g;
  int64_t BH;
  if (!Q || !K || !V || !beta || !log_gamma || !Hbound || !dy || !dHT || !dQ || !dK || !dV ||
      !dbeta || !dlog_gamma || !dH0 || !ws)
    return MG_ERR_ARG;
  if (!dw_geom(B, H, T, nh, dk, dv, chunk, g, BH)) return MG_ERR_ARG;
  if (!al16(ws) || !al16(Hbound)) return MG_ERR_ARG;
  if (dtype == 1) {
    return dw_bwd_bf16_gated(Q, K, V, beta, log_gamma, Hbound, dy, dHT, dQ, dK, dV, dbeta,
                             dlog_gamma, dH0, BH, g, ws, ws_bytes, stream);
  }
  if (dtype != 0) return MG_ERR_ARG;
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 6 * mb + dg_vec_bytes(BH, g)) return MG_ERR_WORKSPACE;
  float* Um = (float*)ws;
  float* Em = (float*)((char*)ws + mb);
  float* G0m = (float*)((char*)ws + 2 * mb);
  float* QdYm = (float*)((char*)ws + 3 * mb);
  float* Gm = (float*)((char*)ws + 4 * mb);
  float* dHn = (float*)((char*)ws + 5 * mb);
  float* vm = (float*)((char*)ws + 6 * mb);
  const float *q = (const float*)Q, *k = (const float*)K, *v = (const float*)V,
              *b = (const float*)beta, *d = (const float*)dy;
  hipLaunchKernelGGL(dg_bwd_prep, dim3(g.nc, (unsigned)BH), dim3(NT), 0, stream, q, k, v, b,
                     log_gamma, d, Hbound, dw_inv_slots(Hbound, BH, g), Um, Em, G0m, QdYm, vm, g);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dg_bwd_chain, dim3(chain_grid(BH, g)), dim3(NT), 0, stream, k, dHT, Em, G0m,
                     QdYm, vm, Gm, dHn, dH0, g, BH);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dg_bwd_grads, dim3(g.nc, (unsigned)BH), dim3(NT), 0, stream, q, k, b,
                     log_gamma, d, Hbound, dHn, Um, Gm, (float*)dQ, (float*)dK, (float*)dV,
                     (float*)dbeta, dlog_gamma, g);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

}  // extern "C"

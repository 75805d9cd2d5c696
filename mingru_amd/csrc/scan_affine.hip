// Block-matrix affine scans: matrix_scan (k=2, v=1) and matrix_affine_scan
// (k in {1,2,4,8,16}, v in {1,2,4,8,16}), fwd + bwd.  The kernels below take
// k <= 4; 8x8 and 16x16 blocks run on the matrix cores (scan_affine_mfma.hip).
//
// Recurrence per plane (reference src/mingru/min_gru.py:1513-1655):
//   Abar_t = A_t Abar_{t-1},  Bbar_t = A_t Bbar_{t-1} + B_t,  Abar_0 = I, Bbar_0 = 0.
// Adjoint (reference kernel src/mingru/triton_scans.py:824-959 derives the same):
//   X_t = G_t + A_{t+1}^T X_{t+1}       (for both the Abar and Bbar streams)
//   dA_t = XA_t Abar_{t-1}^T + XB_t Bbar_{t-1}^T,   dB_t = XB_t.
//
// One thread owns one plane (b, i) and keeps the k x k block product in
// registers.  Planes of one (b, t) are contiguous in memory, so a wave reads
// 64 consecutive planes per time step (1 KiB for k = 2).  Time is split into
// chunks of WAVES*TSUB steps per workgroup; chunks are chained with the same
// decoupled look-back as the elementwise scans, carrying the affine map
// (P, L): S -> P S + L of each chunk.  Inside a workgroup the waves combine
// their sub-chunk maps through one LDS buffer in time order.
//
// For k <= 2 with at most two offset columns every input of the thread's
// sub-chunk stays in registers between the aggregate pass and the final pass
// (one HBM read).  Otherwise the register file cannot hold them: inputs are re-read for the final pass and
// the backward reads the saved forward outputs Abar_{t-1}, Bbar_{t-1}.
#include "mg_affm.h"

#include <algorithm>

namespace {

using namespace mg;

// Chunk shape by block size and direction: waves per workgroup x steps per
// wave.  Longer chunks mean fewer hops in the look-back chain, whose per-hop
// latency (slot round trips that bypass the L2) bounds the 2x2 scans at long T;
// the shapes were chosen by timing on MI355X at B=16, T=4096, n=256.  The 2x2
// forward takes 8 waves since its small held inputs run persistent workgroups with
// two input buffers (16 waves cap a lane at 128 VGPRs, and the second buffer
// spilled there).
template <int K, bool BWD>
constexpr int af_waves() {
  return K == 2 ? 8 : 4;
}

template <int K, bool BWD>
constexpr int af_tsub() {
  return K == 1 ? 16 : 8;
}

// Whether a thread keeps its chunk's inputs in registers for the final pass
// (else it re-reads them).  Holding wins for 1x1 blocks and for 2x2 blocks with
// at most two offset columns; wider 2x2 offsets spill, and re-reading took B=8,
// T=2048, n=256, v=8 from 374/498 us to 319/290 us (fwd/bwd), v=16 from 826/1258
// to 736/644 us.
template <int K, int V>
constexpr bool af_hold() {
  return K == 1 || K * (K + V) <= 8;
}

// Whether the forward runs persistent workgroups with two input buffers: held
// inputs small enough to double (at most 64 floats per buffer).
template <int K, int V>
constexpr bool af_fwd_persistent() {
  return af_hold<K, V>() && K * (K + V) * af_tsub<K, false>() <= 64;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// Forward with the chunk's inputs held in registers, in persistent workgroups
// (mg_persistent's protocol) with two input buffers: the next ticket is shared
// once this chunk's local aggregate is formed, and its inputs load while this
// chunk's carry and outputs run.
template <int K, int V, int TSUB, int WAVES>
__device__ __forceinline__ void affine_fwd_held(const float* __restrict__ A,
                                                const float* __restrict__ Bm,
                                                float* __restrict__ Abar, float* __restrict__ Bbar,
                                                const AfGeom& g, unsigned* header,
                                                mg_slot_t* agg_data, mg_slot_t* incl_data) {
  using RA = float[TSUB][K * K];
  using RB = float[TSUB][K * V];
  const int64_t T = g.T, n = g.n;
  // The thread's TSUB steps of (A_t, B_t) for ticket `ticket` (identity past the end).
  auto load = [&](unsigned ticket, RA& ha, RB& hb) {
    const AfThread th = af_thread_at<false>(g, ticket, 0u);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.ok && t < T) {
        const int64_t row = (th.bb * T + t) * n + th.plane;
        ld<K * K, true>(ha[s], A + row * (K * K));
        ld<K * V, true>(hb[s], Bm + row * (K * V));
      } else {
#pragma unroll
        for (int i = 0; i < K * K; ++i) ha[s][i] = (i / K == i % K) ? 1.f : 0.f;
#pragma unroll
        for (int i = 0; i < K * V; ++i) hb[s][i] = 0.f;
      }
    }
  };
  // Applies step s to x: x <- A_s x + B_s.
  auto step = [&](const RA& ha, const RB& hb, int s, AffM<K, V>& x) {
    AffM<K, V> nx;
#pragma unroll
    for (int i = 0; i < K; ++i) {
#pragma unroll
      for (int j = 0; j < K; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < K; ++m) acc = fmaf(ha[s][i * K + m], x.P[m][j], acc);
        nx.P[i][j] = acc;
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float acc = hb[s][i * V + j];
#pragma unroll
        for (int m = 0; m < K; ++m) acc = fmaf(ha[s][i * K + m], x.L[m][j], acc);
        nx.L[i][j] = acc;
      }
    }
    x = nx;
  };
  // The chunk from its inputs: local aggregate, then `mid` (run by every thread),
  // then the carry and the outputs.
  auto finish = [&](unsigned ticket, unsigned epoch, const RA& ha, const RB& hb, auto&& mid) {
    const AfThread th = af_thread_at<false>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    AffM<K, V> loc, carry, seed;
    affm_identity(loc);
#pragma unroll
    for (int s = 0; s < TSUB; ++s) step(ha, hb, s, loc);
    affm_identity(seed);
    mid();
    af_carry<K, V, WAVES, false>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                 incl_data, carry);
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      step(ha, hb, s, carry);
      const int64_t t = t0 + s;
      if (th.ok && t < T) {
        const int64_t row = (th.bb * T + t) * n + th.plane;
        st<K * K, true>(Abar + row * (K * K), &carry.P[0][0]);
        st<K * V, true>(Bbar + row * (K * V), &carry.L[0][0]);
      }
    }
  };
  __shared__ unsigned s_ticket, s_epoch;
  const unsigned chunks = (unsigned)g.n_lg * (unsigned)g.n_chunks;
  if (threadIdx.x == 0) {
    const unsigned e0 =
        __hip_atomic_load(header + MG_H_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    s_ticket = mg_next_ticket(header, e0, chunks);
    s_epoch = e0;
  }
  __syncthreads();
  unsigned t = s_ticket;
  const unsigned e = s_epoch;
  RA a0, a1;
  RB b0, b1;
  if (t < chunks) load(t, a0, b0);
  auto chunk = [&](unsigned tk, const RA& ha, const RB& hb, RA& nha, RB& nhb) {
    unsigned next = 0u;
    if (threadIdx.x == 0) next = mg_next_ticket(header, e, chunks);
    unsigned tn = 0u;
    finish(tk, e, ha, hb, [&] {
      if (threadIdx.x == 0) s_ticket = next;
      __syncthreads();
      tn = s_ticket;
      if (tn < chunks) load(tn, nha, nhb);
    });
    return tn;
  };
  while (t < chunks) {
    t = chunk(t, a0, b0, a1, b1);
    if (t >= chunks) break;
    t = chunk(t, a1, b1, a0, b0);
  }
}

template <int K, int V, int TSUB, int WAVES>
__global__ __launch_bounds__(MG_WAVE* WAVES) void affine_fwd_kernel(
    const float* __restrict__ A, const float* __restrict__ Bm, float* __restrict__ Abar,
    float* __restrict__ Bbar, AfGeom g, unsigned* header, mg_slot_t* agg_data,
    mg_slot_t* incl_data) {
  constexpr bool HOLD = af_hold<K, V>();
  if constexpr (af_fwd_persistent<K, V>()) {
    affine_fwd_held<K, V, TSUB, WAVES>(A, Bm, Abar, Bbar, g, header, agg_data, incl_data);
    return;
  }
  constexpr int HS = HOLD ? TSUB : 1;
  AfThread th = af_thread<false>(g, header);
  if (!th.valid) return;
  const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
  const int64_t T = g.T, n = g.n;
  auto offA = [&](int64_t t) { return ((th.bb * T + t) * n + th.plane) * (K * K); };
  auto offB = [&](int64_t t) { return ((th.bb * T + t) * n + th.plane) * (K * V); };

  float ha[HS][K * K], hb[HS][K * V];
  auto fetch = [&](int s, float* a, float* b) {
    const int64_t t = t0 + s;
    if (th.ok && t < T) {
      ld<K * K, HOLD>(a, A + offA(t));
      ld<K * V, HOLD>(b, Bm + offB(t));
    } else {
#pragma unroll
      for (int i = 0; i < K * K; ++i) a[i] = (i / K == i % K) ? 1.f : 0.f;
#pragma unroll
      for (int i = 0; i < K * V; ++i) b[i] = 0.f;
    }
  };
  if constexpr (HOLD) {
#pragma unroll
    for (int s = 0; s < TSUB; ++s) fetch(s, ha[s], hb[s]);
  }

  // Local aggregate: S -> A_t S + B_t composed over the sub-chunk.
  AffM<K, V> loc, carry;
  affm_identity(loc);
#pragma unroll
  for (int s = 0; s < TSUB; ++s) {
    float a[K * K], b[K * V];
    if constexpr (HOLD) {
#pragma unroll
      for (int i = 0; i < K * K; ++i) a[i] = ha[s][i];
#pragma unroll
      for (int i = 0; i < K * V; ++i) b[i] = hb[s][i];
    } else {
      fetch(s, a, b);
    }
    AffM<K, V> nx;
#pragma unroll
    for (int i = 0; i < K; ++i) {
#pragma unroll
      for (int j = 0; j < K; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < K; ++m) acc = fmaf(a[i * K + m], loc.P[m][j], acc);
        nx.P[i][j] = acc;
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float acc = b[i * V + j];
#pragma unroll
        for (int m = 0; m < K; ++m) acc = fmaf(a[i * K + m], loc.L[m][j], acc);
        nx.L[i][j] = acc;
      }
    }
    loc = nx;
  }
  AffM<K, V> seed;
  affm_identity(seed);
  af_carry<K, V, WAVES, false>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data, incl_data, carry);

  // Final pass from the carry-in (Abar_{t0-1}, Bbar_{t0-1}).
#pragma unroll
  for (int s = 0; s < TSUB; ++s) {
    float a[K * K], b[K * V];
    if constexpr (HOLD) {
#pragma unroll
      for (int i = 0; i < K * K; ++i) a[i] = ha[s][i];
#pragma unroll
      for (int i = 0; i < K * V; ++i) b[i] = hb[s][i];
    } else {
      fetch(s, a, b);
    }
    AffM<K, V> nx;
#pragma unroll
    for (int i = 0; i < K; ++i) {
#pragma unroll
      for (int j = 0; j < K; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < K; ++m) acc = fmaf(a[i * K + m], carry.P[m][j], acc);
        nx.P[i][j] = acc;
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float acc = b[i * V + j];
#pragma unroll
        for (int m = 0; m < K; ++m) acc = fmaf(a[i * K + m], carry.L[m][j], acc);
        nx.L[i][j] = acc;
      }
    }
    carry = nx;
    const int64_t t = t0 + s;
    if (th.ok && t < T) {
      st<K * K, true>(Abar + offA(t), &carry.P[0][0]);
      st<K * V, true>(Bbar + offB(t), &carry.L[0][0]);
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
template <int K, int V, int TSUB, int WAVES>
__global__ __launch_bounds__(MG_WAVE* WAVES) void affine_bwd_kernel(
    const float* __restrict__ A, const float* __restrict__ Bm, const float* __restrict__ Abar,
    const float* __restrict__ Bbar, const float* __restrict__ GA, const float* __restrict__ GB,
    float* __restrict__ dA, float* __restrict__ dB, AfGeom g, unsigned* header,
    mg_slot_t* agg_data, mg_slot_t* incl_data) {
  constexpr bool HOLD = af_hold<K, V>();
  constexpr int HS = HOLD ? TSUB : 1;
  constexpr int W = K + V;  // adjoint state: [XA | XB]
  mg_persistent(header, (unsigned)g.n_lg * (unsigned)g.n_chunks,
                [&](unsigned ticket, unsigned epoch) {
    AfThread th = af_thread_at<true>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    const int64_t T = g.T, n = g.n;
    auto offA = [&](int64_t t) { return ((th.bb * T + t) * n + th.plane) * (K * K); };
    auto offB = [&](int64_t t) { return ((th.bb * T + t) * n + th.plane) * (K * V); };

    // hb[s] holds the saved Bbar_{t-1} (zero at t = 0): the final pass's forward
    // sweep reads it instead of rebuilding it from B, so only Abar needs a seed row.
    float ha[HS][K * K], hb[HS][K * V], hga[HS][K * K], hgb[HS][K * V];
    auto fetch = [&](int s, float* a, float* bprev, float* ga, float* gb, bool need_b) {
      const int64_t t = t0 + s;
      if (th.ok && t < T) {
        ld<K * K, HOLD>(a, A + offA(t));
        if (need_b) {
          if (t > 0) {
            ld<K * V, HOLD>(bprev, Bbar + offB(t - 1));
          } else {
#pragma unroll
            for (int i = 0; i < K * V; ++i) bprev[i] = 0.f;
          }
        }
        ld<K * K, HOLD>(ga, GA + offA(t));
        ld<K * V, HOLD>(gb, GB + offB(t));
      } else {
#pragma unroll
        for (int i = 0; i < K * K; ++i) {
          a[i] = (i / K == i % K) ? 1.f : 0.f;
          ga[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < K * V; ++i) {
          bprev[i] = 0.f;
          gb[i] = 0.f;
        }
      }
    };
    if constexpr (HOLD) {
#pragma unroll
      for (int s = 0; s < TSUB; ++s) fetch(s, ha[s], hb[s], hga[s], hgb[s], true);
    }

    // Local reverse aggregate: Y -> A_t^T (G_t + Y), composed from the end.
    AffM<K, W> loc, carry;
    affm_identity(loc);
#pragma unroll
    for (int s = TSUB - 1; s >= 0; --s) {
      float a[K * K], b[K * V], ga[K * K], gb[K * V];
      if constexpr (HOLD) {
#pragma unroll
        for (int i = 0; i < K * K; ++i) { a[i] = ha[s][i]; ga[i] = hga[s][i]; }
#pragma unroll
        for (int i = 0; i < K * V; ++i) { b[i] = hb[s][i]; gb[i] = hgb[s][i]; }
      } else {
        fetch(s, a, b, ga, gb, false);
      }
      AffM<K, W> nx;
#pragma unroll
      for (int i = 0; i < K; ++i) {
#pragma unroll
        for (int j = 0; j < K; ++j) {
          float acc = 0.f;
#pragma unroll
          for (int m = 0; m < K; ++m) acc = fmaf(a[m * K + i], loc.P[m][j], acc);
          nx.P[i][j] = acc;
        }
#pragma unroll
        for (int j = 0; j < W; ++j) {
          float acc = 0.f;
#pragma unroll
          for (int m = 0; m < K; ++m) {
            const float gmj = j < K ? ga[m * K + j] : gb[m * V + (j - K)];
            acc = fmaf(a[m * K + i], gmj + loc.L[m][j], acc);
          }
          nx.L[i][j] = acc;
        }
      }
      loc = nx;
    }
    AffM<K, W> seed;
    affm_identity(seed);
    af_carry<K, W, WAVES, true>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data, incl_data, carry);

    // Y entering the sub-chunk from the right (Y_T = 0 seed applied).
    float Y[K][W];
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
      for (int j = 0; j < W; ++j) Y[i][j] = carry.L[i][j];

    if constexpr (HOLD) {
      // Reverse sweep: X_t = G_t + Y; Y <- A_t^T X_t; keep X_t in place of G_t.
#pragma unroll
      for (int s = TSUB - 1; s >= 0; --s) {
        float X[K][W];
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < W; ++j)
            X[i][j] = (j < K ? hga[s][i * K + j] : hgb[s][i * V + (j - K)]) + Y[i][j];
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < W; ++j) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < K; ++m) acc = fmaf(ha[s][m * K + i], X[m][j], acc);
            Y[i][j] = acc;
          }
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < W; ++j) {
            if (j < K) hga[s][i * K + j] = X[i][j];
            else hgb[s][i * V + (j - K)] = X[i][j];
          }
      }
      // Forward sweep: recompute Abar_{t-1} from the saved boundary row; Bbar_{t-1}
      // is held.
      float Sa[K * K];
      if (th.ok && t0 > 0 && t0 <= T) {
        ld<K * K>(Sa, Abar + offA(t0 - 1));
      } else {
#pragma unroll
        for (int i = 0; i < K * K; ++i) Sa[i] = (i / K == i % K) ? 1.f : 0.f;
      }
#pragma unroll
      for (int s = 0; s < TSUB; ++s) {
        float d[K * K];
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < K; ++j) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < K; ++m) acc = fmaf(hga[s][i * K + m], Sa[j * K + m], acc);
#pragma unroll
            for (int m = 0; m < V; ++m) acc = fmaf(hgb[s][i * V + m], hb[s][j * V + m], acc);
            d[i * K + j] = acc;
          }
        float na[K * K];
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < K; ++j) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < K; ++m) acc = fmaf(ha[s][i * K + m], Sa[m * K + j], acc);
            na[i * K + j] = acc;
          }
#pragma unroll
        for (int i = 0; i < K * K; ++i) Sa[i] = na[i];
        const int64_t t = t0 + s;
        if (th.ok && t < T) {
          st<K * K, true>(dA + offA(t), d);
          st<K * V, true>(dB + offB(t), hgb[s]);
        }
      }
    } else {
      // Single reverse sweep reading the saved forward outputs.
      for (int s = TSUB - 1; s >= 0; --s) {
        const int64_t t = t0 + s;
        if (!(th.ok && t < T)) continue;
        float a[K * K], ga[K * K], gb[K * V], b_unused[1];
        (void)b_unused;
        ld<K * K>(a, A + offA(t));
        ld<K * K>(ga, GA + offA(t));
        ld<K * V>(gb, GB + offB(t));
        float Sa[K * K], Sb[K * V];
        if (t > 0) {
          ld<K * K>(Sa, Abar + offA(t - 1));
          ld<K * V>(Sb, Bbar + offB(t - 1));
        } else {
#pragma unroll
          for (int i = 0; i < K * K; ++i) Sa[i] = (i / K == i % K) ? 1.f : 0.f;
#pragma unroll
          for (int i = 0; i < K * V; ++i) Sb[i] = 0.f;
        }
        float X[K][W];
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < W; ++j)
            X[i][j] = (j < K ? ga[i * K + j] : gb[i * V + (j - K)]) + Y[i][j];
        float d[K * K], xb[K * V];
#pragma unroll
        for (int i = 0; i < K; ++i) {
#pragma unroll
          for (int j = 0; j < K; ++j) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < K; ++m) acc = fmaf(X[i][m], Sa[j * K + m], acc);
#pragma unroll
            for (int m = 0; m < V; ++m) acc = fmaf(X[i][K + m], Sb[j * V + m], acc);
            d[i * K + j] = acc;
          }
#pragma unroll
          for (int j = 0; j < V; ++j) xb[i * V + j] = X[i][K + j];
        }
        st<K * K, true>(dA + offA(t), d);
        st<K * V, true>(dB + offB(t), xb);
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
          for (int j = 0; j < W; ++j) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < K; ++m) acc = fmaf(a[m * K + i], X[m][j], acc);
            Y[i][j] = acc;
          }
      }
    }
  });
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
struct AfPlan {
  AfGeom g;
  size_t agg_off, incl_off, total;
};

AfPlan af_plan(int64_t B, int64_t T, int64_t n, int waves, int tsub, int nf) {
  AfPlan p;
  p.g.T = T;
  p.g.n = n;
  p.g.n_tiles = (int)((n + MG_WAVE - 1) / MG_WAVE);
  p.g.n_lg = (int)(B * p.g.n_tiles);
  const int64_t cl = (int64_t)waves * tsub;
  p.g.n_chunks = (int)((T + cl - 1) / cl);
  const size_t cnt = (size_t)p.g.n_lg * p.g.n_chunks;
  const size_t data = cnt * (size_t)nf * MG_WAVE * sizeof(mg_slot_t);
  p.agg_off = MG_HEADER_BYTES;
  p.incl_off = p.agg_off + mg_align_up(data, 256);
  p.total = p.incl_off + mg_align_up(data, 256);
  return p;
}

template <int K>
size_t af_ws_bytes_k(int64_t B, int64_t T, int64_t n, int v) {
  return std::max(af_plan(B, T, n, af_waves<K, false>(), af_tsub<K, false>(), K * K + K * v).total,
                  af_plan(B, T, n, af_waves<K, true>(), af_tsub<K, true>(), K * K + K * (K + v)).total);
}

bool kv_ok(int k, int v) {
  return (k == 1 || k == 2 || k == 4 || k == 8 || k == 16) &&
         (v == 1 || v == 2 || v == 4 || v == 8 || v == 16);
}

// 8x8 and 16x16 blocks: one wave per 16x16 block on the matrix cores.
bool uses_mfma(int k) { return k >= 8; }

bool af_geometry_ok(int64_t B, int64_t T, int64_t n) {
  if (B <= 0 || T <= 0 || n <= 0) return false;
  const int64_t lgs = B * ((n + MG_WAVE - 1) / MG_WAVE);
  const int64_t chunks = (T + 3) / 4;  // every chunk shape spans at least 4 steps
  return lgs * chunks < (1ll << 24);
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int K, int V>
int af_launch_fwd(const float* A, const float* Bm, float* Abar, float* Bbar, int64_t B, int64_t T,
                  int64_t n, void* ws, size_t ws_bytes, hipStream_t stream) {
  constexpr int TS = af_tsub<K, false>(), WV = af_waves<K, false>();
  AfPlan p = af_plan(B, T, n, WV, TS, K * K + K * V);
  if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
  unsigned* header = (unsigned*)ws;
  // Small held inputs run persistent workgroups; the others one workgroup per chunk.
  const unsigned chunks = (unsigned)(p.g.n_lg * p.g.n_chunks);
  const unsigned grid =
      af_fwd_persistent<K, V>()
          ? std::min(chunks, mg_resident((const void*)&affine_fwd_kernel<K, V, TS, WV>, MG_WAVE * WV))
          : chunks;
  hipLaunchKernelGGL((affine_fwd_kernel<K, V, TS, WV>), dim3(grid), dim3(MG_WAVE * WV), 0,
                     stream, A, Bm, Abar, Bbar, p.g, header,
                     (mg_slot_t*)((char*)ws + p.agg_off), (mg_slot_t*)((char*)ws + p.incl_off));
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

template <int K, int V>
int af_launch_bwd(const float* A, const float* Bm, const float* Abar, const float* Bbar,
                  const float* GA, const float* GB, float* dA, float* dB, int64_t B, int64_t T,
                  int64_t n, void* ws, size_t ws_bytes, hipStream_t stream) {
  constexpr int TS = af_tsub<K, true>(), WV = af_waves<K, true>();
  AfPlan p = af_plan(B, T, n, WV, TS, K * K + K * (K + V));
  if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
  unsigned* header = (unsigned*)ws;
  const unsigned chunks = (unsigned)(p.g.n_lg * p.g.n_chunks);
  const unsigned grid =
      std::min(chunks, mg_resident((const void*)&affine_bwd_kernel<K, V, TS, WV>, MG_WAVE * WV));
  hipLaunchKernelGGL((affine_bwd_kernel<K, V, TS, WV>), dim3(grid), dim3(MG_WAVE * WV), 0,
                     stream, A, Bm, Abar, Bbar, GA, GB, dA, dB, p.g, header,
                     (mg_slot_t*)((char*)ws + p.agg_off), (mg_slot_t*)((char*)ws + p.incl_off));
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

#define MG_AF_DISPATCH(FN, ...)                                    \
  switch (k * 100 + v) {                                           \
    case 101: return FN<1, 1>(__VA_ARGS__);                        \
    case 102: return FN<1, 2>(__VA_ARGS__);                        \
    case 104: return FN<1, 4>(__VA_ARGS__);                        \
    case 108: return FN<1, 8>(__VA_ARGS__);                        \
    case 116: return FN<1, 16>(__VA_ARGS__);                       \
    case 201: return FN<2, 1>(__VA_ARGS__);                        \
    case 202: return FN<2, 2>(__VA_ARGS__);                        \
    case 204: return FN<2, 4>(__VA_ARGS__);                        \
    case 208: return FN<2, 8>(__VA_ARGS__);                        \
    case 216: return FN<2, 16>(__VA_ARGS__);                       \
    case 401: return FN<4, 1>(__VA_ARGS__);                        \
    case 402: return FN<4, 2>(__VA_ARGS__);                        \
    case 404: return FN<4, 4>(__VA_ARGS__);                        \
    case 408: return FN<4, 8>(__VA_ARGS__);                        \
    case 416: return FN<4, 16>(__VA_ARGS__);                       \
    default: return MG_ERR_ARG; /* k >= 8 runs on the matrix cores */ \
  }

}  // namespace

extern "C" {

size_t mg_affine_scan_workspace_bytes(int64_t B, int64_t T, int64_t n, int k, int v) {
  if (!kv_ok(k, v) || B <= 0 || T <= 0 || n <= 0) return 256;
  if (uses_mfma(k)) return affine_mfma_workspace_bytes(B, T, n, k);
  switch (k) {
    case 1: return af_ws_bytes_k<1>(B, T, n, v);
    case 2: return af_ws_bytes_k<2>(B, T, n, v);
    default: return af_ws_bytes_k<4>(B, T, n, v);
  }
}

int mg_affine_scan_fwd(const float* A, const float* Bm, float* Abar, float* Bbar, int64_t B,
                       int64_t T, int64_t n, int k, int v, void* ws, size_t ws_bytes,
                       hipStream_t stream) {
  if (!A || !Bm || !Abar || !Bbar || !ws || !kv_ok(k, v) || !af_geometry_ok(B, T, n))
    return MG_ERR_ARG;
  if (!al16(A) || !al16(Bm) || !al16(Abar) || !al16(Bbar)) return MG_ERR_ARG;
  if (uses_mfma(k)) {
    if (!affine_mfma_geometry_ok(B, T, n, k)) return MG_ERR_ARG;
    return affine_mfma_fwd(A, Bm, Abar, Bbar, B, T, n, k, v, ws, ws_bytes, stream);
  }
  MG_AF_DISPATCH(af_launch_fwd, A, Bm, Abar, Bbar, B, T, n, ws, ws_bytes, stream)
}

int mg_affine_scan_bwd(const float* A, const float* Bm, const float* Abar, const float* Bbar,
                       const float* gAbar, const float* gBbar, float* dA, float* dBm, int64_t B,
                       int64_t T, int64_t n, int k, int v, void* ws, size_t ws_bytes,
                       hipStream_t stream) {
  if (!A || !Bm || !Abar || !Bbar || !gAbar || !gBbar || !dA || !dBm || !ws || !kv_ok(k, v) ||
      !af_geometry_ok(B, T, n))
    return MG_ERR_ARG;
  if (!al16(A) || !al16(Bm) || !al16(Abar) || !al16(Bbar) || !al16(gAbar) || !al16(gBbar) ||
      !al16(dA) || !al16(dBm))
    return MG_ERR_ARG;
  if (uses_mfma(k)) {
    if (!affine_mfma_geometry_ok(B, T, n, k)) return MG_ERR_ARG;
    return affine_mfma_bwd(A, Abar, Bbar, gAbar, gBbar, dA, dBm, B, T, n, k, v, ws, ws_bytes,
                           stream);
  }
  MG_AF_DISPATCH(af_launch_bwd, A, Bm, Abar, Bbar, gAbar, gBbar, dA, dBm, B, T, n, ws, ws_bytes,
                 stream)
}

}  // extern "C"

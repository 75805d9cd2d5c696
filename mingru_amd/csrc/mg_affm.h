// Matrix-valued affine maps S -> P S + L (P: K x K, L: K x W) and their
// decoupled look-back across workgroups, shared by the block-matrix scans
// and the angle-fused rotation scan.
#pragma once

#include "mg_common.h"

namespace mg {

struct AfGeom {
  int64_t T, n;
  int n_tiles, n_lg, n_chunks;
};

// Affine map on K x W matrices: S -> P S + L.
template <int K, int W>
struct AffM {
  float P[K][K];
  float L[K][W];
};

template <int K, int W>
__device__ __forceinline__ void affm_identity(AffM<K, W>& r) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
#pragma unroll
    for (int j = 0; j < K; ++j) r.P[i][j] = (i == j) ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < W; ++j) r.L[i][j] = 0.f;
  }
}

// r = outer o inner (apply inner first).  r may alias neither argument.
template <int K, int W>
__device__ __forceinline__ void affm_compose(const AffM<K, W>& inner, const AffM<K, W>& outer,
                                             AffM<K, W>& r) {
#pragma unroll
  for (int i = 0; i < K; ++i) {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < K; ++m) acc = fmaf(outer.P[i][m], inner.P[m][j], acc);
      r.P[i][j] = acc;
    }
#pragma unroll
    for (int j = 0; j < W; ++j) {
      float acc = outer.L[i][j];
#pragma unroll
      for (int m = 0; m < K; ++m) acc = fmaf(outer.P[i][m], inner.L[m][j], acc);
      r.L[i][j] = acc;
    }
  }
}

// Row loads/stores of N floats.  NT_REQ asks for non-temporal accesses, used for
// data a kernel touches exactly once (held inputs, every output); it is honoured
// only for rows of one vector (N <= 4), where a wave's instruction covers whole
// contiguous lines -- longer rows are split into lane-strided pieces that the
// L2 has to merge.
template <int N, bool NT_REQ = false>
__device__ __forceinline__ void ld(float* dst, const float* __restrict__ src) {
  constexpr bool NT = NT_REQ && N <= 4;
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const float4 v = NT ? mg_ld_stream4(src + i) : *reinterpret_cast<const float4*>(src + i);
      dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      if constexpr (NT) {
        const float2 v = mg_ld_stream2(src + i);
        dst[i] = v.x; dst[i + 1] = v.y;
      } else {
        float2 v = *reinterpret_cast<const float2*>(src + i);
        dst[i] = v.x; dst[i + 1] = v.y;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) dst[i] = NT ? mg_ld_stream(src + i) : src[i];
  }
}

template <int N, bool NT_REQ = false>
__device__ __forceinline__ void st(float* __restrict__ dst, const float* src) {
  constexpr bool NT = NT_REQ && N <= 4;
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const float4 v = make_float4(src[i], src[i + 1], src[i + 2], src[i + 3]);
      if constexpr (NT) mg_st_stream4(dst + i, v);
      else *reinterpret_cast<float4*>(dst + i) = v;
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      if constexpr (NT) {
        mg_st_stream2(dst + i, make_float2(src[i], src[i + 1]));
      } else {
        *reinterpret_cast<float2*>(dst + i) = make_float2(src[i], src[i + 1]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if constexpr (NT) mg_st_stream(dst + i, src[i]);
      else dst[i] = src[i];
    }
  }
}


// Look-back slots: [lg][chunk][field][64] tagged words.
template <int K, int W>
__device__ __forceinline__ void af_lb_put(mg_slot_t* base, const AfGeom& g, int lg, int c,
                                          int lane, const AffM<K, W>& x, unsigned epoch) {
  constexpr int NF = K * K + K * W;
  mg_slot_t* p = base + (int64_t)(lg * g.n_chunks + c) * NF * MG_WAVE + lane;
  const float* f = &x.P[0][0];
#pragma unroll
  for (int i = 0; i < K * K; ++i) mg_slot_put(p + i * MG_WAVE, f[i], epoch);
  const float* l = &x.L[0][0];
#pragma unroll
  for (int i = 0; i < K * W; ++i) mg_slot_put(p + (K * K + i) * MG_WAVE, l[i], epoch);
}

template <int K, int W>
__device__ __forceinline__ bool af_lb_try(const mg_slot_t* base, const AfGeom& g, int lg, int c,
                                          int lane, AffM<K, W>& x, unsigned epoch) {
  constexpr int NF = K * K + K * W;
  const mg_slot_t* p = base + (int64_t)(lg * g.n_chunks + c) * NF * MG_WAVE + lane;
  bool ok = true;
  float* f = &x.P[0][0];
#pragma unroll
  for (int i = 0; i < K * K; ++i) ok &= mg_slot_get(p + i * MG_WAVE, f[i], epoch);
  float* l = &x.L[0][0];
#pragma unroll
  for (int i = 0; i < K * W; ++i) ok &= mg_slot_get(p + (K * K + i) * MG_WAVE, l[i], epoch);
  return ok;
}

template <int K, int W>
__device__ __forceinline__ void lds_put(float* s, int lane, const AffM<K, W>& x) {
  const float* f = &x.P[0][0];
#pragma unroll
  for (int i = 0; i < K * K; ++i) s[i * MG_WAVE + lane] = f[i];
  const float* l = &x.L[0][0];
#pragma unroll
  for (int i = 0; i < K * W; ++i) s[(K * K + i) * MG_WAVE + lane] = l[i];
}

template <int K, int W>
__device__ __forceinline__ void lds_get(const float* s, int lane, AffM<K, W>& x) {
  float* f = &x.P[0][0];
#pragma unroll
  for (int i = 0; i < K * K; ++i) f[i] = s[i * MG_WAVE + lane];
  float* l = &x.L[0][0];
#pragma unroll
  for (int i = 0; i < K * W; ++i) l[i] = s[(K * K + i) * MG_WAVE + lane];
}

// Chained intra-workgroup scan + decoupled look-back.  `loc` is this thread's
// sub-chunk map; on return `carry` is the map of everything before
// (forward) / after (REVERSE) the thread's sub-chunk, composed with `seed`,
// the map at the sequence start (forward) / end (reverse).
template <int K, int W, int WAVES, bool REVERSE>
__device__ void af_carry(const AffM<K, W>& loc, const AffM<K, W>& seed, const AfGeom& g, int lg,
                         int c, unsigned* header, unsigned epoch, mg_slot_t* agg_data,
                         mg_slot_t* incl_data, AffM<K, W>& carry) {
  constexpr int NF = K * K + K * W;
  __shared__ float s_buf[NF * MG_WAVE];
  const int lane = threadIdx.x & (MG_WAVE - 1);
  const int w = threadIdx.x / MG_WAVE;
  AffM<K, W> ew, tmp;
  affm_identity(ew);
  // Waves in time order: forward 0..W-1, reverse W-1..0.
  for (int step = 0; step < WAVES; ++step) {
    const int j = REVERSE ? WAVES - 1 - step : step;
    if (w == j) {
      if (step > 0) lds_get(s_buf, lane, ew);
      affm_compose(ew, loc, tmp);
      lds_put(s_buf, lane, tmp);
    }
    __syncthreads();
  }
  // s_buf now holds the workgroup aggregate G.
  if (w == 0) {
    AffM<K, W> G, E, X, acc;
    lds_get(s_buf, lane, G);
    const int first = REVERSE ? g.n_chunks - 1 : 0;
    const int dir = REVERSE ? 1 : -1;
    if (c == first) {
      E = seed;
    } else {
      affm_identity(E);
      af_lb_put(agg_data, g, lg, c, lane, G, epoch);
      int j = c + dir;
      unsigned spins = 0;
      bool done = false;
      while (!done) {
        bool have = af_lb_try(incl_data, g, lg, j, lane, X, epoch);
        const bool incl = have;
        if (!have && j != first) have = af_lb_try(agg_data, g, lg, j, lane, X, epoch);
        if (have) {
          affm_compose(X, E, acc);
          E = acc;
          if (incl) done = true;
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
    affm_compose(E, G, acc);
    af_lb_put(incl_data, g, lg, c, lane, acc, epoch);
    lds_put(s_buf, lane, E);
  }
  __syncthreads();
  AffM<K, W> C;
  lds_get(s_buf, lane, C);
  affm_compose(C, ew, carry);
}


struct AfThread {
  int lane, w, c, lg, bb;
  unsigned epoch;
  bool valid;  // false only for a ticket beyond the grid (workspace protocol broken)
  int64_t plane;
  bool ok;
};

template <bool REVERSE>
__device__ __forceinline__ AfThread af_thread(const AfGeom& g, unsigned* header) {
  AfThread th;
  const MgTicket tk = mg_take_ticket(header);
  th.valid = tk.ticket < gridDim.x;
  const unsigned ticket = th.valid ? tk.ticket : 0u;
  th.epoch = tk.epoch;
  th.lane = threadIdx.x & (MG_WAVE - 1);
  th.w = threadIdx.x / MG_WAVE;
  int kk = (int)(ticket / (unsigned)g.n_lg);
  th.lg = (int)(ticket - (unsigned)kk * (unsigned)g.n_lg);
  th.c = REVERSE ? g.n_chunks - 1 - kk : kk;
  th.bb = th.lg / g.n_tiles;
  const int tile = th.lg - th.bb * g.n_tiles;
  th.plane = (int64_t)tile * MG_WAVE + th.lane;
  th.ok = th.plane < g.n;
  return th;
}

// The thread's chunk, lane group and plane for ticket `ticket` of a persistent
// look-back launch (mg_persistent): the (lane group, chunk) pair ticket % n_lg,
// ticket / n_lg (chunks from the end for the REVERSE backward).
template <bool REVERSE>
__device__ __forceinline__ AfThread af_thread_at(const AfGeom& g, unsigned ticket,
                                                 unsigned epoch) {
  AfThread th;
  th.valid = true;
  th.epoch = epoch;
  th.lane = threadIdx.x & (MG_WAVE - 1);
  th.w = threadIdx.x / MG_WAVE;
  int kk = (int)(ticket / (unsigned)g.n_lg);
  th.lg = (int)(ticket - (unsigned)kk * (unsigned)g.n_lg);
  th.c = REVERSE ? g.n_chunks - 1 - kk : kk;
  th.bb = th.lg / g.n_tiles;
  const int tile = th.lg - th.bb * g.n_tiles;
  th.plane = (int64_t)tile * MG_WAVE + th.lane;
  th.ok = th.plane < g.n;
  return th;
}

// 8x8 and 16x16 blocks run on the matrix cores (scan_affine_mfma.hip).
size_t affine_mfma_workspace_bytes(int64_t B, int64_t T, int64_t n, int k);
bool affine_mfma_geometry_ok(int64_t B, int64_t T, int64_t n, int k);
int affine_mfma_fwd(const float* A, const float* Bm, float* Abar, float* Bbar, int64_t B,
                    int64_t T, int64_t n, int k, int v, void* ws, size_t ws_bytes,
                    hipStream_t stream);
int affine_mfma_bwd(const float* A, const float* Abar, const float* Bbar, const float* GA,
                    const float* GB, float* dA, float* dB, int64_t B, int64_t T, int64_t n, int k,
                    int v, void* ws, size_t ws_bytes, hipStream_t stream);

}  // namespace mg

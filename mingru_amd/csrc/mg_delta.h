// Shared pieces of the DeltaMinGRU chunked-WY kernels (gfx950): chunk geometry,
// operand staging, fp32 MFMA tile helpers, the blocked unit-lower-triangular
// inverse and the host-side envelope.  The fp32-operand kernels live in
// delta_wy.hip, the bf16-operand kernels in delta_wy_bf16.hip.
#pragma once

#include "mg_common.h"

#include <algorithm>

namespace mgd {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int DN = 64;        // padded extent of every chunk matrix
constexpr int LD = 65;        // LDS row stride (floats): conflict-free row and column reads
constexpr int LDS16 = 17;     // LDS row stride of 16-column slices
constexpr int NT = 256;       // threads per workgroup (4 waves)
constexpr int SLICE = 16;     // d_v columns per chain workgroup
constexpr int MAT = DN * DN;  // floats per padded chunk matrix in the workspace

struct DwGeom {
  int64_t T;   // tokens per head
  int nh;      // micro-steps per token
  int dk, dv;  // head dims
  int C;       // tokens per chunk
  int nc;      // chunks per head
  int ns;      // d_v slices per head
};

// ---- element access: fp32 or bf16 (uint16_t storage, round-to-nearest-even) ----
__device__ __forceinline__ float ldf(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float ldf(const uint16_t* p, int64_t i) {
  return __uint_as_float((unsigned)p[i] << 16);
}
// ok ? p[i] : 0 with the load issued whether or not ok holds (from element 0, which
// every caller's buffer has, when it does not): written as a conditional load, the
// compiler gives each load a branch of its own and waits for it there, so a lane's
// loads run one after another instead of all in flight at once.
template <typename T>
__device__ __forceinline__ float ldf_or0(const T* p, int64_t i, bool ok) {
  const float v = ldf(p, ok ? i : 0);
  return ok ? v : 0.f;
}
// p[0] for a workgroup-uniform p, read with a vector load.  The compiler issues a
// uniform load as a scalar load, and scalar loads are counted together with LDS
// operations: a loop that prefetches one and then waits for its LDS writes before
// a barrier waits for the whole memory round trip of the prefetch as well.
__device__ __forceinline__ float ld_uniform_v(const float* p) {
  unsigned z = 0;
  asm volatile("" : "+v"(z));  // an index the compiler cannot prove uniform
  return p[z];
}
__device__ __forceinline__ uint16_t f2bf(float v) {
  unsigned u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ void stf(float* p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void stf(uint16_t* p, int64_t i, float v) { p[i] = f2bf(v); }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// acc += A (16 x KD) * B (KD x 16) with A[i][k] = a[i*ars + k*acs], B[k][j] = b[k*brs + j*bcs].
// Lane group g = lane/16 supplies k in [g*KD/4, (g+1)*KD/4) over the KD/4 steps; any
// bijection of k works as long as A and B agree, and this one keeps each lane's
// k range contiguous.
template <int KD>
__device__ __forceinline__ floatx4 mma(floatx4 acc, const float* a, int ars, int acs,
                                       const float* b, int brs, int bcs, float sa = 1.f) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < KD / 4; ++s) {
    const int k = (KD / 4) * g + s;
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sa * a[r * ars + k * acs], b[k * brs + r * bcs],
                                               acc, 0, 0, 0);
  }
  return acc;
}

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// The four tiles of one 16-row block: acc[J] += A (16 x KD) * B_J (KD x 16) with
// B_J[k][j] = b[J*jstride + k*brs + j*bcs].  The four accumulation chains are
// interleaved (independent MFMAs back to back instead of one dependent chain)
// and each A value is read once for all four tiles.
template <int KD>
__device__ __forceinline__ void mma_row4(floatx4 (&acc)[4], const float* a, int ars, int acs,
                                         const float* b, int brs, int bcs, int jstride,
                                         float sa = 1.f) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < KD / 4; ++s) {
    const int k = (KD / 4) * g + s;
    const float av = sa * a[r * ars + k * acs];
#pragma unroll
    for (int J = 0; J < 4; ++J)
      acc[J] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[J * jstride + k * brs + r * bcs],
                                                    acc[J], 0, 0, 0);
  }
}

__device__ __forceinline__ void zero_row4(floatx4 (&acc)[4]) {
#pragma unroll
  for (int J = 0; J < 4; ++J) acc[J] = zero4();
}

// Accumulator layout: lane (g, r) holds rows 4g..4g+3 of column r.
__device__ __forceinline__ void acc_store_lds(floatx4 acc, float* dst, int ld) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[(4 * g + i) * ld + r] = acc[i];
}
__device__ __forceinline__ floatx4 acc_load_lds(const float* src, int ld) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  floatx4 acc;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = src[(4 * g + i) * ld + r];
  return acc;
}
// Padded 64 x 64 workspace matrices (row stride DN).
__device__ __forceinline__ void acc_store_ws(floatx4 acc, float* dst) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[(4 * g + i) * DN + r] = acc[i];
}
__device__ __forceinline__ floatx4 acc_load_ws(const float* src) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  floatx4 acc;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = src[(4 * g + i) * DN + r];
  return acc;
}

__device__ __forceinline__ float tof(float x) { return x; }
__device__ __forceinline__ float tof(uint16_t x) { return __uint_as_float((unsigned)x << 16); }

// Register staging of a rows x cols block (row stride ldg) of a row-major global
// matrix, written later to a 64 x 64 LDS matrix (stride LD) with zeros outside
// the block.  Each thread holds 16 elements; every load is issued before any LDS
// store, and full-width, 16-byte aligned blocks move as 16-byte vectors.
// Sixteen zero bytes in global memory (never written).
static __device__ uint4 mg_zero16 = {0u, 0u, 0u, 0u};

template <typename TI>
struct Tile {
  static constexpr int EPV = 16 / sizeof(TI);  // elements per 16-byte vector
  static constexpr int NV = 16 / EPV;          // vectors per thread
  static constexpr int VPR = DN / EPV;         // vectors per 64-element row
  uint4 q[NV];
  bool vec;

  __device__ __forceinline__ void load(const TI* src, int rows, int cols, int64_t ldg) {
    vec = cols == DN && ldg == DN && (((uintptr_t)src) & 15u) == 0;
    if (vec) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int idx = threadIdx.x + v * NT;
        const int row = idx / VPR, col = (idx % VPR) * EPV;
        // Rows outside the block read a zero vector instead of being skipped: a
        // conditional load (or a select on its value) gets a branch of its own that
        // waits for it, so the thread's loads would not all be in flight at once.
        q[v] = *(row < rows ? reinterpret_cast<const uint4*>(src + (int64_t)row * DN + col)
                            : &mg_zero16);
      }
    } else {
      TI* e = reinterpret_cast<TI*>(q);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int idx = threadIdx.x + k * NT;
        const int row = idx >> 6, col = idx & 63;
        const bool ok = row < rows && col < cols;
        const TI x = src[ok ? (int64_t)row * ldg + col : 0];
        e[k] = ok ? x : TI(0);
      }
    }
  }

  __device__ __forceinline__ void store(float* s) const {
    const TI* e = reinterpret_cast<const TI*>(q);
    if (vec) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int idx = threadIdx.x + v * NT;
        const int row = idx / VPR, col = (idx % VPR) * EPV;
#pragma unroll
        for (int x = 0; x < EPV; ++x) s[row * LD + col + x] = tof(e[v * EPV + x]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int idx = threadIdx.x + k * NT;
        s[(idx >> 6) * LD + (idx & 63)] = tof(e[k]);
      }
    }
  }

  // Sum over this thread's elements of e * s[row * LD + col], at the positions
  // store() writes them to.
  __device__ __forceinline__ float dot(const float* s) const {
    const TI* e = reinterpret_cast<const TI*>(q);
    float acc = 0.f;
    if (vec) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int idx = threadIdx.x + v * NT;
        const int row = idx / VPR, col = (idx % VPR) * EPV;
#pragma unroll
        for (int x = 0; x < EPV; ++x) acc = fmaf(tof(e[v * EPV + x]), s[row * LD + col + x], acc);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int idx = threadIdx.x + k * NT;
        acc = fmaf(tof(e[k]), s[(idx >> 6) * LD + (idx & 63)], acc);
      }
    }
    return acc;
  }
};

// Chain workgroup -> (head, d_v slice).  Workgroups are dispatched round-robin
// over the 8 XCDs (blockIdx mod 8), each with its own L2; the slices of one
// head are placed on one XCD so that their shared per-chunk operands (W, P, K,
// Q forward; E, K backward) are fetched from HBM once and re-read from that L2.
// The grid is padded to a multiple of 8 heads; padding workgroups return.
constexpr int N_XCD = 8;
__device__ __forceinline__ bool chain_slot(const DwGeom& g, int64_t BH, int64_t& bh, int& col0) {
  const unsigned i = blockIdx.x, x = i % N_XCD, j = i / N_XCD;
  bh = (int64_t)(j / g.ns) * N_XCD + x;
  col0 = (int)(j % g.ns) * SLICE;
  return bh < BH;
}
inline unsigned chain_grid(int64_t BH, const DwGeom& g) {
  return (unsigned)((BH + N_XCD - 1) / N_XCD * N_XCD * g.ns);
}

// Chunk geometry of chunk c: first token, valid tokens, valid micro-rows.
struct Chunk {
  int64_t t0;
  int Ct, M;
};
__device__ __forceinline__ Chunk chunk_of(const DwGeom& g, int c) {
  Chunk ch;
  ch.t0 = (int64_t)c * g.C;
  ch.Ct = (int)min((int64_t)g.C, g.T - ch.t0);
  ch.M = ch.Ct * g.nh;
  return ch;
}

// ---------------------------------------------------------------------------
// Tm^-1 for Tm = I + L, L strictly lower (64 x 64 in LDS), blocked in 16 x 16:
// diagonal blocks by forward substitution (one wave, a lane group per block), then
// T_ab = -T_aa L_ab T_bb for the two 16-blocks below the diagonal of each
// 32 x 32 half, then the lower-left 32 x 32 block -T_22' L' T_11'.
// sT receives the full lower-triangular inverse with zeroed upper blocks.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void unit_lower_inverse(const float* sL, float* sT, float* sY) {
  // Waves 0..3 do the work; further waves of a larger workgroup only join the
  // barriers.  (An earlier form gave each wave one diagonal block and reduced the
  // substitution sums across lane groups with shuffles: 16 dependent LDS round
  // trips per block, about half the cost of the whole inverse.)
  const int w = wave_id(), lane = lane_id(), r = lane & 15, g = lane >> 4;
  if (w == 0) {
    // The four diagonal blocks at once: lane group g inverts block g, lane r
    // solves its column r of X = (I + L_gg)^-1 by forward substitution,
    // X[i][r] = delta_ir - sum_{k<i} L[i][k] X[k][r], with no cross-lane
    // traffic (the L reads are broadcast within the lane group).  Two partial
    // sums shorten the dependency chain of each step.
    const int o = 16 * g;
    const float* Lb = sL + o * LD + o;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float a0 = (i == r) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
      for (int k = 0; k + 1 < i; k += 2) {
        a0 = fmaf(-Lb[i * LD + k], x[k], a0);
        a1 = fmaf(-Lb[i * LD + k + 1], x[k + 1], a1);
      }
      if (i & 1) a0 = fmaf(-Lb[i * LD + i - 1], x[i - 1], a0);
      x[i] = a0 + a1;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sT[(o + i) * LD + o + r] = x[i];
  } else if (w < 4) {
    // Zero the blocks right of the diagonal in block-row w - 1 (rows 0..2 have some).
    const int o = 16 * (w - 1);
    for (int jb = w; jb < 4; ++jb)
#pragma unroll
      for (int q = 0; q < 4; ++q) sT[(o + 4 * q + g) * LD + 16 * jb + r] = 0.f;
  }
  __syncthreads();
  if (w < 2) {
    // Blocks (1,0) and (3,2).
    const int a = 2 * w + 1, b = 2 * w;
    floatx4 y = mma<16>(zero4(), sL + 16 * a * LD + 16 * b, LD, 1, sT + 16 * b * LD + 16 * b, LD, 1);
    floatx4 t = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s)
      t = __builtin_amdgcn_mfma_f32_16x16x4f32(-sT[(16 * a + r) * LD + 16 * a + 4 * g + s], y[s], t,
                                               0, 0, 0);
    acc_store_lds(t, sT + 16 * a * LD + 16 * b, LD);
  }
  __syncthreads();
  // Lower-left 32 x 32: Y = L[32:64, 0:32] T[0:32, 0:32], then -T[32:64, 32:64] Y.
  const int a = 2 + ((w & 3) >> 1), b = w & 1;
  if (w < 4) {
    floatx4 y = mma<32>(zero4(), sL + 16 * a * LD, LD, 1, sT + 16 * b, LD, 1);
    acc_store_lds(y, sY + b * 32 * LDS16 + (a - 2) * 16 * LDS16, LDS16);
  }
  __syncthreads();
  if (w < 4) {
    floatx4 t = mma<32>(zero4(), sT + 16 * a * LD + 32, LD, 1, sY + b * 32 * LDS16, LDS16, 1, -1.f);
    acc_store_lds(t, sT + 16 * a * LD + 16 * b, LD);
  }
  __syncthreads();
}

// T^T = ((I + L)^-1)^T is upper triangular: of its 8-float row chunks (row, q) only
// those with q >= row / 8 can be nonzero, 288 of 512.  They are kept packed, row by
// row, in the first 9 KB of the chunk's matrix slot; this is the packed index of
// chunk (row, q), q >= row / 8.
__device__ __forceinline__ int tri_chunk(int row, int q) {
  const int a = row >> 3;
  return 8 * (8 * a - a * (a - 1) / 2) + (row & 7) * (8 - a) + (q - a);
}

// T^T's possibly nonzero chunks from the fp32 T in LDS (row stride LD) to a packed slot,
// and back into LDS as T with the zero chunks filled in (NTH threads, each taking chunks
// i = tid, tid + NTH, ... of the 512 (row, q)).  The fp32 kernels' backward preparation
// reads the inverse its forward formed instead of forming L and inverting it again.
template <int NTH>
__device__ __forceinline__ void store_inv_packed(float* To, const float* sT) {
#pragma unroll
  for (int i = threadIdx.x; i < DN * 8; i += NTH) {
    const int row = i >> 3, q = i & 7;
    if (q >= row >> 3) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = sT[(8 * q + e) * LD + row];
      float4* t = reinterpret_cast<float4*>(To + 8 * tri_chunk(row, q));
      t[0] = make_float4(x[0], x[1], x[2], x[3]);
      t[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
  }
}
template <int NTH>
__device__ __forceinline__ void load_inv_packed(float* sT, const float* Tin) {
#pragma unroll
  for (int i = threadIdx.x; i < DN * 8; i += NTH) {
    const int row = i >> 3, q = i & 7;
    const bool nz = q >= row >> 3;  // zero chunks read a zero vector (no branch)
    const float4* src = reinterpret_cast<const float4*>(Tin + 8 * tri_chunk(row, nz ? q : row >> 3));
    const float4 a = *(nz ? src : reinterpret_cast<const float4*>(&mg_zero16));
    const float4 b = *(nz ? src + 1 : reinterpret_cast<const float4*>(&mg_zero16));
    float* col = sT + 8 * q * LD + row;
    col[0] = a.x;
    col[LD] = a.y;
    col[2 * LD] = a.z;
    col[3 * LD] = a.w;
    col[4 * LD] = b.x;
    col[5 * LD] = b.y;
    col[6 * LD] = b.z;
    col[7 * LD] = b.w;
  }
}

// L = strict_lower(K K^T) * beta_col into sL; wave w builds block-row w.
__device__ __forceinline__ void build_L(const float* sK, const float* sb, float* sL) {
  const int w = wave_id(), lane = lane_id(), r = lane & 15, g = lane >> 4;
  floatx4 acc[4];
  zero_row4(acc);
  mma_row4<64>(acc, sK + 16 * w * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
  for (int J = 0; J < 4; ++J) {
    // The masked value is formed first and the mask picks a local: a conditional
    // whose arm computes becomes a branch, with the LDS read of sb moved into it.
    const float bc = sb[16 * J + r];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * w + 4 * g + i, col = 16 * J + r;
      const float v = acc[J][i] * bc;
      sL[row * LD + col] = col < row ? v : 0.f;
    }
  }
}


// Column sums of a tile (over the 4 rows of each lane and the 4 lane groups)
// written to s[col]; every (slot, column) is written by exactly one lane, so the
// final reduction order is fixed and the result bitwise reproducible.
__device__ __forceinline__ void put_colsum(floatx4 v, float* s, int col) {
  const float p = mg_pair_sum<32>(mg_pair_sum<16>(v[0] + v[1] + v[2] + v[3]));
  if (lane_id() < 16) s[col] = p;
}


// ---------------------------------------------------------------------------
// Decay tables of the gated chunked-WY kernels (per-token log decay l_t <= 0,
// tau(m) = m / nh the token of micro-row m; every table is rebuilt per chunk).
// ---------------------------------------------------------------------------
constexpr int VECN = 256;  // floats per chunk in the vector region
// Vector region layout per chunk: [0, 64) a_m beta_m, [64, 128) ptok_t,
// [128, 192) p_m, [192] PC.
constexpr int V_AB = 0, V_PT = 64, V_P = 128, V_PC = 192;

// sE[t][t'] = exp(span(t, t')) for t' <= t, 0 above (row stride LDE).  Each wave of the NTH-thread
// workgroup fills 64 / (NTH / 64) consecutive rows t: lane s holds l_s masked to
// s <= t, and an inclusive suffix scan across the wave gives sum_{s' >= s};
// span(t, t') is the scan value of lane t' + 1.  Every span is a sum of its own
// terms only (never a difference of running sums), so a saturated gap affects only
// the spans that contain it.
template <int NTH, int LDE = LD>
__device__ __forceinline__ void decay_tables(const float* sl, float* sE) {
  constexpr int ROWS = DN / (NTH / 64);  // rows per wave
  const int w = wave_id(), lane = lane_id();
  const float lv = sl[lane];
  for (int rr = 0; rr < ROWS; ++rr) {
    const int t = ROWS * w + rr;
    const float ex = mg_wave_next(mg_wave_suffix_sum(lane <= t ? lv : 0.f));
    sE[t * LDE + lane] = lane <= t ? expf(ex) : 0.f;
  }
}

// The chunk's decay vectors, straight from l by wave 0 (no other wave's results are
// read, so no barrier separates them from decay_tables):
//   sLc[t] = Lc_t (inclusive prefix scan), sp[m] = exp(Lc_tau(m)) for m < M,
//   sab[m] = a_m beta_m with a_m = exp(sum_{s=tau(m)+1..Ct-1} l_s) (masked suffix
//   scan, the last row of the span table), and when given spt[t] = exp(Lc_t) for
//   t < Ct and sa[m] = a_m.
__device__ __forceinline__ void decay_vectors(const float* sl, const float* sb, const Chunk& ch,
                                              int nh, float* sLc, float* sp, float* sab,
                                              float* spt = nullptr, float* sa = nullptr) {
  if (wave_id() != 0) return;
  const int lane = lane_id();
  const float lv = sl[lane];
  const float pre = mg_wave_prefix_sum(lv);
  const float carry = mg_wave_next(mg_wave_suffix_sum(lane < ch.Ct ? lv : 0.f));  // (lane, Ct-1]
  sLc[lane] = pre;
  if (spt) spt[lane] = lane < ch.Ct ? expf(pre) : 0.f;
  const int tau = lane / nh;
  const float lc_m = __shfl(pre, tau), carry_m = __shfl(carry, tau);
  const bool ok = lane < ch.M;
  const float a = ok ? expf(carry_m) : 0.f;
  sp[lane] = ok ? expf(lc_m) : 0.f;
  sab[lane] = a * sb[lane];
  if (sa) sa[lane] = a;
}

__device__ __forceinline__ void write_vectors(float* vv, const float* sLc, const float* sp,
                                              const float* sab, const Chunk& ch) {
  const int m = threadIdx.x;
  if (m < DN) {
    vv[V_AB + m] = sab[m];
    vv[V_PT + m] = m < ch.Ct ? expf(sLc[m]) : 0.f;
    vv[V_P + m] = sp[m];
    if (m == 0) vv[V_PC] = expf(sLc[ch.Ct - 1]);
  }
}

// l of token (thread index mod 64) of chunk ch: every wave of a larger workgroup
// loads the same values, so a kernel can store them without a branch on the thread
// index (inside such a branch the compiler issues the load last and waits for it).
__device__ __forceinline__ float ld_l(const float* lg, int64_t bh, const DwGeom& g,
                                      const Chunk& ch) {
  const int t = threadIdx.x & (DN - 1);
  return ldf_or0(lg, bh * g.T + ch.t0 + t, t < ch.Ct);
}


inline bool dw_geom(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv, int chunk, DwGeom& g,
             int64_t& BH) {
  if (B <= 0 || H <= 0 || T <= 0 || nh <= 0 || chunk <= 0) return false;
  if (dk <= 0 || dk > DN || dv <= 0 || dv > DN || (int64_t)nh * chunk > DN) return false;
  BH = B * H;
  g.T = T;
  g.nh = nh;
  g.dk = dk;
  g.dv = dv;
  g.C = chunk;
  const int64_t nc = (T + chunk - 1) / chunk;
  if (nc > 65535 || BH > 65535) return false;
  g.nc = (int)nc;
  g.ns = (dv + SLICE - 1) / SLICE;
  return true;
}

inline size_t dw_mat_bytes(int64_t BH, const DwGeom& g) { return (size_t)BH * g.nc * MAT * sizeof(float); }
// The saved state buffer (Hbound): one padded matrix slot per (head, chunk) for the
// chunk-entry states, then one for each chunk's T^T = ((I + L)^-1)^T, which the forward
// preparation kernels write (packed, tri_chunk) for the backward preparation kernels.
inline size_t dw_state_bytes(int64_t BH, const DwGeom& g) { return 2 * dw_mat_bytes(BH, g); }
inline float* dw_inv_slots(float* Hb, int64_t BH, const DwGeom& g) {
  return Hb + (size_t)BH * g.nc * MAT;
}
inline const float* dw_inv_slots(const float* Hb, int64_t BH, const DwGeom& g) {
  return Hb + (size_t)BH * g.nc * MAT;
}

// bf16-input entry points (delta_wy_bf16.hip).  Q, K, V, beta, y, dy and the
// input gradients are bf16 (uint16_t storage); states and workspaces are fp32.
int dw_fwd_bf16(const void* Q, const void* K, const void* V, const void* beta, const float* H0,
                void* y, float* HT, float* Hb, int64_t BH, const DwGeom& g, void* ws,
                size_t ws_bytes, hipStream_t stream);
int dw_bwd_bf16(const void* Q, const void* K, const void* V, const void* beta, const float* Hb,
                const void* dy, const float* dHT, void* dQ, void* dK, void* dV, void* dbeta,
                float* dH0, int64_t BH, const DwGeom& g, void* ws, size_t ws_bytes,
                hipStream_t stream);

// The bf16 backward preparation kernel, either form (gated: lg and the vector
// region vm), launched from a translation unit of its own (delta_bwd_prep_bf16.hip).
int dwb_bwd_prep_launch(bool gated, const void* Q, const void* K, const void* V, const void* beta,
                        const float* lg, const void* dy, const float* Hb, float* Um, float* Em,
                        float* G0m, float* Apm, float* bpm, float* vm, int64_t BH,
                        const DwGeom& g, hipStream_t stream);

// Decay-gated forms (delta_gated.hip), bf16 inputs: lg / dlg are the
// per-token log decay and its gradient, fp32 (B*H, T); the workspace adds a
// vector region of VECN floats per chunk after the matrices.
int dw_fwd_bf16_gated(const void* Q, const void* K, const void* V, const void* beta,
                      const float* lg, const float* H0, void* y, float* HT, float* Hb, int64_t BH,
                      const DwGeom& g, void* ws, size_t ws_bytes, hipStream_t stream);
int dw_bwd_bf16_gated(const void* Q, const void* K, const void* V, const void* beta,
                      const float* lg, const float* Hb, const void* dy, const float* dHT, void* dQ,
                      void* dK, void* dV, void* dbeta, float* dlg, float* dH0, int64_t BH,
                      const DwGeom& g, void* ws, size_t ws_bytes, hipStream_t stream);

}  // namespace mgd

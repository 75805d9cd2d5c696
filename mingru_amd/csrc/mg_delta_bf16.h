// bf16-MFMA operand machinery and the chunked-WY kernels on it (gfx950), shared by
// the ungated entry points (delta_wy_bf16.hip) and the decay-gated ones
// (delta_gated.hip).  Each kernel is a template on GATED; a translation unit
// instantiates only the form it launches (one unit holding both forms allocated
// the ungated gradient kernel's registers worse: 12 spills instead of 5).
//
// DeltaMinGRU chunked-WY delta rule on bf16 MFMA (gfx950), for bf16 Q, K, V, beta.
//
// Same algorithm, chunk geometry and workspace layout as the fp32-operand
// kernels of delta_wy.hip (reference src/mingru/triton_scans.py:473-605 and
// :1859-2322; the formulas are listed at the top of delta_wy.hip); what
// changes is how the products are evaluated.
//
// Every product is C[i][j] = sum_k A[i][k] B[j][k] over k < 64 with both
// operands held in LDS as 64 x 64 bf16 "row x k" matrices (BMat): the row is
// the operand's free index and k the contracted one, stored contiguously so an
// MFMA fragment (8 consecutive k of one row) is a single 16-byte LDS read.
// Products run on v_mfma_f32_16x16x32_bf16 with fp32 accumulation:
//   - bf16 inputs (Q, K, V, dy) are exact in bf16: one MFMA per fragment pair;
//   - fp32 intermediates (states, Tm^-1, U, G, dS, ...) are stored as a pair
//     hi = bf16(x), lo = bf16(x - hi), and a product takes hi*hi + hi*lo + lo*hi
//     (or in*hi + in*lo against an exact input), which keeps about 16
//     significant bits per operand -- fp32-level results for the reference's
//     fp32 ("ieee") products -- at 2-3 bf16 MFMAs per fp32 one it replaces,
//     each 16x more work per cycle than v_mfma_f32_16x16x4_f32.
#pragma once

#include "mg_delta.h"

namespace {

using namespace mgd;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16;

// ---- bf16 operand matrices in LDS ------------------------------------------------
// Row r holds 8 chunks of 8 consecutive k; chunk q sits at position
// q ^ ((r ^ (r >> 3)) & 7) of the row.  Fragment reads (8 consecutive rows, one
// chunk) and transposed element writes (rows 8 apart, one k) both touch 8
// distinct 16-byte positions, i.e. all LDS banks once.
struct BMat {
  uint4 v[DN * 8];
};

__device__ __forceinline__ int bpos(int r, int q) { return r * 8 + (q ^ ((r ^ (r >> 3)) & 7)); }
__device__ __forceinline__ u16* belem(BMat& m, int r, int k) {
  return reinterpret_cast<u16*>(&m.v[bpos(r, k >> 3)]) + (k & 7);
}
__device__ __forceinline__ float bget(const BMat& m, int r, int k) {
  const u16 h = reinterpret_cast<const u16*>(&m.v[bpos(r, k >> 3)])[k & 7];
  return __uint_as_float((unsigned)h << 16);
}

__device__ __forceinline__ u16 bf_bits(float x) { return __builtin_bit_cast(u16, (__bf16)x); }
__device__ __forceinline__ float bf_val(u16 h) { return __uint_as_float((unsigned)h << 16); }
// x = hi + lo to about 16 significant bits (both round to nearest even), for two
// values at once: hp packs hi(x0) | hi(x1) << 16, lp the lo halves.  Both his come
// from one packed conversion and are widened in place (a shift for the low half, a
// mask for the high one), and both remainders go through one packed conversion:
// six VALU per pair, where splitting each value on its own and packing the halves
// afterwards took eleven (the pair's conversions are also half as many).  The empty asm statements keep the packed words opaque:
// without them the compiler rewrites their uses as per-value conversions again.
__device__ __forceinline__ void bf_split2(float x0, float x1, unsigned& hp, unsigned& lp) {
  const bf16x2 h = {(__bf16)x0, (__bf16)x1};
  hp = __builtin_bit_cast(unsigned, h);
  asm("" : "+v"(hp));
  const float r0 = x0 - __uint_as_float(hp << 16);
  const float r1 = x1 - __uint_as_float(hp & 0xffff0000u);
  const bf16x2 l = {(__bf16)r0, (__bf16)r1};
  lp = __builtin_bit_cast(unsigned, l);
  asm("" : "+v"(lp));
}
__device__ __forceinline__ void bf_split(float x, u16& hi, u16& lo) {
  hi = bf_bits(x);
  lo = bf_bits(x - bf_val(hi));
}

// Split pair (hi, lo) of an fp32 matrix.
typedef BMat BPair[2];

// Two single elements, (r0, k0) = x0 and (r1, k1) = x1, split as a pair.
__device__ __forceinline__ void put_split1x2(BPair& m, int r0, int k0, float x0, int r1, int k1,
                                             float x1) {
  unsigned hp, lp;
  bf_split2(x0, x1, hp, lp);
  *belem(m[0], r0, k0) = (u16)hp;
  *belem(m[1], r0, k0) = (u16)lp;
  *belem(m[0], r1, k1) = (u16)(hp >> 16);
  *belem(m[1], r1, k1) = (u16)(lp >> 16);
}
// Four consecutive k (k % 4 == 0): one 8-byte write per half.
__device__ __forceinline__ void put_split4(BPair& m, int r, int k, float x0, float x1, float x2,
                                           float x3) {
  unsigned h01, l01, h23, l23;
  bf_split2(x0, x1, h01, l01);
  bf_split2(x2, x3, h23, l23);
  *reinterpret_cast<uint2*>(belem(m[0], r, k)) = make_uint2(h01, h23);
  *reinterpret_cast<uint2*>(belem(m[1], r, k)) = make_uint2(l01, l23);
}
// Eight consecutive k (one chunk q): one 16-byte write per half.
__device__ __forceinline__ void put_split8(BPair& m, int r, int q, const float (&x)[8]) {
  unsigned h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) bf_split2(x[2 * p], x[2 * p + 1], h[p], l[p]);
  m[0].v[bpos(r, q)] = make_uint4(h[0], h[1], h[2], h[3]);
  m[1].v[bpos(r, q)] = make_uint4(l[0], l[1], l[2], l[3]);
}

// Accumulator tile (lane (g, r) holds rows R0+4g..R0+4g+3 of column C0+r) into
// a split BMat, either as (row = tile row, k = tile column) or transposed
// (row = tile column, k = tile row).
__device__ __forceinline__ void acc_put(BPair& m, floatx4 a, int R0, int C0) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  put_split1x2(m, R0 + 4 * g, C0 + r, a[0], R0 + 4 * g + 1, C0 + r, a[1]);
  put_split1x2(m, R0 + 4 * g + 2, C0 + r, a[2], R0 + 4 * g + 3, C0 + r, a[3]);
}
// Transposed: lane (g, r) holds k = R0+4g..R0+4g+3 of row C0+r, half of a 16-byte
// chunk.  The lane rows g and g^1 (lanes 16 apart) swap halves with
// v_permlane16_swap: afterwards an even-g lane holds the chunk's 8 hi values and the
// odd-g lane beside it the 8 lo values, so each lane makes one 16-byte store, and a
// group of 8 lanes stores 8 consecutive rows, which the swizzle puts in 8 distinct
// bank groups.  (Four 8-byte stores per lane pair of 16 rows put two rows on each
// bank group.)  The whole wave must be active; R0 is a multiple of 8.
__device__ __forceinline__ void acc_put_t(BPair& m, floatx4 a, int R0, int C0) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  unsigned hx, lx, hy, ly;
  bf_split2(a[0], a[1], hx, lx);
  bf_split2(a[2], a[3], hy, ly);
  // [0]: even lane rows keep their own (hi) words and odd ones receive the even
  // partner's lo words; [1]: even rows receive the odd partner's hi words, odd rows
  // keep their own lo words.
  const auto sx = __builtin_amdgcn_permlane16_swap(hx, lx, false, false);
  const auto sy = __builtin_amdgcn_permlane16_swap(hy, ly, false, false);
  m[g & 1].v[bpos(C0 + r, (R0 >> 3) + (g >> 1))] = make_uint4(sx[0], sy[0], sx[1], sy[1]);
}

__device__ __forceinline__ bf16x8 bneg(bf16x8 x) {
  uint4 u = __builtin_bit_cast(uint4, x);
  u.x ^= 0x80008000u;
  u.y ^= 0x80008000u;
  u.z ^= 0x80008000u;
  u.w ^= 0x80008000u;
  return __builtin_bit_cast(bf16x8, u);
}

// Workgroups of the bf16 kernels: 8 waves; wave w computes the 16 x 32 output
// block of row block rb = w % 4 and column tiles 2 ch, 2 ch + 1 (ch = w / 4).
constexpr int NTB = 512;
constexpr int WB = NTB / MG_WAVE;

// Byte offsets of this lane's MFMA fragments inside a BMat.  Row 16 blk + r,
// chunk q = 4 s + g sits at byte blk * 2048 + r * 128 + 16 (q ^ (r & 7) ^ (r >> 3)
// ^ (2 blk & 7)); the wave's row block and its two column blocks are fixed, so
// six lane constants address every fragment it reads, and each read is one
// ds_read_b128 whose immediate offset is the matrix's LDS base.
struct FragOff {
  unsigned a[2];     // [s]: row block rb (A operand)
  unsigned b[2][2];  // [s][jj]: row block 2 ch + jj (B operand)
  int rb, ch;        // row block, column half

  __device__ static __forceinline__ unsigned at(int blk, unsigned L, int r) {
    return (unsigned)blk * 2048u + (unsigned)r * 128u + ((L ^ ((2u * blk) & 7u)) << 4);
  }
  __device__ __forceinline__ void init() {
    const int lane = lane_id(), r = lane & 15, g = lane >> 4, w = wave_id();
    rb = w & 3;
    ch = w >> 2;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const unsigned L = (unsigned)((4 * s + g) ^ (r & 7) ^ (r >> 3));
      a[s] = at(rb, L, r);
      b[s][0] = at(2 * ch, L, r);
      b[s][1] = at(2 * ch + 1, L, r);
    }
  }
};

__device__ __forceinline__ bf16x8 frag_at(const BMat& m, unsigned off) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                        reinterpret_cast<const char*>(&m) + off));
}

// acc[jj] (+/-)= A[row block rb] . B[row block 2 ch + jj]^T over k < 64 (the wave's
// 16 x 32 output block).  SA / SB: the operand is a split pair (the pointer is
// its hi half, the lo half follows); NEG negates A.
template <bool SA, bool SB, bool NEG = false>
__device__ __forceinline__ void bmm(floatx4 (&acc)[2], const FragOff& F, const BMat* A,
                                    const BMat* B) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bf16x8 ah = frag_at(A[0], F.a[s]), al;
    if constexpr (SA) al = frag_at(A[1], F.a[s]);
    if constexpr (NEG) {
      ah = bneg(ah);
      if constexpr (SA) al = bneg(al);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const unsigned off = F.b[s][jj];
      const bf16x8 bh = frag_at(B[0], off);
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc[jj], 0, 0, 0);
      if constexpr (SB)
        acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, frag_at(B[1], off), acc[jj], 0, 0, 0);
      if constexpr (SA) acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc[jj], 0, 0, 0);
    }
  }
}

__device__ __forceinline__ void zero2(floatx4 (&acc)[2]) { acc[0] = acc[1] = zero4(); }

// Column sums of the wave's tile jj (over its 16 rows) into s[col]: each
// (slot, column) is written by one lane, so reductions stay in a fixed order.
__device__ __forceinline__ void colsum16(floatx4 v, float* s, int col) {
  const float p = mg_pair_sum<32>(mg_pair_sum<16>(v[0] + v[1] + v[2] + v[3]));
  if (lane_id() < 16) s[col] = p;
}

// ---- staging of global blocks ------------------------------------------------------
// bf16 block (rows x cols, row stride ldg) of a row-major input: thread idx holds
// row idx / 8, columns 8 (idx % 8) + 0..7, zero outside the block.
struct BTile {
  uint4 q;

  __device__ __forceinline__ void load(const u16* src, int rows, int cols, int64_t ldg) {
    const int idx = threadIdx.x, row = idx >> 3, c0 = (idx & 7) * 8;
    if (cols == DN && ldg == DN && (((uintptr_t)src) & 15u) == 0) {
      // Loaded whether or not the row is in the block (row 0 when it is not), so the
      // compiler keeps the load out of a branch that would wait for it.
      const unsigned off = (unsigned)((row < rows ? row : 0) * DN + c0);
      const uint4 v = *reinterpret_cast<const uint4*>(src + off);
      q = row < rows ? v : make_uint4(0u, 0u, 0u, 0u);
    } else {
      u16 e[8];
#pragma unroll
      for (int x = 0; x < 8; ++x)
        e[x] = (row < rows && c0 + x < cols) ? src[(int64_t)row * ldg + c0 + x] : (u16)0;
      q = make_uint4(e[0] | ((unsigned)e[1] << 16), e[2] | ((unsigned)e[3] << 16),
                     e[4] | ((unsigned)e[5] << 16), e[6] | ((unsigned)e[7] << 16));
    }
  }
  // (row, k = column)
  __device__ __forceinline__ void put(BMat& m) const {
    m.v[bpos(threadIdx.x >> 3, threadIdx.x & 7)] = q;
  }
  // transposed: (row = column, k = row)
  __device__ __forceinline__ void put_t(BMat& m) const {
    const int row = threadIdx.x >> 3, c0 = (threadIdx.x & 7) * 8;
    const u16* e = reinterpret_cast<const u16*>(&q);
#pragma unroll
    for (int x = 0; x < 8; ++x) *belem(m, c0 + x, row) = e[x];
  }
};

// fp32 block (rows x cols) of a padded 64 x 64 workspace matrix: thread idx holds
// rows (idx + 512 v) / 16, columns 4 ((idx + 512 v) % 16) + 0..3, v = 0, 1; zero
// outside the block.  Every row of a padded matrix is in the buffer, so the loads
// are unconditional and the block's bounds are applied when the tile is put: masking
// at the load made the wave wait for it there, before the loads that follow it were
// issued.
struct FTile {
  float4 f[2];
  int rows, cols;  // the block (wave-uniform)

  __device__ __forceinline__ void load(const float* src, int rows_, int cols_) {
    rows = rows_;
    cols = cols_;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const unsigned off = (threadIdx.x + v * NTB) * 4u;  // row idx / 16, columns 4 (idx % 16)
      f[v] = *reinterpret_cast<const float4*>(src + off);
    }
  }
  __device__ __forceinline__ float4 val(int v) const {
    const int idx = threadIdx.x + v * NTB, row = idx >> 4, c0 = (idx & 15) * 4;
    const int nc = row < rows ? cols - c0 : 0;  // components inside: min(nc, 4)
    return make_float4(nc > 0 ? f[v].x : 0.f, nc > 1 ? f[v].y : 0.f, nc > 2 ? f[v].z : 0.f,
                       nc > 3 ? f[v].w : 0.f);
  }
  __device__ __forceinline__ void put_split(BPair& m) const {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int idx = threadIdx.x + v * NTB;
      const float4 x = val(v);
      put_split4(m, idx >> 4, (idx & 15) * 4, x.x, x.y, x.z, x.w);
    }
  }
  // transposed: (row = column, k = row)
  __device__ __forceinline__ void put_split_t(BPair& m) const {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int idx = threadIdx.x + v * NTB, row = idx >> 4, c0 = (idx & 15) * 4;
      const float4 x = val(v);
      put_split1x2(m, c0 + 0, row, x.x, c0 + 1, row, x.y);
      put_split1x2(m, c0 + 2, row, x.z, c0 + 3, row, x.w);
    }
  }
};

// fp32 block (rows x cols) of a fragment-major workspace matrix (store_tile_frag's
// layout): thread idx holds entry e = idx + 512 v (v = 0, 1), i.e. tile t = e / 64 and
// lane L = e % 64 of it -- rows 16 (t / 4) + 4 (L / 16) + 0..3 of column 16 (t % 4) +
// L % 16 -- with one contiguous 16-byte load; zero outside the block.
struct FTileF {
  float4 f[2];
  int rows, cols;  // the block (wave-uniform); load_rowmajor applies it itself

  __device__ static __forceinline__ void coords(int v, int& d0, int& j) {
    const int e = threadIdx.x + v * NTB, t = e >> 6, L = e & 63;
    d0 = 16 * (t >> 2) + 4 * (L >> 4);
    j = 16 * (t & 3) + (L & 15);
  }
  __device__ __forceinline__ void load(const float* src, int rows_, int cols_) {
    rows = rows_;
    cols = cols_;
#pragma unroll
    for (int v = 0; v < 2; ++v)  // raw loads; the bounds are applied when used (as in FTile)
      f[v] = *reinterpret_cast<const float4*>(src + (threadIdx.x + v * NTB) * 4u);
  }
  // The same entries of a row-major matrix (row stride DN): four rows of one column.
  __device__ __forceinline__ void load_rowmajor(const float* src, int rows, int cols) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      int d0, j;
      coords(v, d0, j);
      const bool c = j < cols;
      f[v] = make_float4(ldf_or0(src, (d0 + 0) * DN + j, c && d0 + 0 < rows),
                         ldf_or0(src, (d0 + 1) * DN + j, c && d0 + 1 < rows),
                         ldf_or0(src, (d0 + 2) * DN + j, c && d0 + 2 < rows),
                         ldf_or0(src, (d0 + 3) * DN + j, c && d0 + 3 < rows));
    }
    this->rows = DN;  // already applied
    this->cols = DN;
  }
  __device__ __forceinline__ float4 val(int v) const {
    int d0, j;
    coords(v, d0, j);
    const int nr = j < cols ? rows - d0 : 0;  // components inside: min(nr, 4)
    return make_float4(nr > 0 ? f[v].x : 0.f, nr > 1 ? f[v].y : 0.f, nr > 2 ? f[v].z : 0.f,
                       nr > 3 ? f[v].w : 0.f);
  }
  // (row, k = column)
  __device__ __forceinline__ void put_split(BPair& m) const {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      int d0, j;
      coords(v, d0, j);
      const float4 x = val(v);
      put_split1x2(m, d0 + 0, j, x.x, d0 + 1, j, x.y);
      put_split1x2(m, d0 + 2, j, x.z, d0 + 3, j, x.w);
    }
  }
  // transposed: (row = column, k = row), four consecutive k per entry
  __device__ __forceinline__ void put_split_t(BPair& m) const {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      int d0, j;
      coords(v, d0, j);
      const float4 x = val(v);
      put_split4(m, j, d0, x.x, x.y, x.z, x.w);
    }
  }
};

// The wave's 16 x 32 output block (rows R0 + 4 g + i, columns C0 + 16 jj + r) into a
// bf16 row-major output with row stride ld, keeping rows < nr and columns < nc.
__device__ __forceinline__ void store_block_bf16(u16* dst, int64_t ld, const floatx4 (&v)[2],
                                                 int R0, int C0, int nr, int nc) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  u16* p = dst + (int64_t)(R0 + 4 * g) * ld + C0 + r;
  if (R0 + 16 <= nr && C0 + 32 <= nc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[0] = bf_bits(v[0][i]);
      p[16] = bf_bits(v[1][i]);
      p += ld;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool rok = R0 + 4 * g + i < nr;
      if (rok && C0 + r < nc) p[0] = bf_bits(v[0][i]);
      if (rok && C0 + 16 + r < nc) p[16] = bf_bits(v[1][i]);
      p += ld;
    }
  }
}

// The wave's 16 x 32 output block into a padded 64 x 64 fp32 workspace matrix.
__device__ __forceinline__ void store_block_f32(float* dst, const floatx4 (&v)[2], int R0, int C0) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  float* p = dst + (R0 + 4 * g) * DN + C0 + r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i * DN] = v[0][i];
    p[i * DN + 16] = v[1][i];
  }
}

// Fragment-major fp32 workspace matrix: the 16 x 16 tile (row block rb, column
// block cb) holds, for lane L = 16 g + r, rows 16 rb + 4 g + i (i = 0..3) of column
// 16 cb + r as 4 consecutive floats, so one wave moves a tile in accumulator layout
// with a single 16-byte access per lane (1 KiB contiguous).  The chains' fp32 chunk
// operands (B, Pu, b') use it: loaded with one instruction per tile instead of
// four, a step keeps fewer vector-memory operations in flight per wave.  So does the
// forward chain's state output Hb (one store per lane per step).
__device__ __forceinline__ void store_block_frag(float* dst, const floatx4 (&v)[2], int R0, int C0) {
  const int t0 = (R0 >> 4) * 4 + (C0 >> 4);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
    *reinterpret_cast<floatx4*>(dst + (t0 + jj) * 256 + lane_id() * 4) = v[jj];
}
__device__ __forceinline__ void store_tile_frag(float* dst, int rb, int cb, const floatx4& v) {
  *reinterpret_cast<floatx4*>(dst + (rb * 4 + cb) * 256 + lane_id() * 4) = v;
}
__device__ __forceinline__ floatx4 load_tile_frag(const float* src, int rb, int cb) {
  return *reinterpret_cast<const floatx4*>(src + (rb * 4 + cb) * 256 + lane_id() * 4);
}

// Split workspace matrix: a 64 x 64 row-major bf16 hi half followed by the lo
// half (the 16 KB of one padded fp32 matrix slot).  E is kept in this form for
// the gradient kernel's row reads; the chains' operands use the fragment order
// below.
constexpr int SPLIT_LO = DN * DN;  // u16 offset of the lo half

__device__ __forceinline__ void store_block_split(u16* dst, const floatx4 (&v)[2], int R0, int C0) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
  u16* p = dst + (R0 + 4 * g) * DN + C0 + r;
  // Value by value: splitting the pairs (tile 0, tile 1) of each row and storing
  // their high halves with global_store_short_d16_hi took the forward preparation
  // kernel from 199 to 212 us at C5.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      u16 hi, lo;
      bf_split(v[jj][i], hi, lo);
      p[i * DN + 16 * jj] = hi;
      p[SPLIT_LO + i * DN + 16 * jj] = lo;
    }
  }
}

// Split workspace matrix in A-fragment order: a hi half and a lo half of 4096
// bf16 each, laid out so that the MFMA A fragment of rows 16 rb..16 rb + 15 and
// k 32 s..32 s + 31 is 1 KB of consecutive memory, lane l's eight values at
// ((rb * 2 + s) * 64 + l) * 8.  Element (row, k) sits at
// ((row / 16 * 2 + k / 32) * 64 + 16 * (k / 8 % 4) + row % 16) * 8 + k % 8.  The
// chains read their operands back with one 16-byte load per fragment and half,
// and a wave's load covers 1 KB without gaps (the row-major form read 16 bytes
// from each of 64 rows).
//
// store_block_splitfrag writes the wave's 16 x 32 accumulator block (rows 16 rb,
// columns 32 ch) in that order.  The block is exactly the A fragment (rb, s = ch),
// so the wave puts it into its own block of an LDS pair `st`,
// reads back each lane's eight hi and eight lo values and stores each with one
// 16-byte write (writing the accumulator's values one by one to their fragment
// slots made the forward preparation kernel 15 us slower at C5).  Only this wave
// touches its block of `st`, and one wave's LDS operations complete in order; the
// empty asm statements keep the compiler from moving one lane's LDS write past
// another lane's read of it (a previous call's reads included).
__device__ __forceinline__ void store_block_splitfrag(BPair& st, const floatx4 (&v)[2],
                                                      const FragOff& F, u16* dst) {
  asm volatile("" ::: "memory");
  acc_put(st, v[0], 16 * F.rb, 32 * F.ch);
  acc_put(st, v[1], 16 * F.rb, 32 * F.ch + 16);
  asm volatile("" ::: "memory");
  const unsigned a = F.ch ? F.a[1] : F.a[0];
  const uint4 hi = __builtin_bit_cast(uint4, frag_at(st[0], a));
  const uint4 lo = __builtin_bit_cast(uint4, frag_at(st[1], a));
  const unsigned off = ((unsigned)(F.rb * 2 + F.ch) * 64u + lane_id()) * 8u;
  *reinterpret_cast<uint4*>(dst + off) = hi;
  *reinterpret_cast<uint4*>(dst + SPLIT_LO + off) = lo;
}

// Split operands from a 64 x 64 fp32 LDS matrix (row stride LD), one chunk of 8
// k per thread: (row, k) = src[row][k], and the transposed forms (row, k) =
// src[k][row] and src[k][row] * scale[k].
__device__ __forceinline__ void stage_split(BPair& m, BPair& mt, BPair& mts, const float* src,
                                            const float* scale) {
  const int row = threadIdx.x >> 3, q = threadIdx.x & 7;
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = src[row * LD + 8 * q + e];
  put_split8(m, row, q, x);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = src[(8 * q + e) * LD + row];
  put_split8(mt, row, q, x);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] *= scale[8 * q + e];
  put_split8(mts, row, q, x);
}

// The serial chains carry each chunk as one affine map of the state, built
// here in parallel over chunks (the products with K^T are done where K^T is
// already in LDS):
//   forward   H <- H + A H + B,     A = -K^T diag(beta) W,  B = K^T diag(beta) U0,
//             y  = Qe H + Pu,       Qe = Q - P W,           Pu = P U0
//   backward  dH <- dH + A' dH + b', A' = -K^T E,  b' = Q^T dy - K^T G0
// (U = U0 - W H and G = G0 + E dH substituted into the chunk recurrences).
// The identity part of each map stays exact: the chains add A H to H in fp32.

// ---------------------------------------------------------------------------
// forward, preparation kernel: one workgroup per (chunk, head)
// ---------------------------------------------------------------------------
//   L = strict(K K^T) * beta_col, T = (I + L)^-1 (fp32, blocked),
//   P = (Q K^T) * beta_col * read, M1 = (beta K)^T T, M2 = P T;
//   A = -M1 K, B = M1 V, Qe = Q - M2 K, Pu = M2 V
//   -> A, Qe (split bf16 pairs, A-fragment order), B, Pu (fp32, fragment-major) in the
//      workspace, and T^T's nonzero row chunks (fp32, packed: tri_chunk) to To for the
//      backward.
// (W = T K and U0 = T V never materialise: A = -K^T diag(beta) W = -M1 K, etc.)
// LDS stays under 80 KB, so two workgroups share a CU.
// GATED (per-token decay, decay tables in mg_delta.h): L and P are weighted by
// the span factors E, M1 = (a beta K)^T T, A = -M1 (p K), Qe = ptok Q - M2 (p K),
// and the chunk's vector region (a beta, ptok, p, PC) is written for the chains.
// The span table lives in T's buffer until the inverse, and the split (p K)^T in
// the buffer of T^T once M1 and M2 are formed, so the LDS plan is unchanged.
template <bool GATED>
__global__ __launch_bounds__(NTB) void dwb_fwd_prep(const u16* __restrict__ Q,
                                                    const u16* __restrict__ K,
                                                    const u16* __restrict__ V,
                                                    const u16* __restrict__ beta,
                                                    const float* __restrict__ lg,
                                                    float* __restrict__ Ao, float* __restrict__ Bo,
                                                    float* __restrict__ Qeo,
                                                    float* __restrict__ Puo,
                                                    float* __restrict__ vo,
                                                    float* __restrict__ To, DwGeom g) {
  __shared__ BMat sKt, sVt;                    // K^T, V^T as (col; m)
  __shared__ BMat sX[2];                       // K, Q; then P split; then M2 split
  __shared__ uint4 sLraw[(DN * LD + 3) / 4];   // L (fp32); then T^T split
  __shared__ uint4 sTraw[(DN * LD + 3) / 4];   // T (fp32); then (beta K)^T split; then M1 split
  __shared__ float sY[2 * 32 * LDS16];
  __shared__ float sb[DN];
  __shared__ float sdec[GATED ? 5 * DN : 1];  // l, Lc, p, a beta, ptok
  float* sL = reinterpret_cast<float*>(sLraw);
  float* sT = reinterpret_cast<float*>(sTraw);
  float* sE = sT;  // span table until the inverse
  float *sl = sdec, *sLc = sdec + DN, *sp = sdec + 2 * DN, *sab = sdec + 3 * DN,
        *spt = sdec + 4 * DN;
  BMat &sK = sX[0], &sQ = sX[1];
  BPair& sP = sX;
  BPair& sM2 = sX;
  BPair& sTt = *reinterpret_cast<BPair*>(sLraw);
  BPair& sPKt = *reinterpret_cast<BPair*>(sLraw);  // (d; m) = p_m K[m][d], gated
  BPair& sBKt = *reinterpret_cast<BPair*>(sTraw);
  BPair& sM1 = *reinterpret_cast<BPair*>(sTraw);
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const int64_t trow0 = bh * g.T + ch.t0;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  FragOff F;
  F.init();
  const int lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int R0 = 16 * F.rb, C0 = 32 * F.ch;
  float qv[2][4];  // Q at the wave's output positions of Qe
  {
    BTile tk, tv, tq;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tv.load(V + row0 * g.dv, ch.M, g.dv, g.dv);
    tq.load(Q + trow0 * g.dk, ch.Ct, g.dk, g.dk);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = R0 + 4 * gg + i, d = C0 + 16 * jj + r;
        qv[jj][i] = ldf_or0(Q, (trow0 + t) * g.dk + d, t < ch.Ct && d < g.dk);
      }
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    tk.put(sK);
    tk.put_t(sKt);
    tv.put_t(sVt);
    tq.put(sQ);
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
    if constexpr (GATED) {
      const float lv = ld_l(lg, bh, g, ch);
      sl[threadIdx.x & (DN - 1)] = lv;
    }
  }
  __syncthreads();
  if constexpr (GATED) {
    decay_tables<NTB>(sl, sE);
    decay_vectors(sl, sb, ch, g.nh, sLc, sp, sab, spt);
    __syncthreads();
  }
  floatx4 pp[2];
  {
    floatx4 kk[2];
    zero2(kk);
    zero2(pp);
    bmm<false, false>(kk, F, &sK, &sK);  // K K^T
    bmm<false, false>(pp, F, &sQ, &sK);  // Q K^T
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int cj = C0 + 16 * jj;
      // Masked values are formed before the masks pick them, and each mask picks
      // between a local and zero: a conditional whose arm computes (or reads LDS)
      // becomes a branch, the LDS read is moved into it and waited for there, one
      // read at a time.  Every index is in range.
      const float bc = sb[cj + r];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = R0 + 4 * gg + i, col = cj + r;
        float kv, pv;
        if constexpr (GATED) {  // spans between the tokens of micro-rows (tau = m / nh)
          const int tc = col / g.nh;
          kv = kk[jj][i] * bc * sE[(row / g.nh) * LD + tc];
          pv = pp[jj][i] * bc * sE[row * LD + tc];
        } else {
          kv = kk[jj][i] * bc;
          pv = pp[jj][i] * bc;
        }
        kk[jj][i] = col < row ? kv : 0.f;
        pp[jj][i] = col < (row + 1) * g.nh ? pv : 0.f;
      }
      acc_store_lds(kk[jj], sL + R0 * LD + cj, LD);
    }
  }
  __syncthreads();  // K and Q are free (and, gated, the span table)
  if constexpr (GATED) write_vectors(vo + ((size_t)bh * g.nc + c) * VECN, sLc, sp, sab, ch);
  acc_put(sP, pp[0], R0, C0);  // P as (t; m): the B operand of M2^T
  acc_put(sP, pp[1], R0, C0 + 16);
  unit_lower_inverse(sL, sT, sY);  // ends with a barrier: sL is free
  {
    const int row = threadIdx.x >> 3, q = threadIdx.x & 7;
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = sT[(8 * q + e) * LD + row];
    put_split8(sTt, row, q, x);  // (m; m') = T[m'][m]
    // T^T's nonzero chunks, packed, for the backward preparation kernel, which
    // would otherwise form L and invert it again.
    if (q >= row >> 3) {
      float4* t = reinterpret_cast<float4*>(To + mat + 8 * tri_chunk(row, q));
      t[0] = make_float4(x[0], x[1], x[2], x[3]);
      t[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
  }
  __syncthreads();  // sT is free
  {
    const int row = threadIdx.x >> 3, q = threadIdx.x & 7;
    const uint4 kq = sKt.v[bpos(row, q)];
    const u16* e = reinterpret_cast<const u16*>(&kq);
    float x[8];
    const float* sc = GATED ? sab : sb;
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = sc[8 * q + k] * bf_val(e[k]);
    put_split8(sBKt, row, q, x);  // (d; m) = beta_m K[m][d]  (gated: a_m beta_m K[m][d])
  }
  __syncthreads();
  {
    floatx4 m1[2], m2[2];
    zero2(m1);
    zero2(m2);
    bmm<true, true>(m1, F, sTt, sBKt);  // M1^T = T^T diag(beta) K   (rows m, cols d)
    bmm<true, true>(m2, F, sTt, sP);    // M2^T = (P T)^T           (rows m, cols t)
    __syncthreads();  // sBKt and sP are free
    acc_put_t(sM1, m1[0], R0, C0);  // M1 as (d; m)
    acc_put_t(sM1, m1[1], R0, C0 + 16);
    acc_put_t(sM2, m2[0], R0, C0);  // M2 as (t; m)
    acc_put_t(sM2, m2[1], R0, C0 + 16);
    if constexpr (GATED) {  // T^T is free: (p K)^T as a split pair
      const int row = threadIdx.x >> 3, q = threadIdx.x & 7;
      const uint4 kq = sKt.v[bpos(row, q)];
      const u16* e = reinterpret_cast<const u16*>(&kq);
      float x[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = sp[8 * q + k] * bf_val(e[k]);
      put_split8(sPKt, row, q, x);
    }
  }
  __syncthreads();
  {
    floatx4 a2[2], b2[2], qe[2], pu[2];
    zero2(a2);
    zero2(b2);
    zero2(pu);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        qe[jj][i] = GATED ? qv[jj][i] * spt[R0 + 4 * gg + i] : qv[jj][i];
    if constexpr (GATED) {
      bmm<true, true, true>(a2, F, sM1, sPKt);  // A = -M1 (p K)
      bmm<true, true, true>(qe, F, sM2, sPKt);  // Qe = ptok Q - M2 (p K)
    } else {
      bmm<true, false, true>(a2, F, sM1, &sKt);  // A = -M1 K
      bmm<true, false, true>(qe, F, sM2, &sKt);  // Qe = Q - M2 K
    }
    bmm<true, false>(b2, F, sM1, &sVt);  // B = M1 V
    bmm<true, false>(pu, F, sM2, &sVt);  // Pu = M2 V
    store_block_frag(Bo + mat, b2, R0, C0);
    store_block_frag(Puo + mat, pu, R0, C0);
    // A and Qe leave through T^T's pair, free since M1 and M2 were formed (gated:
    // it holds (p K)^T, which every wave has read once past the barrier).
    if constexpr (GATED) __syncthreads();
    store_block_splitfrag(sTt, a2, F, reinterpret_cast<u16*>(Ao + mat));
    store_block_splitfrag(sTt, qe, F, reinterpret_cast<u16*>(Qeo + mat));
  }
}

// A fragments of a row-major bf16 input block (rows x cols, row stride ld):
// row `row`, chunks g and 4 + g, zero outside the block.
__device__ __forceinline__ void load_in_frag(uint4 (&a)[2], const u16* src, int64_t ld, int row,
                                             int rows, int cols) {
  const int g = lane_id() >> 4;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int c0 = 8 * (4 * s + g);
    const u16* p = src + (int64_t)row * ld + c0;
    if (row < rows && c0 + 8 <= cols && ld == DN) {
      a[s] = *reinterpret_cast<const uint4*>(p);
    } else {
      u16 e[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) e[x] = (row < rows && c0 + x < cols) ? p[x] : (u16)0;
      a[s] = make_uint4(e[0] | ((unsigned)e[1] << 16), e[2] | ((unsigned)e[3] << 16),
                        e[4] | ((unsigned)e[5] << 16), e[6] | ((unsigned)e[7] << 16));
    }
  }
}

// acc[jj] += A . B[row block 2 ch + jj]^T with A an exact bf16 operand whose two
// fragments (the wave's rows, chunks g and 4 + g) are held in registers.
template <bool SB>
__device__ __forceinline__ void rmm(floatx4 (&acc)[2], const FragOff& F, const uint4 (&a)[2],
                                    const BMat* B) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bf16x8 ah = __builtin_bit_cast(bf16x8, a[s]);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, frag_at(B[0], F.b[s][jj]), acc[jj], 0, 0, 0);
      if constexpr (SB)
        acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, frag_at(B[1], F.b[s][jj]), acc[jj], 0, 0, 0);
    }
  }
}

// ---- register operands built from LDS ---------------------------------------------
// An fp32 A fragment as a split pair: x[e] = hi + lo (about 16 significant bits).
__device__ __forceinline__ void split_frag(const float (&x)[8], uint4& hi, uint4& lo) {
  unsigned h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) bf_split2(x[2 * p], x[2 * p + 1], h[p], l[p]);
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// Split A fragments of rows R0 + r of an fp32 LDS matrix (row stride LD): with
// TRANS, row m of its transpose (x = T[k][m]), optionally times scale[k].
template <bool TRANS>
__device__ __forceinline__ void t_frags(uint4 (&hi)[2], uint4 (&lo)[2], const float* T, int R0,
                                        const float* scale) {
  const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int k0 = 8 * (4 * s + g);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = TRANS ? T[(k0 + e) * LD + R0 + r] : T[(R0 + r) * LD + k0 + e];
      if (scale) x[e] *= scale[k0 + e];
    }
    split_frag(x, hi[s], lo[s]);
  }
}

// Fragments of the transpose of an exact bf16 BMat, gathered by column: row n of
// M^T, i.e. (k, n) elements M[k][n] for the lane's 8 consecutive k.
__device__ __forceinline__ uint4 col_frag(const BMat& M, int n, int s) {
  const int k0 = 8 * (4 * s + (lane_id() >> 4));
  const u16* base = reinterpret_cast<const u16*>(&M);
  unsigned p[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int k = k0 + 2 * e;
    const u16 a = base[bpos(k, n >> 3) * 8 + (n & 7)], b = base[bpos(k + 1, n >> 3) * 8 + (n & 7)];
    p[e] = a | ((unsigned)b << 16);
  }
  return make_uint4(p[0], p[1], p[2], p[3]);
}

// acc[jj] (+/-)= A . B[row block 2 ch + jj]^T with A a split pair in registers and
// B a split pair in LDS (hi hi + hi lo + lo hi) or, with !SB, an exact BMat.
template <bool SB, bool NEG = false>
__device__ __forceinline__ void smm(floatx4 (&acc)[2], const FragOff& F, const uint4 (&ah)[2],
                                    const uint4 (&al)[2], const BMat* B) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bf16x8 h = __builtin_bit_cast(bf16x8, ah[s]), l = __builtin_bit_cast(bf16x8, al[s]);
    if constexpr (NEG) {
      h = bneg(h);
      l = bneg(l);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const bf16x8 bh = frag_at(B[0], F.b[s][jj]);
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h, bh, acc[jj], 0, 0, 0);
      if constexpr (SB)
        acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h, frag_at(B[1], F.b[s][jj]), acc[jj], 0, 0, 0);
      acc[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l, bh, acc[jj], 0, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// backward, preparation kernel: one workgroup per (chunk, head)
// ---------------------------------------------------------------------------
//   T = (I + L)^-1, L = strict(K K^T) * beta_col: read as the forward formed it
//   R = V - K Hc, U = T R, P = (Q K^T) * beta_col * read, D1 = P^T dy
//   E = T^T diag(beta) K, G0 = T^T D1, QdY = Q^T dy
//   -> U, G0 (fp32), E (split) for the gradients; A' (split), b' (fp32, fragment-major) for the
//      reverse chain.
// GATED: L and P weighted by the span factors, R = V - diag(p) K Hc,
// E = T^T diag(a beta) K, b' = Q^T diag(ptok) dy - (p K)^T G0, A' = -(p K)^T E, with
// the span weights between the tokens tau(m) = m / nh of the micro-rows.
//
// The products run in dependency order so that few 64 x 64 operands are live at
// once, and LDS stays under 80 KB (two workgroups per CU):
//   A  T^T (fp32) from the forward, written into LDS as T; the gated span table
//      sits in a split region that is still free;
//   B  Hc^T (split) -> R = V - K Hc, V read per element from memory -> R^T (split);
//   C  U = T R;
//   D  P = Q K^T with Q as register fragments -> P^T (split); Q^T dy; D1 = P^T dy;
//   E  G0 = T^T D1 -> G0^T; E = (T diag(beta))^T K;  F  A' and b' from E^T, G0^T.
// Every operand derived from T (rows of T, of T^T, of (T diag(beta))^T) is split
// into registers straight from the fp32 T, the K^T operands are gathered by column
// from K, and the gated diag(ptok) and diag(p) scalings are applied to those
// register operands, so none of them takes LDS.
template <bool GATED>
__global__ __launch_bounds__(NTB) void dwb_bwd_prep(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ beta, const float* __restrict__ lg, const u16* __restrict__ dy,
    const float* __restrict__ Hb, const float* __restrict__ Tin, float* __restrict__ Uo,
    float* __restrict__ Eo, float* __restrict__ G0o, float* __restrict__ Apo,
    float* __restrict__ bpo, float* __restrict__ vo, DwGeom g) {
  __shared__ BMat sK;        // K as (m; d), exact
  __shared__ BMat sQD[2];    // Q^T as (d; t), dy^T as (j; t), exact
  __shared__ BPair sR1;      // [gated span table] -> Hc^T -> P^T -> G0^T
  __shared__ BPair sR2;      // R^T -> D1^T -> E^T
  __shared__ float sT[DN * LD];  // T, as the forward preparation kernel formed it
  __shared__ float sb[DN];
  __shared__ float sdec[GATED ? 5 * DN : 1];  // l, Lc, p, a beta, ptok
  float *sl = sdec, *sLc = sdec + DN, *sp = sdec + 2 * DN, *sab = sdec + 3 * DN,
        *spt = sdec + 4 * DN;
  BMat &sQt = sQD[0], &sDyt = sQD[1];
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const int64_t trow0 = bh * g.T + ch.t0;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  FragOff F;
  F.init();
  const int lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int R0 = 16 * F.rb, C0 = 32 * F.ch;
  FTileF th;  // Hc, staged in stage B
  // V at the wave's positions of R (stage B) and Q as A fragments (stage D): loaded
  // with the tiles, so the first barrier waits for all of them at once instead of
  // each stage paying its own memory round trip.
  float vpre[2][4];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = R0 + 4 * gg + i, j = C0 + 16 * jj + r;
      vpre[jj][i] = ldf_or0(V, (row0 + m) * g.dv + j, m < ch.M && j < g.dv);
    }
  uint4 qf[2];
  load_in_frag(qf, Q + trow0 * g.dk, g.dk, R0 + r, ch.Ct, g.dk);
  {
    BTile tk, tq, td;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tq.load(Q + trow0 * g.dk, ch.Ct, g.dk, g.dk);
    td.load(dy + trow0 * g.dv, ch.Ct, g.dv, g.dv);
    th.load(Hb + mat, g.dk, g.dv);
    // T^T row tr, columns 8 tc..8 tc + 7, written back transposed (row stride LD:
    // the 64 lanes of a wave write 64 distinct banks).  The forward stores only the
    // packed chunks that can be nonzero; the others read a zero vector.
    const int tr = threadIdx.x >> 3, tc = threadIdx.x & 7;
    const bool tnz = tc >= tr >> 3;
    const float4* tsrc =
        reinterpret_cast<const float4*>(Tin + mat + 8 * tri_chunk(tr, tnz ? tc : tr >> 3));
    const float4 t0 = *(tnz ? tsrc : reinterpret_cast<const float4*>(&mg_zero16));
    const float4 t1 = *(tnz ? tsrc + 1 : reinterpret_cast<const float4*>(&mg_zero16));
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    tk.put(sK);
    tq.put_t(sQt);
    td.put_t(sDyt);
    float* tcol = sT + 8 * tc * LD + tr;
    tcol[0] = t0.x;
    tcol[LD] = t0.y;
    tcol[2 * LD] = t0.z;
    tcol[3 * LD] = t0.w;
    tcol[4 * LD] = t1.x;
    tcol[5 * LD] = t1.y;
    tcol[6 * LD] = t1.z;
    tcol[7 * LD] = t1.w;
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
    if constexpr (!GATED) th.put_split_t(sR1);  // Hc^T as (j; d): sR1 is free from the start
    if constexpr (GATED) {
      const float lv = ld_l(lg, bh, g, ch);
      sl[threadIdx.x & (DN - 1)] = lv;
    }
  }
  __syncthreads();
  // ---- A: T = (I + L)^-1 is in sT (formed by the forward preparation kernel) ----
  // gated: the span weights of P at the wave's fragment positions (token row,
  // micro-row col: E[row][tau(col)]).
  float ewp[2][4];
  if constexpr (GATED) {
    float* sE = reinterpret_cast<float*>(&sR1);  // span table, row stride DN
    decay_tables<NTB, DN>(sl, sE);
    decay_vectors(sl, sb, ch, g.nh, sLc, sp, sab, spt);
    write_vectors(vo + ((size_t)bh * g.nc + c) * VECN, sLc, sp, sab, ch);  // wave 0's own values
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = R0 + 4 * gg + i, col = C0 + 16 * jj + r;
        const float e = sE[row * DN + col / g.nh];  // read first, then picked
        ewp[jj][i] = col < (row + 1) * g.nh ? e : 0.f;
      }
    __syncthreads();  // the span table is read: Hc^T takes its region
  }
  // ---- B: R = V - K Hc (gated: V - diag(p) K Hc) -> R^T ----
  if constexpr (GATED) {  // the span table held sR1 until now
    th.put_split_t(sR1);  // Hc^T as (j; d)
    __syncthreads();
  }
  {
    floatx4 rr[2];
    zero2(rr);
    bmm<false, true>(rr, F, &sK, sR1);  // K Hc
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int cj = C0 + 16 * jj;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = R0 + 4 * gg + i;
        rr[jj][i] = fmaf(GATED ? -sp[m] : -1.f, rr[jj][i], vpre[jj][i]);
      }
      acc_put_t(sR2, rr[jj], R0, cj);
    }
  }
  __syncthreads();
  // ---- C: U = T R ----
  {
    uint4 ah[2], al[2];
    t_frags<false>(ah, al, sT, R0, nullptr);
    floatx4 u[2];
    zero2(u);
    smm<true>(u, F, ah, al, sR2);
    store_block_f32(Uo + mat, u, R0, C0);
  }
  // ---- D: P = (Q K^T) * beta_col * read -> P^T; qd = Q^T dy; D1 = P^T dy ----
  floatx4 qd[2];  // Q^T dy (gated: Q^T diag(ptok) dy), kept for b'
  zero2(qd);
  {
    floatx4 pp[2];
    zero2(pp);
    rmm<false>(pp, F, qf, &sK);  // Q K^T
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int cj = C0 + 16 * jj;
      const float bc = sb[cj + r];  // masked value formed first, then picked
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = R0 + 4 * gg + i, col = cj + r;
        const float pv = GATED ? pp[jj][i] * bc * ewp[jj][i] : pp[jj][i] * bc;
        pp[jj][i] = col < (row + 1) * g.nh ? pv : 0.f;
      }
      acc_put_t(sR1, pp[jj], R0, cj);  // P^T as (m; t)
    }
  }
  if constexpr (GATED) {  // (Q diag(ptok))^T as split register fragments
    uint4 ah[2], al[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int k0 = 8 * (4 * s + gg);
      const uint4 qv = sQt.v[bpos(R0 + r, 4 * s + gg)];
      const u16* e = reinterpret_cast<const u16*>(&qv);
      float x[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) x[q] = bf_val(e[q]) * spt[k0 + q];
      split_frag(x, ah[s], al[s]);
    }
    smm<false>(qd, F, ah, al, &sDyt);
  } else {
    bmm<false, false>(qd, F, &sQt, &sDyt);  // Q^T dy
  }
  __syncthreads();  // P^T complete; every wave is past C (R^T free)
  {
    floatx4 d1[2];
    zero2(d1);
    bmm<true, false>(d1, F, sR1, &sDyt);  // P^T dy
    acc_put_t(sR2, d1[0], R0, C0);        // D1^T as (j; m)
    acc_put_t(sR2, d1[1], R0, C0 + 16);
  }
  __syncthreads();
  // ---- E: G0 = T^T D1 -> G0^T; E = (T diag(s))^T K, s = beta (gated: a beta) ----
  floatx4 ev[2];
  {
    uint4 ah[2], al[2];
    t_frags<true>(ah, al, sT, R0, nullptr);
    floatx4 g0[2];
    zero2(g0);
    smm<true>(g0, F, ah, al, sR2);
    store_block_f32(G0o + mat, g0, R0, C0);
    acc_put_t(sR1, g0[0], R0, C0);  // G0^T as (j; m); P^T is free
    acc_put_t(sR1, g0[1], R0, C0 + 16);
    t_frags<true>(ah, al, sT, R0, GATED ? sab : sb);
    zero2(ev);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bf16x8 h = __builtin_bit_cast(bf16x8, ah[s]), l = __builtin_bit_cast(bf16x8, al[s]);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const bf16x8 kb = __builtin_bit_cast(bf16x8, col_frag(sK, C0 + 16 * jj + r, s));
        ev[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h, kb, ev[jj], 0, 0, 0);
        ev[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l, kb, ev[jj], 0, 0, 0);
      }
    }
    store_block_split(reinterpret_cast<u16*>(Eo + mat), ev, R0, C0);
  }
  __syncthreads();  // D1^T read by every wave
  acc_put_t(sR2, ev[0], R0, C0);  // E^T as (d; m)
  acc_put_t(sR2, ev[1], R0, C0 + 16);
  __syncthreads();
  // ---- F: A' = -K^T E, b' = qd - K^T G0 (gated: (p K)^T) ----
  {
    floatx4 a2[2];
    zero2(a2);
    if constexpr (GATED) {
      uint4 ah[2], al[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int k0 = 8 * (4 * s + gg);
        const uint4 kv = col_frag(sK, R0 + r, s);
        const u16* e = reinterpret_cast<const u16*>(&kv);
        float x[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = bf_val(e[q]) * sp[k0 + q];
        split_frag(x, ah[s], al[s]);
      }
      smm<true, true>(a2, F, ah, al, sR2);  // -(p K)^T E
      smm<true, true>(qd, F, ah, al, sR1);  // b' = Q^T diag(ptok) dy - (p K)^T G0
    } else {
      uint4 kf[2];
      kf[0] = col_frag(sK, R0 + r, 0);
      kf[1] = col_frag(sK, R0 + r, 1);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 a = bneg(__builtin_bit_cast(bf16x8, kf[s]));
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const unsigned off = F.b[s][jj];
          a2[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, frag_at(sR2[0], off), a2[jj], 0, 0, 0);
          a2[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, frag_at(sR2[1], off), a2[jj], 0, 0, 0);
          qd[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, frag_at(sR1[0], off), qd[jj], 0, 0, 0);
          qd[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, frag_at(sR1[1], off), qd[jj], 0, 0, 0);
        }
      }
    }
    store_block_frag(bpo + mat, qd, R0, C0);
    store_block_splitfrag(sQD, a2, F, reinterpret_cast<u16*>(Apo + mat));  // Q^T, dy^T are free
  }
}

// ---------------------------------------------------------------------------
// backward, gradient kernel: one workgroup per (chunk, head)
// ---------------------------------------------------------------------------
//   G = G0 + E dHn, dV = G
//   S = Q K^T, dP = dy U^T, dS = dP * beta_col * read         (rows t, cols m)
//   dQ = dy Hc^T + dS K
//   dT = -G U^T, D2 = dT * beta_col * strict + (dT * beta_col * strict)^T
//   dK = dS^T Q - G Hc^T + D2 K + beta_row (U dHn^T)
//   dbeta_m = sum_t dP S read + sum_i dT KK strict + sum_d K[m][d] (U dHn^T)[m][d]
// Q and dy enter the products as A fragments straight from memory; the split
// operands rotate through three 16 KB regions, so LDS stays under 80 KB (two
// workgroups per CU).  D2 is symmetrised in registers from dT and dT^T = -U G^T.
// GATED (decay tables in mg_delta.h): the products are weighted as in
// the forward -- dS = (dy U^T) beta_col E_read, D2 = (-G U^T) beta E_mm (both
// triangles), dQ = diag(ptok) dy Hc^T + dS K, dK = -diag(p) G Hc^T + dS^T Q + D2 K
// + diag(a beta) U dHn^T, dbeta's U (K dHn) term times a -- and the span
// gradients F[t][t'] = dP P + dT L (token level, registers), the row Ct-1 term
// a beta rowsum(U (K dHn)) and f[t] (ptok: ptok_t sum_d Q (dy Hc^T), p: p_m
// sum_d K (-G Hc^T), PC: PC <dHn, Hc>) give dl_s = sum_{t >= s} (f[t] +
// sum_{t' < s} F[t][t']) by wave-level prefix scans.  The span table needs its
// own 16 KB and the span gradients stay in registers to the end (about 180 VGPRs),
// so a gated workgroup has the CU to itself.
template <bool GATED>
__global__ __launch_bounds__(NTB, GATED ? 2 : 4) void dwb_bwd_grads(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ beta,
    const float* __restrict__ lg, const u16* __restrict__ dy, const float* __restrict__ Hb,
    const float* __restrict__ dHn, const float* __restrict__ Um, const float* __restrict__ Em,
    const float* __restrict__ G0m, u16* __restrict__ dQ, u16* __restrict__ dK,
    u16* __restrict__ dV, u16* __restrict__ dbeta, float* __restrict__ dlg, DwGeom g) {
  __shared__ BMat sK, sKt, sQt;  // exact inputs
  // Split regions: [E, dHn^T] -> [G, U, Hc] -> [dS, U, dS^T] -> [D2, U, dHn].  The gated
  // form runs one workgroup per CU anyway (registers), so it takes three more regions and
  // no result overwrites an operand that other waves may still read: regions
  // 0, 1 = E, dHn^T -> dS, dS^T and 3, 4, 5 = G, U, Hc -> D2, U, dHn, which drops the
  // three barriers that only waited for those reads.
  __shared__ BPair sR[GATED ? 6 : 3];
  constexpr int RG = GATED ? 3 : 0, RU = GATED ? 4 : 1, RH = GATED ? 5 : 2;
  constexpr int RDS = 0, RDST = GATED ? 1 : 2, RD2 = RG, RDHN = RH;
  __shared__ float sb[DN];
  // dbeta partials: [0..3] read-term column sums per row block, [4..7] strict-term
  // column sums per row block, [8..9] row sums of K * (U dHn^T) per column half.
  __shared__ float sdb[10][DN];
  // gated: span table; l, Lc, p, a beta, a, ptok; f partials (ptok and p terms per
  // column half); <dHn, Hc> per wave; dl partials per wave.
  __shared__ float sEg[GATED ? DN * LD : 1];
  __shared__ float sdec[GATED ? 6 * DN : 1];
  __shared__ float sfp[GATED ? 4 * DN : 1];
  __shared__ float sred[GATED ? WB : 1];
  __shared__ float sdl[GATED ? WB * DN : 1];
  float *sl = sdec, *sLc = sdec + DN, *sp = sdec + 2 * DN, *sab = sdec + 3 * DN,
        *sa = sdec + 4 * DN, *spt = sdec + 5 * DN;
  const int c = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const Chunk ch = chunk_of(g, c);
  const int64_t row0 = (bh * g.T + ch.t0) * g.nh;
  const int64_t trow0 = bh * g.T + ch.t0;
  const size_t mat = ((size_t)bh * g.nc + c) * MAT;
  FragOff F;
  F.init();
  const int lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int R0 = 16 * F.rb, C0 = 32 * F.ch;
  floatx4 gacc[2];
  {
    BTile tk, tq;
    FTile tn;
    tk.load(K + row0 * g.dk, ch.M, g.dk, g.dk);
    tq.load(Q + trow0 * g.dk, ch.Ct, g.dk, g.dk);
    tn.load(dHn + mat, g.dk, g.dv);
    const u16* es = reinterpret_cast<const u16*>(Em + mat);
    const int erow = threadIdx.x >> 3, eq = threadIdx.x & 7;
    const uint4 ehi = *reinterpret_cast<const uint4*>(es + erow * DN + 8 * eq);
    const uint4 elo = *reinterpret_cast<const uint4*>(es + SPLIT_LO + erow * DN + 8 * eq);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) gacc[jj] = acc_load_ws(G0m + mat + R0 * DN + C0 + 16 * jj);
    const float bv = ldf_or0(beta, row0 + (threadIdx.x & (DN - 1)), (threadIdx.x & (DN - 1)) < ch.M);
    tk.put(sK);
    tk.put_t(sKt);
    tq.put_t(sQt);
    sR[0][0].v[bpos(erow, eq)] = ehi;
    sR[0][1].v[bpos(erow, eq)] = elo;
    tn.put_split_t(sR[1]);
    sb[threadIdx.x & (DN - 1)] = bv;  // every wave stores the same values (no branch)
    if constexpr (GATED) {
      const float lv = ld_l(lg, bh, g, ch);
      sl[threadIdx.x & (DN - 1)] = lv;
    }
  }
  __syncthreads();
  if constexpr (GATED) {
    decay_tables<NTB>(sl, sEg);
    decay_vectors(sl, sb, ch, g.nh, sLc, sp, sab, spt, sa);
  }
  {
    // U and Hc are fetched while G forms, and staged once E and dHn^T are free.
    FTile tu;
    FTileF th;
    tu.load(Um + mat, ch.M, g.dv);
    th.load(Hb + mat, g.dk, g.dv);
    bmm<true, true>(gacc, F, sR[0], sR[1]);  // G = G0 + E dHn   (rows m, cols j)
    store_block_bf16(dV + row0 * g.dv, g.dv, gacc, R0, C0, ch.M, g.dv);
    if constexpr (GATED) {  // <dHn, Hc> from two fp32 tiles of the same layout
      FTileF tn2;  // dHn at th's positions (row-major source)
      tn2.load_rowmajor(dHn + mat, g.dk, g.dv);
      float part = 0.f;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const float4 a = tn2.val(v), b = th.val(v);
        part += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
      }
      part = mg_group_sum<64>(part);
      if (lane == 0) sred[wave_id()] = part;
    }
    if constexpr (!GATED) __syncthreads();  // E and dHn^T are read
    acc_put(sR[RG], gacc[0], R0, C0);  // G as (m; j)
    acc_put(sR[RG], gacc[1], R0, C0 + 16);
    tu.put_split(sR[RU]);              // U as (m; j)
    th.put_split(sR[RH]);              // Hc as (d; j)
  }
  uint4 qf[2], yf[2];  // Q and dy fragments of the wave's rows t
  load_in_frag(qf, Q + trow0 * g.dk, g.dk, R0 + r, ch.Ct, g.dk);
  load_in_frag(yf, dy + trow0 * g.dv, g.dv, R0 + r, ch.Ct, g.dv);
  __syncthreads();
  BPair &sG = sR[RG], &sU = sR[RU], &sHc = sR[RH];
  floatx4 ds2[2], d2[2], dq[2], dk[2];
  // gated: span gradients at the wave's positions: f1 of the (token t, micro-row m)
  // products, f2 of the (micro-row m, micro-row j) ones.
  floatx4 f1[2], f2[2];
  {
    floatx4 s2[2], dp2[2];
    zero2(s2);
    zero2(dp2);
    rmm<false>(s2, F, qf, &sK);  // S = Q K^T
    rmm<true>(dp2, F, yf, sU);   // dP = dy U^T
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int cj = C0 + 16 * jj;
      // Masked values are formed before the masks pick them, and each mask picks
      // between a local and zero: a conditional whose arm computes (or reads LDS)
      // becomes a branch, the LDS read is moved into it and waited for there, one
      // read at a time.  Every index is in range.
      const float bm = sb[cj + r];
      floatx4 db;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = R0 + 4 * gg + i, m = cj + r;
        const bool rd = m < (t + 1) * g.nh;
        if constexpr (GATED) {
          const float e = sEg[t * LD + m / g.nh];
          const float er = rd ? e : 0.f;
          ds2[jj][i] = dp2[jj][i] * bm * er;
          db[i] = dp2[jj][i] * s2[jj][i] * er;
          f1[jj][i] = db[i] * bm;
        } else {
          const float dv = dp2[jj][i] * bm, bv = dp2[jj][i] * s2[jj][i];
          ds2[jj][i] = rd ? dv : 0.f;
          db[i] = rd ? bv : 0.f;
        }
      }
      colsum16(db, sdb[F.rb], cj + r);
    }
  }
  {
    floatx4 dt2[2], dtt2[2], kk2[2];
    zero2(dt2);
    zero2(dtt2);
    zero2(kk2);
    bmm<true, true, true>(dt2, F, sG, sU);   // dT = -G U^T
    bmm<true, true, true>(dtt2, F, sU, sG);  // dT^T = -U G^T
    bmm<false, false>(kk2, F, &sK, &sK);     // K K^T
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int cj = C0 + 16 * jj;
      const float bj = sb[cj + r];  // masked values formed first, then picked
      floatx4 db;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = R0 + 4 * gg + i, j = cj + r;
        const float bmi = sb[m];
        if constexpr (GATED) {
          const int tm = m / g.nh, tj = j / g.nh;
          const float e0 = sEg[tm * LD + tj], e1 = sEg[tj * LD + tm];
          const float elo = j < m ? e0 : 0.f, ehi = m < j ? e1 : 0.f;
          const float lo = dt2[jj][i] * bj * elo, hi = dtt2[jj][i] * bmi * ehi;
          d2[jj][i] = j < m ? lo : hi;  // locals: a select
          db[i] = dt2[jj][i] * kk2[jj][i] * elo;
          f2[jj][i] = db[i] * bj;
        } else {
          // Nested: the compiler keeps branches here (one LDS read waits in one), which
          // costs less than the 10 spilled registers of the branch-free form.
          const float lo = dt2[jj][i] * bj, hi = dtt2[jj][i] * bmi;
          const float dd = dt2[jj][i] * kk2[jj][i];
          d2[jj][i] = j < m ? lo : (m < j ? hi : 0.f);
          db[i] = j < m ? dd : 0.f;
        }
      }
      colsum16(db, sdb[4 + F.rb], cj + r);
    }
  }
  zero2(dq);
  zero2(dk);
  rmm<true>(dq, F, yf, sHc);              // dy Hc^T
  bmm<true, true, true>(dk, F, sG, sHc);  // -G Hc^T
  if constexpr (GATED) {
    // f terms: ptok_t sum_d Q[t][d] (dy Hc^T)[t][d] and p_m sum_d K[m][d] (-G Hc^T)[m][d],
    // then the row scalings diag(ptok) and diag(p) of those two products.
    float fq[4], fpv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = R0 + 4 * gg + i;
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int d = C0 + 16 * jj + r;
        a = fmaf(bget(sQt, d, row), dq[jj][i], a);
        b = fmaf(bget(sK, row, d), dk[jj][i], b);
      }
      fq[i] = mg_group_sum<16>(a);  // over the 16 lanes r of this row group
      fpv[i] = mg_group_sum<16>(b);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        dq[jj][i] *= spt[row];
        dk[jj][i] *= sp[row];
      }
    }
    if (r == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = R0 + 4 * gg + i;
        sfp[F.ch * DN + row] = spt[row] * fq[i];
        sfp[(2 + F.ch) * DN + row] = sp[row] * fpv[i];
      }
    }
  }
  if constexpr (!GATED) __syncthreads();  // G and Hc are free
  acc_put(sR[RDS], ds2[0], R0, C0);  // dS as (t; m)
  acc_put(sR[RDS], ds2[1], R0, C0 + 16);
  acc_put_t(sR[RDST], ds2[0], R0, C0);  // dS^T as (m; t)
  acc_put_t(sR[RDST], ds2[1], R0, C0 + 16);
  __syncthreads();
  FTile tn;  // dHn again (an L2 hit), fetched while the dS products run
  tn.load(dHn + mat, g.dk, g.dv);
  bmm<true, false>(dq, F, sR[RDS], &sKt);  // + dS K
  bmm<true, false>(dk, F, sR[RDST], &sQt);  // + dS^T Q
  store_block_bf16(dQ + trow0 * g.dk, g.dk, dq, R0, C0, ch.Ct, g.dk);
  if constexpr (!GATED) __syncthreads();  // dS and dS^T are free
  acc_put_t(sR[RD2], d2[0], R0, C0);  // D2 (symmetric)
  acc_put_t(sR[RD2], d2[1], R0, C0 + 16);
  tn.put_split(sR[RDHN]);  // dHn as (d; j)
  __syncthreads();
  {
    floatx4 bu2[2];
    zero2(bu2);
    bmm<true, false>(dk, F, sR[RD2], &sKt);  // + D2 K
    bmm<true, true>(bu2, F, sU, sR[RDHN]);   // U dHn^T
    float rowp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = R0 + 4 * gg + i;
      const float sc = GATED ? sab[m] : sb[m];
      dk[0][i] += sc * bu2[0][i];
      dk[1][i] += sc * bu2[1][i];
      rowp[i] = mg_group_sum<16>(bget(sK, m, C0 + r) * bu2[0][i] +
                                 bget(sK, m, C0 + 16 + r) * bu2[1][i]);
    }
    store_block_bf16(dK + row0 * g.dk, g.dk, dk, R0, C0, ch.M, g.dk);
    if (r == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sdb[8 + F.ch][R0 + 4 * gg + i] = rowp[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < ch.M) {
    const int m = threadIdx.x;
    float acc = sdb[8][m] + sdb[9][m];
    if constexpr (GATED) acc *= sa[m];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc += sdb[q][m];
    stf(dbeta, row0 + m, acc);
  }
  if constexpr (GATED) {
    // Token-level F[t][t'] (t' < t) and f[t] (in sdec's l slot).  With one micro-step
    // per token the micro-rows are the tokens: F is the wave's f1 + f2 plus the carry
    // term on row Ct - 1.  With nh > 1 the (t, m) and (m, j) span gradients go to two
    // tables and are summed over the micro-rows of each token pair:
    //   F[t][t'] = sum_j f1[t][t' nh + j] + sum_{a,b} f2[t nh + a][t' nh + b]
    //              (+ sum_j a beta rowsum terms of t' nh + j on row Ct - 1),
    // and the p terms of f over the micro-rows of each token.
    float pcs = 0.f;
#pragma unroll
    for (int q = 0; q < WB; ++q) pcs += sred[q];
    float* sF;
    if (g.nh == 1) {
      sF = reinterpret_cast<float*>(&sR[1]);  // 64 x 64, stride DN
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = R0 + 4 * gg + i, tp = C0 + 16 * jj + r;
          sF[t * DN + tp] = (tp < t && t < ch.Ct) ? f1[jj][i] + f2[jj][i] : 0.f;
        }
      __syncthreads();
      if (threadIdx.x < DN) {
        const int t = threadIdx.x;
        if (t < ch.Ct - 1)
          sF[(ch.Ct - 1) * DN + t] += sab[t] * (sdb[8][t] + sdb[9][t]);
        float f = 0.f;
        if (t < ch.Ct) {
          f = sfp[t] + sfp[DN + t] + sfp[2 * DN + t] + sfp[3 * DN + t];
          if (t == ch.Ct - 1) f = fmaf(expf(sLc[t]), pcs, f);
        }
        sl[t] = f;
      }
    } else {
      const int nh = g.nh;
      float* sA = reinterpret_cast<float*>(&sR[1]);  // f1 at (t; m)
      float* sB = reinterpret_cast<float*>(&sR[2]);  // f2 at (m; j)
      sF = reinterpret_cast<float*>(&sR[0]);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = R0 + 4 * gg + i, col = C0 + 16 * jj + r;
          sA[row * DN + col] = f1[jj][i];
          sB[row * DN + col] = f2[jj][i];
        }
      __syncthreads();
      for (int e = threadIdx.x; e < DN * DN; e += NTB) {
        const int t = e >> 6, tp = e & 63;
        float v = 0.f;
        if (t < ch.Ct && tp < t) {
          for (int j = 0; j < nh; ++j) v += sA[t * DN + tp * nh + j];
          for (int a = 0; a < nh; ++a)
            for (int b = 0; b < nh; ++b) v += sB[(t * nh + a) * DN + tp * nh + b];
          if (t == ch.Ct - 1)
            for (int j = 0; j < nh; ++j) {
              const int m = tp * nh + j;
              v = fmaf(sab[m], sdb[8][m] + sdb[9][m], v);
            }
        }
        sF[e] = v;
      }
      if (threadIdx.x < DN) {
        const int t = threadIdx.x;
        float f = 0.f;
        if (t < ch.Ct) {
          f = sfp[t] + sfp[DN + t];
          for (int a = 0; a < nh; ++a) f += sfp[2 * DN + t * nh + a] + sfp[3 * DN + t * nh + a];
          if (t == ch.Ct - 1) f = fmaf(expf(sLc[t]), pcs, f);
        }
        sl[t] = f;
      }
    }
    __syncthreads();
    // dl_s = sum_{t >= s} (f[t] + sum_{t' < s} F[t][t']): wave-level prefix scans of
    // the rows of F, per-wave column partials summed in a fixed order.
    {
      constexpr int ROWS = DN / WB;
      const int w = wave_id();
      float acc = 0.f;
      for (int rr = 0; rr < ROWS; ++rr) {
        const int t = ROWS * w + rr;
        const float ex = mg_wave_prev(mg_wave_prefix_sum(sF[t * DN + lane]));
        if (t >= lane && t < ch.Ct) acc += sl[t] + ex;
      }
      sdl[w * DN + lane] = acc;
    }
    __syncthreads();
    if (threadIdx.x < ch.Ct) {
      const int s = threadIdx.x;
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < WB; ++q) acc += sdl[q * DN + s];
      dlg[trow0 + s] = acc;
    }
  }
}

// ---------------------------------------------------------------------------
// serial chains: one workgroup of 4 waves per (head, 16-column d_v slice)
// ---------------------------------------------------------------------------
// Wave w keeps the state rows 16 w .. 16 w + 15 of the slice in an MFMA
// accumulator.  The chunk maps (A, Qe split; B, Pu fp32) are loaded straight
// into registers two chunks ahead; the state's transpose H^T passes through
// LDS (double-buffered, one barrier per chunk).

// LDS fragment offsets of rows 0..15 (lane row r, chunk 4 s + g).
struct RowFrag {
  unsigned o[2];
  __device__ __forceinline__ void init() {
    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int s = 0; s < 2; ++s) o[s] = FragOff::at(0, (unsigned)((4 * s + g) ^ (r & 7) ^ (r >> 3)), r);
  }
};

__device__ __forceinline__ bf16x8 as_bf(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// acc += A B^T, A split in registers ([s] fragments), B a split 16-row BMat pair.
__device__ __forceinline__ floatx4 amm(floatx4 acc, const uint4 (&ah)[2], const uint4 (&al)[2],
                                       const BMat* B, const RowFrag& rf) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bf16x8 bh = frag_at(B[0], rf.o[s]), bl = frag_at(B[1], rf.o[s]);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah[s]), bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah[s]), bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(al[s]), bh, acc, 0, 0, 0);
  }
  return acc;
}

// Two independent products against the same B (the chain's state update and
// readout): each B fragment is read once and the two MFMA chains interleave.
__device__ __forceinline__ void amm2(floatx4& acc0, const uint4 (&ah0)[2], const uint4 (&al0)[2],
                                     floatx4& acc1, const uint4 (&ah1)[2], const uint4 (&al1)[2],
                                     const BMat* B, const RowFrag& rf) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bf16x8 bh = frag_at(B[0], rf.o[s]), bl = frag_at(B[1], rf.o[s]);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah0[s]), bh, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah1[s]), bh, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah0[s]), bl, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah1[s]), bl, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(al0[s]), bh, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(al1[s]), bh, acc1, 0, 0, 0);
  }
}

// A fragments of a fragment-ordered split workspace matrix: rows 16 rb..16 rb + 15,
// k halves s = 0, 1.
__device__ __forceinline__ void load_split_frag(uint4 (&hi)[2], uint4 (&lo)[2], const u16* m,
                                                int rb) {
  const unsigned lane = lane_id();
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const unsigned off = ((unsigned)(rb * 2 + s) * 64u + lane) * 8u;
    hi[s] = *reinterpret_cast<const uint4*>(m + off);
    lo[s] = *reinterpret_cast<const uint4*>(m + SPLIT_LO + off);
  }
}

struct FwdOps {
  uint4 ah[2], al[2], qh[2], ql[2];
  floatx4 b, pu;
  float pc;  // gated: the chunk's total decay PC
};

//   H_c saved, y = Qe H_c + Pu, H_{c+1} = H_c + A H_c + B (gated: PC H_c + A H_c + B).
template <bool GATED>
__global__ __launch_bounds__(NT) void dwb_fwd_chain(const float* __restrict__ H0,
                                                    const float* __restrict__ Am,
                                                    const float* __restrict__ Bm,
                                                    const float* __restrict__ Qem,
                                                    const float* __restrict__ Pum,
                                                    const float* __restrict__ vm,
                                                    u16* __restrict__ y, float* __restrict__ HT,
                                                    float* __restrict__ Hb, DwGeom g, int64_t BH) {
  __shared__ BPair sHt[2];
  int64_t bh;
  int col0;
  if (!chain_slot(g, BH, bh, col0)) return;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int col = col0 + r;
  RowFrag rf;
  rf.init();
  floatx4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    h[i] = (d < g.dk && col < g.dv) ? H0[(bh * g.dk + d) * g.dv + col] : 0.f;
  }
  auto fetch = [&](FwdOps& o, int c) {
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    load_split_frag(o.ah, o.al, reinterpret_cast<const u16*>(Am + mat), w);
    load_split_frag(o.qh, o.ql, reinterpret_cast<const u16*>(Qem + mat), w);
    o.b = load_tile_frag(Bm + mat, w, col0 >> 4);
    o.pu = load_tile_frag(Pum + mat, w, col0 >> 4);
    if constexpr (GATED) o.pc = ld_uniform_v(vm + ((size_t)bh * g.nc + c) * VECN + V_PC);
  };
  // Chunk c + 2 is fetched while chunk c computes: three operand buffers in a
  // ring, the loop unrolled by three so the buffers never move.  The fetch is
  // unconditional (the index clamped to the last chunk): a conditional one leaves
  // the compiler a merge of old and new buffer contents, resolved by register
  // copies that wait for the loads at once.
  auto step = [&](const FwdOps& cur, FwdOps& fill, int c) {
    fetch(fill, min(c + 2, g.nc - 1));
    const Chunk ch = chunk_of(g, c);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    BPair& ht = sHt[c & 1];
    acc_put_t(ht, h, 16 * w, 0);
    store_tile_frag(Hb + mat, w, col0 >> 4, h);
    __syncthreads();
    floatx4 yy = {0.f, 0.f, 0.f, 0.f};  // Pu is added after the products
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = GATED ? fmaf(cur.pc, h[i], cur.b[i]) : h[i] + cur.b[i];
    amm2(h, cur.ah, cur.al, yy, cur.qh, cur.ql, ht, rf);  // H + A H + B, y = Qe H + Pu
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * gg + i;
      if (t < ch.Ct && col < g.dv)
        y[(bh * g.T + ch.t0 + t) * g.dv + col] = bf_bits(yy[i] + cur.pu[i]);
    }
  };
  FwdOps b0, b1, b2;
  fetch(b0, 0);
  fetch(b1, min(1, g.nc - 1));
  int c = 0;
  for (; c + 3 <= g.nc; c += 3) {
    step(b0, b2, c);
    step(b1, b0, c + 1);
    step(b2, b1, c + 2);
  }
  if (c < g.nc) step(b0, b2, c);
  if (c + 1 < g.nc) step(b1, b0, c + 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    if (d < g.dk && col < g.dv) HT[(bh * g.dk + d) * g.dv + col] = h[i];
  }
}

struct BwdOps {
  uint4 ah[2], al[2];
  floatx4 b;
  float pc;  // gated: the chunk's total decay PC
};

//   dH (chunk exit) saved, dH <- dH + A' dH + b' (gated: PC dH + A' dH + b').
template <bool GATED>
__global__ __launch_bounds__(NT) void dwb_bwd_chain(const float* __restrict__ dHT,
                                                    const float* __restrict__ Apm,
                                                    const float* __restrict__ bpm,
                                                    const float* __restrict__ vm,
                                                    float* __restrict__ dHn,
                                                    float* __restrict__ dH0, DwGeom g,
                                                    int64_t BH) {
  __shared__ BPair sHt[2];
  int64_t bh;
  int col0;
  if (!chain_slot(g, BH, bh, col0)) return;
  const int w = wave_id(), lane = lane_id(), r = lane & 15, gg = lane >> 4;
  const int col = col0 + r;
  RowFrag rf;
  rf.init();
  floatx4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    h[i] = (d < g.dk && col < g.dv) ? dHT[(bh * g.dk + d) * g.dv + col] : 0.f;
  }
  auto fetch = [&](BwdOps& o, int c) {
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    load_split_frag(o.ah, o.al, reinterpret_cast<const u16*>(Apm + mat), w);
    o.b = load_tile_frag(bpm + mat, w, col0 >> 4);
    if constexpr (GATED) o.pc = ld_uniform_v(vm + ((size_t)bh * g.nc + c) * VECN + V_PC);
  };
  // Chunk c - 2 is fetched while chunk c computes (ring of three buffers).
  auto step = [&](const BwdOps& cur, BwdOps& fill, int c) {
    if (c >= 2) fetch(fill, c - 2);
    const size_t mat = ((size_t)bh * g.nc + c) * MAT;
    BPair& ht = sHt[c & 1];
    acc_put_t(ht, h, 16 * w, 0);
    acc_store_ws(h, dHn + mat + 16 * w * DN + col0);
    __syncthreads();
    floatx4 hn;
#pragma unroll
    for (int i = 0; i < 4; ++i) hn[i] = GATED ? fmaf(cur.pc, h[i], cur.b[i]) : h[i] + cur.b[i];
    h = amm(hn, cur.ah, cur.al, ht, rf);
  };
  BwdOps b0, b1, b2;
  fetch(b0, g.nc - 1);
  if (g.nc > 1) fetch(b1, g.nc - 2);
  int c = g.nc - 1;
  for (; c - 2 >= 0; c -= 3) {
    step(b0, b2, c);
    step(b1, b0, c - 1);
    step(b2, b1, c - 2);
  }
  if (c >= 0) step(b0, b2, c);
  if (c - 1 >= 0) step(b1, b0, c - 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 16 * w + 4 * gg + i;
    if (d < g.dk && col < g.dv) dH0[(bh * g.dk + d) * g.dv + col] = h[i];
  }
}

}  // namespace

// Elementwise (diagonal) scans: linear_scan and parallel_scan_log, fwd + bwd.
//
// Recurrence per column: h_t = a_t h_{t-1} + b_t.
//   linear_scan       (reference src/mingru/min_gru.py:1454-1510): outputs the
//                     running product A_t and the zero-start solution Bc_t.
//   parallel_scan_log (reference src/mingru/min_gru.py:755-807): a = exp(lc),
//                     b = exp(lv[t+1]), h_{-1} = exp(lv[0]); all terms positive,
//                     so the linear-space fp32 recurrence has no cancellation.
//
// Work decomposition (one pass over HBM, decoupled look-back):
//   * a lane group is (batch row, tile of 64*VEC consecutive columns); each
//     thread owns VEC consecutive columns, so a wave's loads/stores along D
//     are contiguous (1 KiB per row for VEC=4); VEC is chosen per launch (4, or
//     2 or 1 for rows narrower than 256 columns and for problems too small to
//     give every CU a workgroup);
//   * a workgroup of WAVES waves owns a chunk of WAVES*TSUB time steps; wave w
//     owns TSUB consecutive steps and keeps all its inputs in registers;
//   * per thread: local affine aggregate -> LDS combine across waves ->
//     look-back over earlier chunks (wave 0) -> final recompute from the carry
//     and streaming stores;
//   * small problems (few chunks per sequence, inputs that stay cached) run as
//     two launches over the same grid instead: chunk
//     aggregates, then every chunk folds its predecessors' aggregates itself
//     (EW_REDUCE / EW_FINAL), so no workgroup waits on another.
// The backward is the same machinery run in reverse time order over the
// adjoint recurrence y_t = a_t (g_t + y_{t+1}); forward values needed for the
// gradient (A_{t-1}, Bc_{t-1} or h_{t-1}) are recomputed from one saved
// forward output per thread sub-chunk boundary.
#include "mg_common.h"
#include "mg_gates.h"

#include <initializer_list>
#include <atomic>
#include <mutex>
#include <type_traits>

#include <algorithm>
#include <cstdlib>

namespace {

// Chunk = WAVES * TSUB time steps per workgroup.
constexpr int EW_WAVES_FWD = 8;
constexpr int EW_TSUB_FWD = 8;
constexpr int EW_WAVES_BWD = 8;
constexpr int EW_TSUB_BWD = 8;
// Fused gate backward: four arrays per step stay live (sigmoid, tanh, hpre,
// adjoint), so each wave holds 4 steps (32-step chunks) to stay clear of spills.
constexpr int GATE_WAVES_BWD = 8;
constexpr int GATE_TSUB_BWD = 4;
// Fused gate forward with 1 or 2 columns per lane (small problems): 8 steps per
// wave (13.4 against 15.6 us at B=4, T=1024, D=256).
constexpr int GATE_TSUB_FWD_NARROW = 8;
// Workgroups a launch needs before it runs 4 columns per lane: one per CU.
constexpr int64_t EW_FILL_WGS = 256;

// Launch forms of the chunked scans.  EW_LOOKBACK is one launch whose
// workgroups combine chunk carries by decoupled look-back.  A small problem
// instead runs two launches over the same grid: EW_REDUCE stores every chunk's
// aggregate map (the first chunk's with the sequence seed folded in, in the
// look-back slots with a tag no launch uses), and
// EW_FINAL folds the stored aggregates of all a chunk's predecessors -- at most
// EW_FINAL_MAX_CHUNKS - 1, loaded a few per wave at once, so nothing waits on
// another workgroup -- then recomputes the chunk from its carry.  The second
// launch re-reads the inputs; the same grid puts each chunk on the XCD whose L2
// the first launch filled with them, and EW_TWO_LAUNCH_BYTES keeps them there.
// At B=4, T=1024, D=256 a sequence is 16 chunks, and the look-back walks them
// one round trip after another.
// EW_AGG does both in one launch when the whole grid fits on the chip at once:
// every workgroup publishes its chunk aggregate (tagged with the launch's epoch,
// before it waits on anything), then folds its predecessors' published
// aggregates -- all loaded at once, never an inclusive prefix, so there is no
// chain of workgroups waiting one after another -- and recomputes its chunk.
enum : int { EW_LOOKBACK = 0, EW_REDUCE = 1, EW_FINAL = 2, EW_AGG = 3 };
constexpr int EW_FINAL_MAX_CHUNKS = 32;
constexpr int64_t EW_TWO_LAUNCH_BYTES = (int64_t)32 << 20;  // input bytes of both launches

// Affine map y -> p*y + l (NL independent offsets sharing one slope).  The
// look-back machinery below moves any map type that names its NF fp32 fields
// (get / set), an identity and compose(inner, outer).
template <int NL>
struct Aff {
  static constexpr int NF = NL + 1;
  float p;
  float l[NL];
  __device__ __forceinline__ float get(int f) const { return f == 0 ? p : l[f > 0 ? f - 1 : 0]; }
  __device__ __forceinline__ void set(int f, float v) {
    if (f == 0)
      p = v;
    else
      l[f > 0 ? f - 1 : 0] = v;
  }
  __device__ __forceinline__ static Aff identity() {
    Aff r;
    r.p = 1.f;
#pragma unroll
    for (int i = 0; i < NL; ++i) r.l[i] = 0.f;
    return r;
  }
};

template <int NL>
__device__ __forceinline__ Aff<NL> aff_identity() {
  return Aff<NL>::identity();
}

// outer o inner: apply `inner` first, then `outer`.
template <int NL>
__device__ __forceinline__ Aff<NL> compose(const Aff<NL>& inner, const Aff<NL>& outer) {
  Aff<NL> r;
  r.p = outer.p * inner.p;
#pragma unroll
  for (int i = 0; i < NL; ++i) r.l[i] = fmaf(outer.p, inner.l[i], outer.l[i]);
  return r;
}

// ---------------------------------------------------------------------------
// Extended-range values for parallel_scan_log
// ---------------------------------------------------------------------------
// The log scan's inputs are logs: a term exp(lv) or a product of exp(lc) can
// leave fp32's range (e^-87 .. e^88) while the output h stays inside it (an
// initial state e^-150 grown by e^+1 per step), and the backward's adjoint can
// overflow while the gradients it forms stay finite.  Such values are held as
// Xf {s, e} = s * 2^e: an fp32 significand s and an integer-valued fp32
// exponent e, with zero as {0, -inf}.  Products multiply significands and add
// exponents, sums align on the larger exponent, so no intermediate overflows or
// underflows and each operation keeps fp32's relative rounding.  The reference
// reaches the same range by evaluating in log space
// (src/mingru/min_gru.py:804-807; its kernel's online max-shift,
// src/mingru/triton_scans.py:797-821).
struct Xf {
  float s, e;
};

__device__ __forceinline__ Xf xf_zero() { return Xf{0.f, -INFINITY}; }

// s * 2^d for an alignment or output shift d; |d| beyond 512 is as good as
// infinite for an fp32 significand (and a NaN shift only pairs with s = 0).
__device__ __forceinline__ float xf_ldexp(float s, float d) {
  return __builtin_amdgcn_ldexpf(s, (int)fminf(fmaxf(d, -512.f), 512.f));
}

// e^x split as s * 2^k with |log s| <= ln2 / 2: k = rint(x log2 e) and the
// remainder x - k ln2 taken with ln2 in two parts (Cody & Waite), so the
// remainder is exact to fp32 rounding for any |x| below 1e6.  Inputs are clamped
// to +-1e6 (e^-1e6 is zero and e^1e6 infinite for every fp32 combination);
// NaN passes through.
__device__ __forceinline__ Xf xf_exp(float x) {
  constexpr float LOG2E = 1.44269504088896341f;
  constexpr float LN2_HI = 0.693145751953125f;
  constexpr float LN2_LO = 1.42860682030941723e-6f;
  x = x < -1.0e6f ? -1.0e6f : x;
  x = x > 1.0e6f ? 1.0e6f : x;
  const float k = rintf(x * LOG2E);
  float r = fmaf(-k, LN2_HI, x);
  r = fmaf(-k, LN2_LO, r);
  return Xf{__builtin_amdgcn_exp2f(r * LOG2E), k};
}

// Significand into [0.5, 1); an exact zero gets exponent -inf.
__device__ __forceinline__ Xf xf_norm(Xf v) {
  const float m = __builtin_amdgcn_frexp_mantf(v.s);
  const int ex = __builtin_amdgcn_frexp_expf(v.s);
  return Xf{m, m == 0.f ? -INFINITY : v.e + (float)ex};
}

__device__ __forceinline__ Xf xf_from(float x) { return xf_norm(Xf{x, 0.f}); }

__device__ __forceinline__ float xf_to_float(Xf v) { return xf_ldexp(v.s, v.e); }

__device__ __forceinline__ Xf xf_mul(Xf a, Xf b) { return Xf{a.s * b.s, a.e + b.e}; }

__device__ __forceinline__ Xf xf_add(Xf a, Xf b) {
  const float em = fmaxf(a.e, b.e);
  return Xf{xf_ldexp(a.s, a.e - em) + xf_ldexp(b.s, b.e - em), em};
}

// a * y + b
__device__ __forceinline__ Xf xf_fma(Xf a, Xf y, Xf b) { return xf_add(xf_mul(a, y), b); }

// Affine map y -> p*y + l over Xf values (one offset); four look-back fields.
struct XAff {
  static constexpr int NF = 4;
  Xf p, l;
  __device__ __forceinline__ float get(int f) const {
    return f == 0 ? p.s : f == 1 ? p.e : f == 2 ? l.s : l.e;
  }
  __device__ __forceinline__ void set(int f, float v) {
    if (f == 0)
      p.s = v;
    else if (f == 1)
      p.e = v;
    else if (f == 2)
      l.s = v;
    else
      l.e = v;
  }
  __device__ __forceinline__ static XAff identity() { return XAff{Xf{1.f, 0.f}, xf_zero()}; }
};

__device__ __forceinline__ XAff compose(const XAff& inner, const XAff& outer) {
  return XAff{xf_norm(xf_mul(outer.p, inner.p)), xf_norm(xf_fma(outer.p, inner.l, outer.l))};
}

// Data streams are read and written once: non-temporal accesses.  NT = false
// for a read that a later launch repeats (EW_REDUCE), so the lines stay cached.
template <int VEC, bool NT = true>
__device__ __forceinline__ void load_vec(float (&dst)[VEC], const float* __restrict__ src) {
  if constexpr (VEC == 4) {
    const float4 v = NT ? mg_ld_stream4(src) : *reinterpret_cast<const float4*>(src);
    dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
  } else if constexpr (VEC == 2) {
    const float2 v = NT ? mg_ld_stream2(src) : *reinterpret_cast<const float2*>(src);
    dst[0] = v.x; dst[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) dst[i] = NT ? mg_ld_stream(src + i) : src[i];
  }
}

template <int VEC>
__device__ __forceinline__ void store_vec(float* __restrict__ dst, const float (&src)[VEC]) {
  if constexpr (VEC == 4) {
    mg_st_stream4(dst, make_float4(src[0], src[1], src[2], src[3]));
  } else if constexpr (VEC == 2) {
    mg_st_stream2(dst, make_float2(src[0], src[1]));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) mg_st_stream(dst + i, src[i]);
  }
}

struct EwGeom {
  int64_t T, D;
  int n_tiles, n_lg, n_chunks;
};

// Look-back slots: [lg][chunk][field][VEC][64 lanes] tagged words, so each wave
// store of one (field, vector element) covers 512 contiguous bytes (whole lines).
template <typename Map, int VEC>
__device__ __forceinline__ void lb_put(mg_slot_t* base, const EwGeom& g, int lg, int c, int lane,
                                       const Map (&x)[VEC], unsigned epoch) {
  constexpr int TILE = MG_WAVE * VEC;
  mg_slot_t* p = base + ((int64_t)(lg * g.n_chunks + c) * Map::NF) * TILE + lane;
#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int f = 0; f < Map::NF; ++f) mg_slot_put(p + f * TILE + v * MG_WAVE, x[v].get(f), epoch);
}

template <typename Map, int VEC>
__device__ __forceinline__ bool lb_try(const mg_slot_t* base, const EwGeom& g, int lg, int c,
                                       int lane, Map (&x)[VEC], unsigned epoch) {
  constexpr int TILE = MG_WAVE * VEC;
  const mg_slot_t* p = base + ((int64_t)(lg * g.n_chunks + c) * Map::NF) * TILE + lane;
  bool ok = true;
#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int f = 0; f < Map::NF; ++f) {
      float val;
      ok &= mg_slot_get(p + f * TILE + v * MG_WAVE, val, epoch);
      x[v].set(f, val);
    }
  return ok;
}

// Stored chunk aggregates of the two-launch form, in the look-back slot layout
// [lg][chunk][field][VEC][64 lanes] and format, with tag 0: the slot regions are
// shared with look-back launches on the same workspace, whose epochs are never
// 0, so these words can never pass for a later launch's published values (a raw
// float there could: a denormal's bit pattern is a small integer, like an epoch).
template <typename Map, int VEC>
__device__ __forceinline__ void agg_store(mg_slot_t* base, const EwGeom& g, int lg, int c,
                                          int lane, const Map (&x)[VEC]) {
  constexpr int TILE = MG_WAVE * VEC;
  mg_slot_t* p = base + ((int64_t)(lg * g.n_chunks + c) * Map::NF) * TILE + lane;
#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int f = 0; f < Map::NF; ++f)
      p[f * TILE + v * MG_WAVE] = (mg_slot_t)__float_as_uint(x[v].get(f));
}

template <typename Map, int VEC>
__device__ __forceinline__ void agg_load(const mg_slot_t* base, const EwGeom& g, int lg, int c,
                                         int lane, Map (&x)[VEC]) {
  constexpr int TILE = MG_WAVE * VEC;
  const mg_slot_t* p = base + ((int64_t)(lg * g.n_chunks + c) * Map::NF) * TILE + lane;
#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int f = 0; f < Map::NF; ++f)
      x[v].set(f, __uint_as_float((unsigned)p[f * TILE + v * MG_WAVE]));
}

// The launch tag of an EW_AGG workgroup, in LDS: thread 0 takes it (ew_agg_begin)
// at the start of the kernel and writes it here just before the first barrier of
// ew_carry, so its round trip overlaps the chunk's input loads.
__device__ __forceinline__ unsigned& ew_agg_epoch() {
  __shared__ unsigned s_epoch;
  return s_epoch;
}

// Workspace protocol of an EW_AGG launch: one 64-bit header word {low: count,
// high: epoch}.  Every workgroup adds 1 (one atomic round trip, with no other
// access waiting on it); the old value's epoch e is the launch's, and the
// workgroup that finds count == grid - 1 -- every other workgroup of the launch
// has added by then -- stores {0, e + 1} for the next launch.  Tags are
// (e + 1) | 2^31: never 0 (the two-launch form's stored aggregates) and apart from
// the look-back launches' epochs (MG_H_EPOCH, far below 2^31), whose slots share
// the region.  A workgroup's chunk is its workgroup index, since every workgroup
// of the grid is resident.  Returns the tag in thread 0 (0 elsewhere).
constexpr int EW_H_AGG = 4;  // header words 4, 5 (8-byte aligned)
__device__ __forceinline__ unsigned long long ew_agg_begin(unsigned* header) {
  if (threadIdx.x != 0) return 0ull;
  return __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(header + EW_H_AGG), 1ull,
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0, at the first barrier: the launch tag from ew_agg_begin's word, and the
// hand-over to the next launch by the workgroup that added last.
__device__ __forceinline__ unsigned ew_agg_tag(unsigned* header, unsigned long long old) {
  const unsigned count = (unsigned)old, e = (unsigned)(old >> 32);
  if (count == gridDim.x - 1u)
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(header + EW_H_AGG),
                       (unsigned long long)(e + 1u) << 32, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  else if (count >= gridDim.x)
    mg_count_error(header);
  return (e + 1u) | 0x80000000u;
}

// Intra-workgroup combine + the carry from earlier chunks: decoupled look-back
// (PH = EW_LOOKBACK) or the stored aggregates of the two-launch form (PH =
// EW_FINAL; PH = EW_REDUCE only stores this chunk's aggregate and leaves
// `carry` unset).  On return `carry` holds, for this thread's columns, the
// composition of everything before (forward) or after (REVERSE) this thread's
// sub-chunk.  `seed` is the map applied at the sequence start (forward) or end
// (reverse).
template <typename Map, int VEC, int WAVES, bool REVERSE, int PH = EW_LOOKBACK>
__device__ __forceinline__ void ew_carry(const Map (&loc)[VEC], const Map (&seed)[VEC],
                                         const EwGeom& g, int lg, int c, unsigned* header,
                                         unsigned long long epoch, mg_slot_t* agg_data,
                                         mg_slot_t* incl_data, Map (&carry)[VEC]) {
  constexpr int TILE = MG_WAVE * VEC;
  constexpr int NF = Map::NF;
  constexpr int PER = EW_FINAL_MAX_CHUNKS / WAVES;  // predecessors per wave (EW_FINAL)
  static_assert(EW_FINAL_MAX_CHUNKS % WAVES == 0, "predecessors split evenly over the waves");
  __shared__ float s_agg[WAVES][NF][TILE];
  __shared__ float s_carry[PH == EW_FINAL || PH == EW_AGG ? WAVES : 1][NF][TILE];
  const int lane = threadIdx.x & (MG_WAVE - 1);
  const int w = threadIdx.x / MG_WAVE;
  const int first = REVERSE ? g.n_chunks - 1 : 0;

#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int f = 0; f < NF; ++f) s_agg[w][f][v * MG_WAVE + lane] = loc[v].get(f);
  if constexpr (PH == EW_AGG) {
    if (threadIdx.x == 0) ew_agg_epoch() = ew_agg_tag(header, epoch);  // thread 0's word
    __syncthreads();  // every wave's aggregate, and the tag, are in LDS
    const unsigned ep = ew_agg_epoch();
    if (w == 0) {  // publish this chunk's aggregate (the first chunk's with the seed)
      Map G[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        G[v] = c == first ? seed[v] : Map::identity();
        for (int j = 0; j < WAVES; ++j) {
          const int jj = REVERSE ? WAVES - 1 - j : j;
          Map a;
#pragma unroll
          for (int f = 0; f < NF; ++f) a.set(f, s_agg[jj][f][v * MG_WAVE + lane]);
          G[v] = compose(G[v], a);
        }
      }
      lb_put<Map, VEC>(agg_data, g, lg, c, lane, G, ep);
    }
    // Wave w folds predecessors w*PER .. w*PER+PER-1 in application order, every
    // slot polled at once and the missing ones again until all have arrived.
    const int npred = REVERSE ? g.n_chunks - 1 - c : c;
    Map X[PER][VEC];
    bool ok[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int k = w * PER + i;
      ok[i] = k >= npred ||
              lb_try<Map, VEC>(agg_data, g, lg, REVERSE ? g.n_chunks - 1 - k : k, lane, X[i], ep);
    }
    for (unsigned spins = 0;;) {
      bool all = true;
#pragma unroll
      for (int i = 0; i < PER; ++i) all &= ok[i];
      if (all) break;
      if (++spins >= MG_SPIN_LIMIT) {
        mg_count_error(header);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int k = w * PER + i;
        if (!ok[i])
          ok[i] = lb_try<Map, VEC>(agg_data, g, lg, REVERSE ? g.n_chunks - 1 - k : k, lane, X[i],
                                   ep);
      }
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      Map part = (w == 0 && c == first) ? seed[v] : Map::identity();
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (w * PER + i < npred) part = compose(part, X[i][v]);
#pragma unroll
      for (int f = 0; f < NF; ++f) s_carry[w][f][v * MG_WAVE + lane] = part.get(f);
    }
  }
  if constexpr (PH == EW_FINAL) {
    // Wave w folds predecessors w*PER .. w*PER+PER-1 in application order
    // (forward: chunks 0, 1, ...; reverse: chunks n-1, n-2, ...), all its loads
    // issued before the first compose.
    const int npred = REVERSE ? g.n_chunks - 1 - c : c;
    Map X[PER][VEC];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int k = w * PER + i;
      if (k < npred) agg_load<Map, VEC>(agg_data, g, lg, REVERSE ? g.n_chunks - 1 - k : k, lane, X[i]);
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      // Only wave 0 holds the seed; it matters only to the first chunk, which has
      // no predecessors.
      Map part = (w == 0 && c == first) ? seed[v] : Map::identity();
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (w * PER + i < npred) part = compose(part, X[i][v]);
#pragma unroll
      for (int f = 0; f < NF; ++f) s_carry[w][f][v * MG_WAVE + lane] = part.get(f);
    }
  }
  __syncthreads();

  auto wave_agg = [&](int j, int v) {
    Map r;
#pragma unroll
    for (int f = 0; f < NF; ++f) r.set(f, s_agg[j][f][v * MG_WAVE + lane]);
    return r;
  };

  if constexpr (PH == EW_REDUCE) {
    if (w == 0) {
      Map G[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        G[v] = c == first ? seed[v] : Map::identity();
        if (!REVERSE) {
          for (int j = 0; j < WAVES; ++j) G[v] = compose(G[v], wave_agg(j, v));
        } else {
          for (int j = WAVES - 1; j >= 0; --j) G[v] = compose(G[v], wave_agg(j, v));
        }
      }
      agg_store<Map, VEC>(agg_data, g, lg, c, lane, G);
    }
    return;
  }

  // Exclusive prefix of this wave inside the workgroup.
  Map ew[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    ew[v] = Map::identity();
    if (!REVERSE) {
      for (int j = 0; j < w; ++j) ew[v] = compose(ew[v], wave_agg(j, v));
    } else {
      for (int j = WAVES - 1; j > w; --j) ew[v] = compose(ew[v], wave_agg(j, v));
    }
  }

  if constexpr (PH == EW_FINAL || PH == EW_AGG) {
    // The partials in order; the first chunk's stored aggregate carries the seed.
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      Map E = Map::identity();
      for (int j = 0; j < WAVES; ++j) {
        Map P;
#pragma unroll
        for (int f = 0; f < NF; ++f) P.set(f, s_carry[j][f][v * MG_WAVE + lane]);
        E = compose(E, P);
      }
      carry[v] = compose(E, ew[v]);
    }
    return;
  }

  if (w == 0) {
    Map G[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      G[v] = Map::identity();
      if (!REVERSE) {
        for (int j = 0; j < WAVES; ++j) G[v] = compose(G[v], wave_agg(j, v));
      } else {
        for (int j = WAVES - 1; j >= 0; --j) G[v] = compose(G[v], wave_agg(j, v));
      }
    }
    const int first = REVERSE ? g.n_chunks - 1 : 0;
    const int dir = REVERSE ? 1 : -1;  // step towards predecessors
    Map E[VEC];
    if (c == first) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) E[v] = seed[v];
    } else {
      lb_put<Map, VEC>(agg_data, g, lg, c, lane, G, epoch);
#pragma unroll
      for (int v = 0; v < VEC; ++v) E[v] = Map::identity();
      // Per-lane walk over predecessors: an inclusive prefix ends the walk, an
      // aggregate is composed in and the walk continues; the first chunk only
      // ever publishes its inclusive prefix.
      int j = c + dir;
      unsigned spins = 0;
      bool done = false;
      while (!done) {
        Map X[VEC];
        if (lb_try<Map, VEC>(incl_data, g, lg, j, lane, X, epoch)) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) E[v] = compose(X[v], E[v]);
          done = true;
        } else if (j != first && lb_try<Map, VEC>(agg_data, g, lg, j, lane, X, epoch)) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) E[v] = compose(X[v], E[v]);
          j += dir;
        } else {
          __builtin_amdgcn_s_sleep(1);
          if (++spins >= MG_SPIN_LIMIT) {
            mg_count_error(header);
            done = true;
          }
        }
      }
    }
    Map I[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) I[v] = compose(E[v], G[v]);
    lb_put<Map, VEC>(incl_data, g, lg, c, lane, I, epoch);
#pragma unroll
    for (int v = 0; v < VEC; ++v)
#pragma unroll
      for (int f = 0; f < NF; ++f) s_carry[0][f][v * MG_WAVE + lane] = E[v].get(f);
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    Map C;
#pragma unroll
    for (int f = 0; f < NF; ++f) C.set(f, s_carry[0][f][v * MG_WAVE + lane]);
    carry[v] = compose(C, ew[v]);
  }
}

struct EwThread {
  int lane, w, c, lg, bb;
  unsigned long long epoch;  // the look-back epoch; EW_AGG: ew_agg_begin's word (thread 0)
  bool valid;  // false only for a ticket beyond the grid (workspace protocol broken)
  int64_t col;
  bool col_ok;
};

// The thread's chunk, lane group and columns for ticket `ticket` of the launch:
// the (lane group, chunk) pair ticket % n_lg, ticket / n_lg (chunks from the end
// for a REVERSE scan).
// UNI: the wave index is marked wave-uniform as well (see mg_persistent's UNIFORM).
template <int VEC, bool REVERSE, bool UNI = false>
__device__ __forceinline__ EwThread ew_thread_at(const EwGeom& g, unsigned ticket,
                                                 unsigned long long epoch) {
  EwThread th;
  th.valid = true;
  th.epoch = epoch;
  th.lane = threadIdx.x & (MG_WAVE - 1);
  th.w = UNI ? (int)mg_uniform(threadIdx.x / MG_WAVE) : (int)(threadIdx.x / MG_WAVE);
  int k = (int)(ticket / (unsigned)g.n_lg);
  th.lg = (int)(ticket - (unsigned)k * (unsigned)g.n_lg);
  th.c = REVERSE ? g.n_chunks - 1 - k : k;
  th.bb = th.lg / g.n_tiles;
  int tile = th.lg - th.bb * g.n_tiles;
  th.col = (int64_t)tile * (MG_WAVE * VEC) + th.lane * VEC;
  th.col_ok = th.col < g.D;
  return th;
}

// Runs body(ticket, epoch) for the chunks of this workgroup: with the look-back
// (PH = EW_LOOKBACK) a persistent workgroup takes tickets until they run out
// (mg_persistent); the two-launch forms take one chunk per workgroup, in
// workgroup order, since no workgroup waits on another.
template <int PH, bool UNI = false, typename Body>
__device__ __forceinline__ void ew_chunks(const EwGeom& g, unsigned* header, Body&& body) {
  if constexpr (PH == EW_LOOKBACK) {
    mg_persistent<UNI>(header, (unsigned)g.n_lg * (unsigned)g.n_chunks, body);
  } else {
    body(blockIdx.x, PH == EW_AGG ? ew_agg_begin(header) : 0ull);
  }
}

// ---------------------------------------------------------------------------
// Forward of linear_scan: a, b -> A (running product), Bc (zero-start solution).
// ---------------------------------------------------------------------------
template <int VEC, int TSUB, int WAVES, int PH = EW_LOOKBACK>
__global__ __launch_bounds__(MG_WAVE* WAVES) void ew_fwd_kernel(
    const float* __restrict__ x0, const float* __restrict__ x1, float* __restrict__ out0,
    float* __restrict__ out1, EwGeom g, unsigned* header, mg_slot_t* agg_data,
    mg_slot_t* incl_data) {
  constexpr bool NT = PH != EW_REDUCE;
  using Rows = float[TSUB][VEC];
  const int64_t T = g.T, D = g.D;
  // The thread's TSUB rows of a and b for ticket `ticket` (identity past the end).
  auto load = [&](unsigned ticket, Rows& av, Rows& bv) {
    const EwThread th = ew_thread_at<VEC, false>(g, ticket, 0u);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        load_vec<VEC, NT>(av[s], x0 + (th.bb * T + t) * D + th.col);
        load_vec<VEC, NT>(bv[s], x1 + (th.bb * T + t) * D + th.col);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          av[s][v] = 1.f;
          bv[s][v] = 0.f;
        }
      }
    }
  };
  // The chunk from its rows: local aggregates, then `mid` (run by every thread),
  // then the carry and the outputs.
  auto finish = [&](unsigned ticket, unsigned long long epoch, const Rows& av, const Rows& bv, auto&& mid) {
    const EwThread th = ew_thread_at<VEC, false>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    Aff<1> loc[VEC], seed[VEC], carry[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      loc[v] = aff_identity<1>();
#pragma unroll
      for (int s = 0; s < TSUB; ++s) {
        loc[v].l[0] = fmaf(av[s][v], loc[v].l[0], bv[s][v]);
        loc[v].p *= av[s][v];
      }
      seed[v] = aff_identity<1>();
    }
    mid();
    ew_carry<Aff<1>, VEC, WAVES, false, PH>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                            incl_data, carry);
    if constexpr (PH == EW_REDUCE) return;

    float P[VEC], L[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      P[v] = carry[v].p;
      L[v] = carry[v].l[0];
    }
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        L[v] = fmaf(av[s][v], L[v], bv[s][v]);
        P[v] *= av[s][v];
      }
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        const int64_t off = (th.bb * T + t) * D + th.col;
        store_vec<VEC>(out0 + off, P);
        store_vec<VEC>(out1 + off, L);
      }
    }
  };
  if constexpr (PH != EW_LOOKBACK) {
    const unsigned long long tag = PH == EW_AGG ? ew_agg_begin(header) : 0ull;
    Rows av, bv;
    load(blockIdx.x, av, bv);
    finish(blockIdx.x, tag, av, bv, [] {});
  } else {
    // Persistent workgroups (mg_persistent's protocol) with two row buffers: the
    // next ticket is shared once this chunk's local aggregates are formed, and its
    // rows load while this chunk's carry and outputs run.
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
    Rows a0, b0, a1, b1;
    if (t < chunks) load(t, a0, b0);
    auto step = [&](unsigned tk, const Rows& av, const Rows& bv, Rows& nav, Rows& nbv) {
      unsigned next = 0u;
      if (threadIdx.x == 0) next = mg_next_ticket(header, e, chunks);
      unsigned tn = 0u;
      finish(tk, e, av, bv, [&] {
        if (threadIdx.x == 0) s_ticket = next;
        __syncthreads();
        tn = s_ticket;
        if (tn < chunks) load(tn, nav, nbv);
      });
      return tn;
    };
    while (t < chunks) {
      t = step(t, a0, b0, a1, b1);
      if (t >= chunks) break;
      t = step(t, a1, b1, a0, b0);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward of linear_scan.  Inputs a, saved A, Bc and grads gA, gB (b is not
// read); outputs da, db.  Adjoint: x_t = g_t + a_{t+1} x_{t+1} for both streams;
// da_t = xA_t A_{t-1} + xB_t Bc_{t-1}, db_t = xB_t.  Bc_{t-1} is read per step
// (the saved rows shifted by one, as many bytes as b's); A_{t-1} follows from the
// row before the wave's first step, times a.
// ---------------------------------------------------------------------------
template <int VEC, int TSUB, int WAVES, int PH = EW_LOOKBACK>
__global__ __launch_bounds__(MG_WAVE* WAVES) void linear_bwd_kernel(
    const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ A,
    const float* __restrict__ Bc, const float* __restrict__ gA, const float* __restrict__ gB,
    float* __restrict__ da, float* __restrict__ db, EwGeom g, unsigned* header,
    mg_slot_t* agg_data, mg_slot_t* incl_data) {
  constexpr bool NT = PH != EW_REDUCE;
  // Uniform tickets: without them this kernel spills 38 registers at the cap.
  ew_chunks<PH, true>(g, header, [&](unsigned ticket, unsigned long long epoch) {
    EwThread th = ew_thread_at<VEC, true, true>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    const int64_t T = g.T, D = g.D;

    // bp[s] = Bc_{t0+s-1} (zero before the sequence start).
    float av[TSUB][VEC], bp[TSUB][VEC], xa[TSUB][VEC], xb[TSUB][VEC];
    float Ap[VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        const int64_t off = (th.bb * T + t) * D + th.col;
        load_vec<VEC, NT>(av[s], a + off);
        if constexpr (PH != EW_REDUCE) {
          if (t > 0) {
            load_vec<VEC>(bp[s], Bc + off - D);
          } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) bp[s][v] = 0.f;
          }
        }
        load_vec<VEC, NT>(xa[s], gA + off);
        load_vec<VEC, NT>(xb[s], gB + off);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          av[s][v] = 1.f;
          bp[s][v] = 0.f;
          xa[s][v] = 0.f;
          xb[s][v] = 0.f;
        }
      }
    }
    if (th.col_ok && t0 > 0 && t0 <= T) {
      load_vec<VEC>(Ap, A + (th.bb * T + t0 - 1) * D + th.col);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) Ap[v] = 1.f;
    }

    Aff<2> loc[VEC], seed[VEC], carry[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      loc[v] = aff_identity<2>();
#pragma unroll
      for (int s = TSUB - 1; s >= 0; --s) {
        const float al = av[s][v];
        loc[v].l[0] = al * (xa[s][v] + loc[v].l[0]);
        loc[v].l[1] = al * (xb[s][v] + loc[v].l[1]);
        loc[v].p *= al;
      }
      seed[v] = aff_identity<2>();
    }
    ew_carry<Aff<2>, VEC, WAVES, true, PH>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                           incl_data, carry);
    if constexpr (PH == EW_REDUCE) return;

    float ya[VEC], yb[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      ya[v] = carry[v].l[0];
      yb[v] = carry[v].l[1];
    }
#pragma unroll
    for (int s = TSUB - 1; s >= 0; --s) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        xa[s][v] += ya[v];
        xb[s][v] += yb[v];
        ya[v] = av[s][v] * xa[s][v];
        yb[v] = av[s][v] * xb[s][v];
      }
    }
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      float d_a[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        d_a[v] = fmaf(xa[s][v], Ap[v], xb[s][v] * bp[s][v]);
        Ap[v] *= av[s][v];
      }
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        const int64_t off = (th.bb * T + t) * D + th.col;
        store_vec<VEC>(da + off, d_a);
        store_vec<VEC>(db + off, xb[s]);
      }
    }
  });
}

// ---------------------------------------------------------------------------
// parallel_scan_log (reference src/mingru/min_gru.py:755-807) on
// extended-range values (Xf above).
//   forward:  h_t = a_t h_{t-1} + b_t with a_t = e^{lc_t}, b_t = e^{lv_{t+1}}
//             and h_{-1} = e^{lv_0}.  Every term is positive, so there is no
//             cancellation and each step keeps fp32's relative rounding.  The
//             forward also records h_{t0-1} (as Xf) at every sub-chunk start
//             t0 into `hstate` (B, ceil(T/LOG_TSUB), 2, D) when it is given, so
//             the backward restarts the recurrence from values that an fp32 h
//             could not hold.
//   backward: adjoint x_t = gh_t + a_{t+1} x_{t+1};  dlc_t = x_t a_t h_{t-1};
//             dlv_{t+1} = x_t b_t;  dlv_0 = a_0 x_0 h_{-1}.
// Both directions use LOG_TSUB-step sub-chunks, the granularity of `hstate`.
// ---------------------------------------------------------------------------
constexpr int LOG_TSUB = 8;
constexpr int LOG_WAVES = 8;

template <int VEC, bool NT = true>
__device__ __forceinline__ void load_xf_exp(Xf (&dst)[VEC], const float* __restrict__ src) {
  float x[VEC];
  load_vec<VEC, NT>(x, src);
#pragma unroll
  for (int v = 0; v < VEC; ++v) dst[v] = xf_exp(x[v]);
}

template <int VEC, int WAVES, int PH = EW_LOOKBACK>
__global__ __launch_bounds__(MG_WAVE* WAVES) void log_fwd_kernel(
    const float* __restrict__ lc, const float* __restrict__ lv, float* __restrict__ h,
    float* __restrict__ hstate, EwGeom g, unsigned* header, mg_slot_t* agg_data,
    mg_slot_t* incl_data) {
  constexpr int TSUB = LOG_TSUB;
  constexpr bool NT = PH != EW_REDUCE;
  ew_chunks<PH>(g, header, [&](unsigned ticket, unsigned long long epoch) {
    EwThread th = ew_thread_at<VEC, false>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    const int64_t T = g.T, D = g.D;

    // Every raw load first, then the exponentials: with each step's exponentials
    // next to its loads the compiler waited for them step by step.
    float ra[TSUB][VEC], rb[TSUB][VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        load_vec<VEC, NT>(ra[s], lc + (th.bb * T + t) * D + th.col);
        load_vec<VEC, NT>(rb[s], lv + (th.bb * (T + 1) + t + 1) * D + th.col);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          ra[s][v] = 0.f;  // unused: the step is past the end
          rb[s][v] = 0.f;
        }
      }
    }
    Xf av[TSUB][VEC], bv[TSUB][VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const bool ok = th.col_ok && t0 + s < T;
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        av[s][v] = ok ? xf_exp(ra[s][v]) : Xf{1.f, 0.f};
        bv[s][v] = ok ? xf_exp(rb[s][v]) : xf_zero();
      }
    }

    XAff loc[VEC], seed[VEC], carry[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      Xf P{1.f, 0.f}, L = xf_zero();
#pragma unroll
      for (int s = 0; s < TSUB; ++s) {
        L = xf_fma(av[s][v], L, bv[s][v]);
        P = xf_mul(P, av[s][v]);
      }
      loc[v] = XAff{xf_norm(P), xf_norm(L)};
      seed[v] = XAff::identity();
    }
    if (th.c == 0 && th.w == 0 && th.col_ok) {
      Xf h0[VEC];
      load_xf_exp<VEC>(h0, lv + (th.bb * (T + 1)) * D + th.col);
#pragma unroll
      for (int v = 0; v < VEC; ++v) seed[v].l = h0[v];
    }
    ew_carry<XAff, VEC, WAVES, false, PH>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                          incl_data, carry);
    if constexpr (PH == EW_REDUCE) return;

    Xf L[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) L[v] = carry[v].l;
    if (hstate != nullptr && th.col_ok && t0 < T) {
      const int64_t nsub = (T + TSUB - 1) / TSUB;
      float* st = hstate + ((th.bb * nsub + t0 / TSUB) * 2) * D + th.col;
      float ss[VEC], se[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        ss[v] = L[v].s;
        se[v] = L[v].e;
      }
      store_vec<VEC>(st, ss);
      store_vec<VEC>(st + D, se);
    }
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      float out[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        L[v] = xf_fma(av[s][v], L[v], bv[s][v]);
        out[v] = xf_to_float(L[v]);
      }
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) store_vec<VEC>(h + (th.bb * T + t) * D + th.col, out);
    }
  });
}

template <int VEC, int WAVES, int PH = EW_LOOKBACK>
__global__ __launch_bounds__(MG_WAVE* WAVES) void log_bwd_kernel(
    const float* __restrict__ lc, const float* __restrict__ lv, const float* __restrict__ h,
    const float* __restrict__ hstate, const float* __restrict__ gh, float* __restrict__ dlc,
    float* __restrict__ dlv, EwGeom g, unsigned* header, mg_slot_t* agg_data,
    mg_slot_t* incl_data) {
  constexpr int TSUB = LOG_TSUB;
  constexpr bool NT = PH != EW_REDUCE;
  ew_chunks<PH>(g, header, [&](unsigned ticket, unsigned long long epoch) {
    EwThread th = ew_thread_at<VEC, true>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    const int64_t T = g.T, D = g.D;

    // a as Xf; lv and gh raw until needed.
    float ra[TSUB][VEC], lvr[TSUB][VEC], gr[TSUB][VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        load_vec<VEC, NT>(ra[s], lc + (th.bb * T + t) * D + th.col);
        if constexpr (PH != EW_REDUCE) load_vec<VEC>(lvr[s], lv + (th.bb * (T + 1) + t + 1) * D + th.col);
        load_vec<VEC, NT>(gr[s], gh + (th.bb * T + t) * D + th.col);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          ra[s][v] = 0.f;  // unused: the step is past the end
          lvr[s][v] = -INFINITY;
          gr[s][v] = 0.f;
        }
      }
    }
    // The exponentials after every load is issued (as in the forward).
    Xf av[TSUB][VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const bool ok = th.col_ok && t0 + s < T;
#pragma unroll
      for (int v = 0; v < VEC; ++v) av[s][v] = ok ? xf_exp(ra[s][v]) : Xf{1.f, 0.f};
    }
    // An fp32 value as Xf without normalising: only an exact zero needs exponent -inf.
    auto raw = [](float x) { return Xf{x, x == 0.f ? -INFINITY : 0.f}; };

    XAff loc[VEC], seed[VEC], carry[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      Xf P{1.f, 0.f}, L = xf_zero();
#pragma unroll
      for (int s = TSUB - 1; s >= 0; --s) {
        L = xf_mul(av[s][v], xf_add(raw(gr[s][v]), L));
        P = xf_mul(P, av[s][v]);
      }
      loc[v] = XAff{xf_norm(P), xf_norm(L)};
      seed[v] = XAff::identity();
    }
    ew_carry<XAff, VEC, WAVES, true, PH>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                         incl_data, carry);
    if constexpr (PH == EW_REDUCE) return;

    // Total adjoint x_s of every step; y ends as a_{t0} x_{t0}.
    Xf x[TSUB][VEC], y[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) y[v] = carry[v].l;
#pragma unroll
    for (int s = TSUB - 1; s >= 0; --s) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        x[s][v] = xf_add(raw(gr[s][v]), y[v]);
        y[v] = xf_mul(av[s][v], x[s][v]);
      }
    }

    // h_{t0-1}: e^{lv_0} at the sequence start, else the forward's record.
    Xf hp[VEC];
    const bool first_sub = (t0 == 0);
#pragma unroll
    for (int v = 0; v < VEC; ++v) hp[v] = xf_zero();
    if (th.col_ok && t0 < T) {
      if (first_sub) {
        load_xf_exp<VEC>(hp, lv + (th.bb * (T + 1)) * D + th.col);
      } else if (hstate != nullptr) {
        const int64_t nsub = (T + TSUB - 1) / TSUB;
        const float* st = hstate + ((th.bb * nsub + t0 / TSUB) * 2) * D + th.col;
        float ss[VEC], se[VEC];
        load_vec<VEC>(ss, st);
        load_vec<VEC>(se, st + D);
#pragma unroll
        for (int v = 0; v < VEC; ++v) hp[v] = Xf{ss[v], se[v]};
      } else {
        float hv[VEC];
        load_vec<VEC>(hv, h + (th.bb * T + t0 - 1) * D + th.col);
#pragma unroll
        for (int v = 0; v < VEC; ++v) hp[v] = xf_from(hv[v]);
      }
    }
    if (first_sub && th.col_ok) {
      float d0[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) d0[v] = xf_to_float(xf_mul(y[v], hp[v]));
      store_vec<VEC>(dlv + (th.bb * (T + 1)) * D + th.col, d0);
    }
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      float d_c[VEC], d_v[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const Xf b = lvr[s][v] == -INFINITY ? xf_zero() : xf_exp(lvr[s][v]);
        d_c[v] = xf_to_float(xf_mul(xf_mul(x[s][v], av[s][v]), hp[v]));
        d_v[v] = xf_to_float(xf_mul(x[s][v], b));
        hp[v] = xf_fma(av[s][v], hp[v], b);
      }
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        store_vec<VEC>(dlc + (th.bb * T + t) * D + th.col, d_c);
        store_vec<VEC>(dlv + (th.bb * (T + 1) + t + 1) * D + th.col, d_v);
      }
    }
  });
}

// ---------------------------------------------------------------------------
// Fused gates + scan.  The coefficients are formed in registers from the
// mixer's pre-activations and the scan is seeded with h0, so one pass reads
// the pre-activations and writes only h; the backward returns the
// pre-activation gradients directly.
//   GATE_SIGNED (/_COUPLED): SignedMinGRU (reference src/mingru/min_gru.py:
//     1788-1857), inputs s, z, hpre and h0:
//     a = tanh(s) [* (1 - sigmoid(z))], b = sigmoid(z) * hpre, h = A h0 + Bc.
//   GATE_MINGRU: MinGRU (reference :1366-1397), inputs k, hpre and log h0:
//     a = sigmoid(-k) = exp(-softplus(k)), b = sigmoid(k) g(hpre)
//     = exp(log z + log_g(hpre)), h0 = exp(log h0); the log-space scan
//     parallel_scan_log(log a, [log h0, log b]) run in linear space, where every
//     term is positive.  g(x) = x + 1/2 for x >= 0, sigmoid(x) otherwise.
// ---------------------------------------------------------------------------
// Pre-activation inputs: (s, z, hpre) for the signed gates, (k, hpre) for MinGRU.
template <int G>
constexpr int gate_inputs() {
  return G == GATE_MINGRU ? 2 : 3;
}

// Time decay of the fused gate scans (DEC): the coefficient a is multiplied by
// gamma = exp(-lam[d] dt[b, t]) (the mixers' DecayMixin, reference
// src/mingru/min_gru.py:1807-1813 for SignedMinGRU; MinGRU's log-space form
// log a - lam dt, :1383-1393, is the same factor).  dt (B, T) is already
// normalised by the caller, lam (D) holds the per-channel rate (a fixed rate
// broadcast).  The backward writes, when asked, deterministic partial sums of
//   dL/dlam[d]  = -sum_{b,t} dt a dL/da      into dlam [B * chunks][D] (one row per
//                                            (batch row, 32-step backward chunk)),
//   dL/ddt[b,t] = -sum_d lam a dL/da         into ddt [ceil(D / 64)][B][T] (one row
//                                            per tile of 64 columns),
// with a the decayed coefficient; the caller sums the rows.
struct GateDecay {
  const float* dt;
  const float* lam;
  float* dlam;  // backward; may be null
  float* ddt;   // backward; may be null
};

constexpr float GATE_LOG2E = 1.44269504088896341f;

// -lam log2(e) for the thread's VEC columns: one vector load where all of them exist
// and the address allows it (a caller's pointer may have any alignment).
template <int VEC>
__device__ __forceinline__ void decay_rates(float (&nlam)[VEC], const float* lam, int64_t col,
                                            int64_t D) {
  if (col + VEC <= D && ((uintptr_t)(lam + col) & (sizeof(float) * VEC - 1)) == 0) {
    load_vec<VEC, false>(nlam, lam + col);
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) nlam[v] = col + v < D ? lam[col + v] : 0.f;
  }
#pragma unroll
  for (int v = 0; v < VEC; ++v) nlam[v] *= -GATE_LOG2E;
}

// dt[row + s] for a wave's TSUB steps (0 from step n on), the same in every lane:
// lane s loads step s, and each step's value is read back from its lane, one
// vector load per wave instead of one per step.
template <int TSUB>
__device__ __forceinline__ void decay_gaps(float (&dts)[TSUB], const float* dt, int64_t row,
                                           int64_t n, int lane) {
  static_assert(TSUB <= MG_WAVE, "one lane per step");
  const float mine = lane < TSUB && lane < n ? dt[row + lane] : 0.f;
#pragma unroll
  for (int s = 0; s < TSUB; ++s)
    dts[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), s));
}

template <int VEC, int TSUB, int WAVES, int G, bool DEC, int PH = EW_LOOKBACK>
__global__ __launch_bounds__(MG_WAVE* WAVES) void gate_fwd_kernel(
    const float* __restrict__ p0, const float* __restrict__ p1, const float* __restrict__ p2,
    const float* __restrict__ h0, float* __restrict__ h, GateDecay dec, EwGeom g,
    unsigned* header, mg_slot_t* agg_data, mg_slot_t* incl_data) {
  constexpr bool NT = PH != EW_REDUCE;
  ew_chunks<PH>(g, header, [&](unsigned ticket, unsigned long long epoch) {
    EwThread th = ew_thread_at<VEC, false>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    const int64_t T = g.T, D = g.D;
    float nlam[VEC], dts[TSUB];  // -lam log2(e) per column, dt per step
    if constexpr (DEC) {
      decay_rates<VEC>(nlam, dec.lam, th.col, D);
      decay_gaps<TSUB>(dts, dec.dt, th.bb * T + t0, T - t0, th.lane);
    }

    float av[TSUB][VEC], bv[TSUB][VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        const int64_t off = (th.bb * T + t) * D + th.col;
        float x0[VEC], x1[VEC], x2[VEC];
        load_vec<VEC, NT>(x0, p0 + off);
        load_vec<VEC, NT>(x1, p1 + off);
        if constexpr (gate_inputs<G>() == 3) load_vec<VEC, NT>(x2, p2 + off);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          gate_coeffs<G>(x0[v], x1[v], gate_inputs<G>() == 3 ? x2[v] : 0.f, av[s][v], bv[s][v]);
          if constexpr (DEC) av[s][v] *= __builtin_amdgcn_exp2f(nlam[v] * dts[s]);
        }
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          av[s][v] = 1.f;
          bv[s][v] = 0.f;
        }
      }
    }
    Aff<1> loc[VEC], seed[VEC], carry[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      loc[v] = aff_identity<1>();
#pragma unroll
      for (int s = 0; s < TSUB; ++s) {
        loc[v].l[0] = fmaf(av[s][v], loc[v].l[0], bv[s][v]);
        loc[v].p *= av[s][v];
      }
      seed[v] = aff_identity<1>();
    }
    if (th.c == 0 && th.w == 0 && th.col_ok) {
      float x[VEC];
      load_vec<VEC>(x, h0 + th.bb * D + th.col);
#pragma unroll
      for (int v = 0; v < VEC; ++v) seed[v].l[0] = G == GATE_MINGRU ? expf(x[v]) : x[v];
    }
    ew_carry<Aff<1>, VEC, WAVES, false, PH>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                            incl_data, carry);
    if constexpr (PH == EW_REDUCE) return;
    float L[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) L[v] = carry[v].l[0];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) L[v] = fmaf(av[s][v], L[v], bv[s][v]);
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) store_vec<VEC>(h + (th.bb * T + t) * D + th.col, L);
    }
  });
}

// Backward: x_t = dL/dh_t in total (reverse scan of g_t with the a's), then
// da = x h_{t-1}, db = x, dh0 = a_1 x_1, through the gate derivatives.  Per step
// the kernel keeps the adjoint and three gate values:
//   signed: sigmoid(z), tanh(s), hpre;   MinGRU: sigmoid(-k), sigmoid(k), hpre.
template <int VEC, int TSUB, int WAVES, int G, bool DEC, int PH = EW_LOOKBACK>
__global__ __launch_bounds__(MG_WAVE* WAVES) void gate_bwd_kernel(
    const float* __restrict__ p0, const float* __restrict__ p1, const float* __restrict__ p2,
    const float* __restrict__ h0, const float* __restrict__ h, const float* __restrict__ gh,
    float* __restrict__ d0, float* __restrict__ d1, float* __restrict__ d2,
    float* __restrict__ dh0, GateDecay dec, EwGeom g, unsigned* header, mg_slot_t* agg_data,
    mg_slot_t* incl_data) {
  // dL/dlam partials of the workgroup's waves (DEC with dlam).
  __shared__ float s_dlam[DEC ? WAVES : 1][DEC ? MG_WAVE * VEC : 1];
  ew_chunks<PH>(g, header, [&](unsigned ticket, unsigned long long epoch) {
    EwThread th = ew_thread_at<VEC, true>(g, ticket, epoch);
    const int64_t t0 = (int64_t)th.c * (WAVES * TSUB) + th.w * TSUB;
    const int64_t T = g.T, D = g.D;
    constexpr bool MIN = G == GATE_MINGRU;
    constexpr bool NT = PH != EW_REDUCE;
    // Decay: -lam log2(e) per column and dt per step (one value per wave and step).
    float nlam[VEC], dts[TSUB];
    if constexpr (DEC) {
      decay_rates<VEC>(nlam, dec.lam, th.col, D);
      decay_gaps<TSUB>(dts, dec.dt, th.bb * T + t0, T - t0, th.lane);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) nlam[v] = 0.f;
#pragma unroll
      for (int s = 0; s < TSUB; ++s) dts[s] = 0.f;
    }
    auto gam = [&](int s, int v) {
      return DEC ? __builtin_amdgcn_exp2f(nlam[v] * dts[s]) : 1.f;
    };

    float ua[TSUB][VEC], ub[TSUB][VEC], hv[TSUB][VEC], x[TSUB][VEC];
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      const int64_t t = t0 + s;
      if (th.col_ok && t < T) {
        const int64_t off = (th.bb * T + t) * D + th.col;
        float x0[VEC];
        load_vec<VEC, NT>(x0, p0 + off);
        load_vec<VEC, NT>(x[s], gh + off);
        if constexpr (MIN) {
          if constexpr (PH != EW_REDUCE) load_vec<VEC>(hv[s], p1 + off);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            ua[s][v] = mg_sigmoid(-x0[v]);  // a
            ub[s][v] = mg_sigmoid(x0[v]);   // z
          }
        } else {
          float x1[VEC];
          load_vec<VEC, NT>(x1, p1 + off);
          if constexpr (PH != EW_REDUCE) load_vec<VEC>(hv[s], p2 + off);
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            ua[s][v] = mg_sigmoid(x1[v]);  // sigmoid(z)
            ub[s][v] = mg_tanh(x0[v]);     // tanh(s)
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          ua[s][v] = 0.f;  // a = 0 closes the adjoint chain past T
          ub[s][v] = 0.f;
          hv[s][v] = 0.f;
          x[s][v] = 0.f;
        }
      }
    }
    auto coef_a0 = [&](int s, int v) {  // the coefficient before decay
      if constexpr (MIN) return ua[s][v];
      else if constexpr (G == GATE_SIGNED_COUPLED) return (1.f - ua[s][v]) * ub[s][v];
      else return ub[s][v];
    };
    auto coef_a = [&](int s, int v) { return DEC ? coef_a0(s, v) * gam(s, v) : coef_a0(s, v); };
    const bool first_sub = (t0 == 0);
    float hprev[VEC];
    if (th.col_ok && t0 <= T) {
      if (first_sub) {
        load_vec<VEC>(hprev, h0 + th.bb * D + th.col);
        if constexpr (MIN) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) hprev[v] = expf(hprev[v]);
        }
      } else {
        load_vec<VEC>(hprev, h + (th.bb * T + t0 - 1) * D + th.col);
      }
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) hprev[v] = 0.f;
    }

    Aff<1> loc[VEC], seed[VEC], carry[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      loc[v] = aff_identity<1>();
#pragma unroll
      for (int s = TSUB - 1; s >= 0; --s) {
        const float a = coef_a(s, v);
        loc[v].l[0] = a * (x[s][v] + loc[v].l[0]);
        loc[v].p *= a;
      }
      seed[v] = aff_identity<1>();
    }
    ew_carry<Aff<1>, VEC, WAVES, true, PH>(loc, seed, g, th.lg, th.c, header, th.epoch, agg_data,
                                           incl_data, carry);
    if constexpr (PH == EW_REDUCE) return;
    float y[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) y[v] = carry[v].l[0];
#pragma unroll
    for (int s = TSUB - 1; s >= 0; --s) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        x[s][v] += y[v];
        y[v] = coef_a(s, v) * x[s][v];
      }
    }
    if (first_sub && th.col_ok) {
      // dL/dh0 = a_1 x_1; the MinGRU input is log h0: times h0.
      if constexpr (MIN) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) y[v] *= hprev[v];
      }
      store_vec<VEC>(dh0 + th.bb * D + th.col, y);
    }
    // Decay: dL/dlam accumulated over this wave's steps, per column.
    float dl[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) dl[v] = 0.f;
#pragma unroll
    for (int s = 0; s < TSUB; ++s) {
      float o0[VEC], o1[VEC], o2[VEC];
      float cdt = 0.f;  // this lane's share of dL/ddt at this step
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        // dL/da_t of the decayed coefficient, and (da) of the coefficient before decay.
        const float xv = x[s][v], dae = xv * hprev[v];
        const float gm = gam(s, v), da = DEC ? dae * gm : dae;
        float a, b;
        if constexpr (MIN) {
          // a = sigmoid(-k): da/dk = -a z;  b = z g(hpre): db/dk = z a g, db/dhpre = z g'.
          const float hp = hv[s][v], am = ua[s][v], zk = ub[s][v];
          const float gv = hp >= 0.f ? hp + 0.5f : mg_sigmoid(hp);
          const float gp = hp >= 0.f ? 1.f : gv * (1.f - gv);
          a = am;
          b = zk * gv;
          o0[v] = (xv * gv - da) * am * zk;
          o1[v] = xv * zk * gp;
        } else {
          const float sg = ua[s][v], tv = ub[s][v], dsg = sg * (1.f - sg);
          a = G == GATE_SIGNED_COUPLED ? (1.f - sg) * tv : tv;
          b = sg * hv[s][v];
          o0[v] = da * (G == GATE_SIGNED_COUPLED ? (1.f - sg) : 1.f) * (1.f - tv * tv);
          o1[v] = xv * hv[s][v] * dsg - (G == GATE_SIGNED_COUPLED ? da * tv * dsg : 0.f);
          o2[v] = xv * sg;
        }
        if constexpr (DEC) {
          a *= gm;
          const float w = a * dae;  // (decayed a) dL/da; zero past the end and on idle columns
          dl[v] = fmaf(-dts[s], w, dl[v]);
          cdt = fmaf(nlam[v], w, cdt);  // -lam log2(e) a dL/da
        }
        hprev[v] = fmaf(a, hprev[v], b);
      }
      const int64_t t = t0 + s;
      if constexpr (DEC) {
        if (dec.ddt != nullptr) {
          // Sum over each 64-column tile: the 64 / VEC lanes that hold it.
          cdt = mg_group_sum<MG_WAVE / VEC>(cdt);
          const int64_t tile = th.col / MG_WAVE;
          if ((th.lane & (MG_WAVE / VEC - 1)) == 0 && th.col < D && t < T)
            dec.ddt[(tile * (int64_t)(g.n_lg / g.n_tiles) + th.bb) * T + t] =
                cdt * 0.693147180559945309f;  // undo the log2(e) of nlam
        }
      }
      if (th.col_ok && t < T) {
        const int64_t off = (th.bb * T + t) * D + th.col;
        store_vec<VEC>(d0 + off, o0);
        store_vec<VEC>(d1 + off, o1);
        if constexpr (!MIN) store_vec<VEC>(d2 + off, o2);
      }
    }
    if constexpr (DEC) {
      if (dec.dlam != nullptr) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) s_dlam[th.w][th.lane * VEC + v] = dl[v];
        __syncthreads();
        if (th.w == 0 && th.col_ok) {
          float acc[VEC];
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            acc[v] = 0.f;
            for (int j = 0; j < WAVES; ++j) acc[v] += s_dlam[j][th.lane * VEC + v];
          }
          float* row = dec.dlam + ((int64_t)th.bb * g.n_chunks + th.c) * D + th.col;
#pragma unroll
          for (int v = 0; v < VEC; ++v)
            if (th.col + v < D) row[v] = acc[v];
        }
        __syncthreads();  // s_dlam is free for the workgroup's next chunk
      }
    }
  });
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

struct EwPlan {
  EwGeom g;
  int waves;
  size_t agg_off, incl_off, total;
};

EwPlan ew_plan(int64_t B, int64_t T, int64_t D, int vec, int tsub, int waves, int nl) {
  EwPlan p;
  p.waves = waves;
  p.g.T = T;
  p.g.D = D;
  const int tile = MG_WAVE * vec;
  p.g.n_tiles = (int)((D + tile - 1) / tile);
  p.g.n_lg = (int)(B * p.g.n_tiles);
  const int64_t cl = (int64_t)waves * tsub;
  p.g.n_chunks = (int)((T + cl - 1) / cl);
  const size_t n = (size_t)p.g.n_lg * p.g.n_chunks;
  const size_t slot_bytes = n * (size_t)(nl + 1) * tile * sizeof(mg_slot_t);
  p.agg_off = MG_HEADER_BYTES;
  p.incl_off = p.agg_off + mg_align_up(slot_bytes, 256);
  p.total = p.incl_off + mg_align_up(slot_bytes, 256);
  return p;
}

bool is_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Columns per lane of a launch.  4 (16-byte accesses) when the inputs allow it,
// the row is at least one 256-column tile wide and the launch still gives every
// CU a workgroup; otherwise the widest of 2 and 1 that does, or 1.  Narrower lanes
// multiply a small problem's workgroups: at B=4, T=1024, D=256 the log scan's
// forward and backward take 9.8 and 11.4 us with 1 column per lane against 21.0
// and 17.8 us with 4 (32 and 64 workgroups).
int ew_vec(int64_t B, int64_t T, int64_t D, bool v4ok, int chunk) {
  if (!v4ok) return 1;
  const int64_t chunks = (T + chunk - 1) / chunk;
  for (int vec = 4; vec > 1; vec /= 2) {
    const int64_t tile = (int64_t)MG_WAVE * vec;
    if (tile <= D && B * ((D + tile - 1) / tile) * chunks >= EW_FILL_WGS) return vec;
  }
  return 1;
}

// Calls f(std::integral_constant<int, vec>) for vec in {4, 2, 1}.
template <typename F>
int by_vec(int vec, F&& f) {
  if (vec == 4) return f(std::integral_constant<int, 4>{});
  if (vec == 2) return f(std::integral_constant<int, 2>{});
  return f(std::integral_constant<int, 1>{});
}

bool geometry_ok(int64_t B, int64_t T, int64_t D) {
  if (B <= 0 || T <= 0 || D <= 0) return false;
  // Tickets, look-back indices and grid sizes stay well inside 32 bits.
  const int64_t lgs = B * ((D + MG_WAVE - 1) / MG_WAVE);
  const int64_t chunks = (T + 7) / 8;
  return lgs * chunks < (1ll << 24);
}

template <typename Kernel, typename... Args>
int ew_launch(Kernel k, const EwPlan& p, void* ws, hipStream_t stream, bool persistent,
              Args... args) {
  unsigned* header = (unsigned*)ws;
  mg_slot_t* agg = (mg_slot_t*)((char*)ws + p.agg_off);
  mg_slot_t* incl = (mg_slot_t*)((char*)ws + p.incl_off);
  const unsigned chunks = (unsigned)p.g.n_lg * (unsigned)p.g.n_chunks;
  const unsigned grid =
      persistent ? std::min(chunks, mg_resident((const void*)k, MG_WAVE * p.waves)) : chunks;
  hipLaunchKernelGGL(k, dim3(grid), dim3(MG_WAVE * p.waves), 0, stream, args..., p.g, header,
                     agg, incl);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

// The two-launch form (EW_REDUCE then EW_FINAL) for a problem of `arrays` input
// arrays of B*T*D floats: few enough chunks per sequence for EW_FINAL's fold,
// and inputs small enough to stay cached between the launches.
bool ew_two_launch(const EwPlan& p, int64_t B, int64_t T, int64_t D, int arrays) {
  return p.g.n_chunks <= EW_FINAL_MAX_CHUNKS &&
         B * T * D * (int64_t)sizeof(float) * arrays <= EW_TWO_LAUNCH_BYTES;
}

// One look-back launch, or for a small problem one EW_AGG launch when its whole
// grid is resident at once (so the workgroups it waits on are running), else the
// reduce and final launches over the same grid.
// MINGRU_HIP_EW_FORM=two keeps a small problem on the two-launch form even where
// EW_AGG fits (the tests use it to cover both forms); unset, or any other value,
// leaves the choice to the residency check.
bool ew_force_two() {
  const char* v = getenv("MINGRU_HIP_EW_FORM");
  return v && v[0] == 't' && v[1] == 'w' && v[2] == 'o' && v[3] == 0;
}

template <typename K0, typename K1, typename K2, typename K3, typename... Args>
int ew_run(bool two, K0 lookback, K1 reduce, K2 fin, K3 agg, const EwPlan& p, void* ws,
           hipStream_t stream, Args... args) {
  if (!two) return ew_launch(lookback, p, ws, stream, true, args...);
  const unsigned chunks = (unsigned)p.g.n_lg * (unsigned)p.g.n_chunks;
  if (!ew_force_two() && chunks <= mg_resident((const void*)agg, MG_WAVE * p.waves))
    return ew_launch(agg, p, ws, stream, false, args...);
  const int rc = ew_launch(reduce, p, ws, stream, false, args...);
  return rc != MG_OK ? rc : ew_launch(fin, p, ws, stream, false, args...);
}

size_t ew_ws_bytes(int64_t B, int64_t T, int64_t D) {
  size_t m = 0;
  for (int vec : {1, 2, 4}) {
    m = std::max(m, ew_plan(B, T, D, vec, EW_TSUB_FWD, EW_WAVES_FWD, 1).total);
    m = std::max(m, ew_plan(B, T, D, vec, EW_TSUB_BWD, EW_WAVES_BWD, 2).total);
  }
  return m;
}

// Columns per lane of the log scans: 2 or 1.  Their extended-range values take
// twice the registers of the linear scan's, and 4 columns per lane spill.
int log_vec(int64_t B, int64_t T, int64_t D, std::initializer_list<const void*> ps) {
  uintptr_t bits = 0;
  for (const void* p : ps) bits |= (uintptr_t)p;
  const bool v2 = D % 2 == 0 && bits % 8 == 0;
  return std::min(2, ew_vec(B, T, D, v2, LOG_WAVES * LOG_TSUB));
}

// parallel_scan_log: Xf maps carry four look-back fields (ew_plan's nl = 3).
size_t log_ws_bytes(int64_t B, int64_t T, int64_t D) {
  size_t m = 0;
  for (int vec : {1, 2, 4}) m = std::max(m, ew_plan(B, T, D, vec, LOG_TSUB, LOG_WAVES, 3).total);
  return m;
}

size_t gate_ws_bytes(int64_t B, int64_t T, int64_t D) {
  size_t m = ew_ws_bytes(B, T, D);
  for (int vec : {1, 2, 4})
    m = std::max(m, ew_plan(B, T, D, vec, GATE_TSUB_BWD, GATE_WAVES_BWD, 1).total);
  for (int vec : {1, 2})
    m = std::max(m, ew_plan(B, T, D, vec, GATE_TSUB_FWD_NARROW, EW_WAVES_FWD, 1).total);
  return m;
}

bool all_aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && !is_aligned16(p)) return false;
  return true;
}

template <int G, bool DEC>
int gate_fwd_launch(const float* p0, const float* p1, const float* p2, const float* h0, float* h,
                    GateDecay dec, int64_t B, int64_t T, int64_t D, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
  const bool v4 = D % 4 == 0 && all_aligned16({p0, p1, p2, h0, h});
  const int vec = ew_vec(B, T, D, v4, EW_WAVES_FWD * EW_TSUB_FWD);
  return by_vec(vec, [&](auto v) {
    constexpr int V = decltype(v)::value;
    constexpr int TS = V == 4 ? EW_TSUB_FWD : GATE_TSUB_FWD_NARROW;
    EwPlan p = ew_plan(B, T, D, V, TS, EW_WAVES_FWD, 1);
    if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
    return ew_run(ew_two_launch(p, B, T, D, gate_inputs<G>()),
                  gate_fwd_kernel<V, TS, EW_WAVES_FWD, G, DEC>,
                  gate_fwd_kernel<V, TS, EW_WAVES_FWD, G, DEC, EW_REDUCE>,
                  gate_fwd_kernel<V, TS, EW_WAVES_FWD, G, DEC, EW_FINAL>,
                  gate_fwd_kernel<V, TS, EW_WAVES_FWD, G, DEC, EW_AGG>, p, ws, stream, p0, p1, p2,
                  h0, h, dec);
  });
}

// ---------------------------------------------------------------------------
// Static look-back scratch for callers that cannot allocate
// ---------------------------------------------------------------------------
// One array per device, holding the workspace of mg_linear_scan_fwd_noalloc.
// In host code `scratch` names a host-side stand-in, never the device memory:
// every host use goes through the address hipGetSymbolAddress returns for the
// current device, which is looked up once per device and cached.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;  // == MG_NOALLOC_SCRATCH_BYTES
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;

struct NoallocDevice {
  std::mutex mu;                     // serialises the one-time set-up
  std::atomic<void*> ptr{nullptr};   // device address of `scratch`, once set up
};
NoallocDevice g_noalloc[NOALLOC_MAX_DEVICES];

__global__ void zero_fill_kernel(uint4* __restrict__ p, size_t n16) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

int noalloc_device(int* dev) {
  if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= NOALLOC_MAX_DEVICES)
    return MG_ERR_RUNTIME;
  return MG_OK;
}

// The current device's scratch address, set up by the first call per device:
// the symbol lookup, then one zero fill on `stream` (the look-back workspace
// protocol starts from zeroed memory; later calls ordered on a stream after it
// reuse the contents unchanged).  The set-up is refused while `stream` is being
// captured: a captured fill would not run at capture time and would run again
// on every replay.
int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (noalloc_device(&dev) != MG_OK) return MG_ERR_RUNTIME;
  NoallocDevice& d = g_noalloc[dev];
  void* p = d.ptr.load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(d.mu);
    p = d.ptr.load(std::memory_order_relaxed);
    if (p == nullptr) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return MG_ERR_RUNTIME;
      if (cs != hipStreamCaptureStatusNone) return MG_ERR_CAPTURE;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
        return MG_ERR_RUNTIME;
      hipLaunchKernelGGL(zero_fill_kernel, dim3(1024), dim3(256), 0, stream, (uint4*)p,
                         NOALLOC_SCRATCH_BYTES / 16);
      if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
      d.ptr.store(p, std::memory_order_release);
    }
  }
  *out = p;
  return MG_OK;
}

template <int G, bool DEC>
int gate_bwd_launch(const float* p0, const float* p1, const float* p2, const float* h0,
                    const float* h, const float* gh, float* d0, float* d1, float* d2, float* dh0,
                    GateDecay dec, int64_t B, int64_t T, int64_t D, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
  const bool v4 = D % 4 == 0 && all_aligned16({p0, p1, p2, h0, h, gh, d0, d1, d2, dh0});
  const int vec = ew_vec(B, T, D, v4, GATE_WAVES_BWD * GATE_TSUB_BWD);
  return by_vec(vec, [&](auto v) {
    constexpr int V = decltype(v)::value;
    EwPlan p = ew_plan(B, T, D, V, GATE_TSUB_BWD, GATE_WAVES_BWD, 1);
    if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
    return ew_run(ew_two_launch(p, B, T, D, gate_inputs<G>() + 1),
                  gate_bwd_kernel<V, GATE_TSUB_BWD, GATE_WAVES_BWD, G, DEC>,
                  gate_bwd_kernel<V, GATE_TSUB_BWD, GATE_WAVES_BWD, G, DEC, EW_REDUCE>,
                  gate_bwd_kernel<V, GATE_TSUB_BWD, GATE_WAVES_BWD, G, DEC, EW_FINAL>,
                  gate_bwd_kernel<V, GATE_TSUB_BWD, GATE_WAVES_BWD, G, DEC, EW_AGG>, p, ws, stream,
                  p0, p1, p2, h0, h, gh, d0, d1, d2, dh0, dec);
  });
}

int linear_fwd_launch(const float* a, const float* b, float* A, float* Bc, int64_t B, int64_t T,
                      int64_t D, void* ws, size_t ws_bytes, hipStream_t stream) {
  const bool v4 = D % 4 == 0 && is_aligned16(a) && is_aligned16(b) && is_aligned16(A) &&
                  is_aligned16(Bc);
  const int vec = ew_vec(B, T, D, v4, EW_WAVES_FWD * EW_TSUB_FWD);
  return by_vec(vec, [&](auto v) {
    constexpr int V = decltype(v)::value;
    EwPlan p = ew_plan(B, T, D, V, EW_TSUB_FWD, EW_WAVES_FWD, 1);
    if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
    return ew_run(ew_two_launch(p, B, T, D, 2), ew_fwd_kernel<V, EW_TSUB_FWD, EW_WAVES_FWD>,
                  ew_fwd_kernel<V, EW_TSUB_FWD, EW_WAVES_FWD, EW_REDUCE>,
                  ew_fwd_kernel<V, EW_TSUB_FWD, EW_WAVES_FWD, EW_FINAL>,
                  ew_fwd_kernel<V, EW_TSUB_FWD, EW_WAVES_FWD, EW_AGG>, p, ws, stream, a, b, A,
                  Bc);
  });
}

// Workspace of the linear_scan forward alone, whatever lane width it picks.
size_t linear_fwd_ws_bytes(int64_t B, int64_t T, int64_t D) {
  size_t m = 0;
  for (int vec : {1, 2, 4})
    m = std::max(m, ew_plan(B, T, D, vec, EW_TSUB_FWD, EW_WAVES_FWD, 1).total);
  return m;
}

}  // namespace

extern "C" {

size_t mg_linear_scan_workspace_bytes(int64_t B, int64_t T, int64_t D) {
  return ew_ws_bytes(B, T, D);
}

size_t mg_log_scan_workspace_bytes(int64_t B, int64_t T, int64_t D) {
  return log_ws_bytes(B, T, D);
}

size_t mg_log_scan_state_bytes(int64_t B, int64_t T, int64_t D) {
  if (B <= 0 || T <= 0 || D <= 0) return 0;
  return (size_t)B * (size_t)((T + LOG_TSUB - 1) / LOG_TSUB) * 2 * (size_t)D * sizeof(float);
}

int mg_linear_scan_fwd(const float* a, const float* b, float* A, float* Bc, int64_t B, int64_t T,
                       int64_t D, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!a || !b || !A || !Bc || !ws || !geometry_ok(B, T, D)) return MG_ERR_ARG;
  return linear_fwd_launch(a, b, A, Bc, B, T, D, ws, ws_bytes, stream);
}

int mg_linear_scan_fwd_noalloc(const float* a, const float* b, float* A, float* Bc, int64_t B,
                               int64_t T, int64_t D, hipStream_t stream) {
  if (!a || !b || !A || !Bc || !geometry_ok(B, T, D)) return MG_ERR_ARG;
  if (linear_fwd_ws_bytes(B, T, D) > NOALLOC_SCRATCH_BYTES) return MG_ERR_TOO_LARGE;
  void* ws = nullptr;
  const int rc = noalloc_scratch(stream, &ws);
  if (rc != MG_OK) return rc;
  return linear_fwd_launch(a, b, A, Bc, B, T, D, ws, NOALLOC_SCRATCH_BYTES, stream);
}

int mg_scan_workspace_errors(const void* ws, unsigned* count, hipStream_t stream) {
  if (!ws || !count) return MG_ERR_ARG;
  unsigned v = 0;
  if (hipMemcpyAsync(&v, (const unsigned*)ws + MG_H_ERROR, sizeof(unsigned),
                     hipMemcpyDeviceToHost, stream) != hipSuccess)
    return MG_ERR_RUNTIME;
  if (hipStreamSynchronize(stream) != hipSuccess) return MG_ERR_RUNTIME;
  *count = v;
  return MG_OK;
}

int mg_linear_scan_noalloc_errors(unsigned* count, hipStream_t stream) {
  if (!count) return MG_ERR_ARG;
  int dev = -1;
  if (noalloc_device(&dev) != MG_OK) return MG_ERR_RUNTIME;
  const void* p = g_noalloc[dev].ptr.load(std::memory_order_acquire);
  if (p == nullptr) {  // never set up on this device: nothing has run
    *count = 0;
    return MG_OK;
  }
  return mg_scan_workspace_errors(p, count, stream);
}

int mg_linear_scan_bwd(const float* a, const float* b, const float* A, const float* Bc,
                       const float* gA, const float* gB, float* da, float* db, int64_t B,
                       int64_t T, int64_t D, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!a || !b || !A || !Bc || !gA || !gB || !da || !db || !ws || !geometry_ok(B, T, D))
    return MG_ERR_ARG;
  const bool v4 = D % 4 == 0 && is_aligned16(a) && is_aligned16(b) && is_aligned16(A) &&
                  is_aligned16(Bc) && is_aligned16(gA) && is_aligned16(gB) &&
                  is_aligned16(da) && is_aligned16(db);
  const int vec = ew_vec(B, T, D, v4, EW_WAVES_BWD * EW_TSUB_BWD);
  return by_vec(vec, [&](auto v) {
    constexpr int V = decltype(v)::value;
    EwPlan p = ew_plan(B, T, D, V, EW_TSUB_BWD, EW_WAVES_BWD, 2);
    if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
    return ew_run(ew_two_launch(p, B, T, D, 4), linear_bwd_kernel<V, EW_TSUB_BWD, EW_WAVES_BWD>,
                  linear_bwd_kernel<V, EW_TSUB_BWD, EW_WAVES_BWD, EW_REDUCE>,
                  linear_bwd_kernel<V, EW_TSUB_BWD, EW_WAVES_BWD, EW_FINAL>,
                  linear_bwd_kernel<V, EW_TSUB_BWD, EW_WAVES_BWD, EW_AGG>, p, ws, stream, a, b,
                  A, Bc, gA, gB, da, db);
  });
}

size_t mg_signed_gate_scan_workspace_bytes(int64_t B, int64_t T, int64_t D) {
  return gate_ws_bytes(B, T, D);
}

int mg_signed_gate_scan_fwd(const float* s, const float* z, const float* hpre, const float* h0,
                            float* h, int64_t B, int64_t T, int64_t D, int coupled, void* ws,
                            size_t ws_bytes, hipStream_t stream) {
  if (!s || !z || !hpre || !h0 || !h || !ws || !geometry_ok(B, T, D) || (coupled & ~1))
    return MG_ERR_ARG;
  const GateDecay nd{};
  return coupled ? gate_fwd_launch<GATE_SIGNED_COUPLED, false>(s, z, hpre, h0, h, nd, B, T, D, ws,
                                                               ws_bytes, stream)
                 : gate_fwd_launch<GATE_SIGNED, false>(s, z, hpre, h0, h, nd, B, T, D, ws,
                                                       ws_bytes, stream);
}

int mg_signed_gate_scan_bwd(const float* s, const float* z, const float* hpre, const float* h0,
                            const float* h, const float* gh, float* ds, float* dz, float* dhpre,
                            float* dh0, int64_t B, int64_t T, int64_t D, int coupled, void* ws,
                            size_t ws_bytes, hipStream_t stream) {
  if (!s || !z || !hpre || !h0 || !h || !gh || !ds || !dz || !dhpre || !dh0 || !ws ||
      !geometry_ok(B, T, D) || (coupled & ~1))
    return MG_ERR_ARG;
  const GateDecay nd{};
  return coupled ? gate_bwd_launch<GATE_SIGNED_COUPLED, false>(s, z, hpre, h0, h, gh, ds, dz,
                                                               dhpre, dh0, nd, B, T, D, ws,
                                                               ws_bytes, stream)
                 : gate_bwd_launch<GATE_SIGNED, false>(s, z, hpre, h0, h, gh, ds, dz, dhpre, dh0,
                                                       nd, B, T, D, ws, ws_bytes, stream);
}

int mg_signed_gate_scan_decay_fwd(const float* s, const float* z, const float* hpre,
                                  const float* h0, const float* dt, const float* lam, float* h,
                                  int64_t B, int64_t T, int64_t D, int coupled, void* ws,
                                  size_t ws_bytes, hipStream_t stream) {
  if (!s || !z || !hpre || !h0 || !dt || !lam || !h || !ws || !geometry_ok(B, T, D) ||
      (coupled & ~1))
    return MG_ERR_ARG;
  const GateDecay dec{dt, lam, nullptr, nullptr};
  return coupled ? gate_fwd_launch<GATE_SIGNED_COUPLED, true>(s, z, hpre, h0, h, dec, B, T, D, ws,
                                                              ws_bytes, stream)
                 : gate_fwd_launch<GATE_SIGNED, true>(s, z, hpre, h0, h, dec, B, T, D, ws,
                                                      ws_bytes, stream);
}

int mg_signed_gate_scan_decay_bwd(const float* s, const float* z, const float* hpre,
                                  const float* h0, const float* dt, const float* lam,
                                  const float* h, const float* gh, float* ds, float* dz,
                                  float* dhpre, float* dh0, float* dlam, float* ddt, int64_t B,
                                  int64_t T, int64_t D, int coupled, void* ws, size_t ws_bytes,
                                  hipStream_t stream) {
  if (!s || !z || !hpre || !h0 || !dt || !lam || !h || !gh || !ds || !dz || !dhpre || !dh0 ||
      !ws || !geometry_ok(B, T, D) || (coupled & ~1))
    return MG_ERR_ARG;
  const GateDecay dec{dt, lam, dlam, ddt};
  return coupled ? gate_bwd_launch<GATE_SIGNED_COUPLED, true>(s, z, hpre, h0, h, gh, ds, dz,
                                                              dhpre, dh0, dec, B, T, D, ws,
                                                              ws_bytes, stream)
                 : gate_bwd_launch<GATE_SIGNED, true>(s, z, hpre, h0, h, gh, ds, dz, dhpre, dh0,
                                                      dec, B, T, D, ws, ws_bytes, stream);
}

size_t mg_mingru_gate_scan_workspace_bytes(int64_t B, int64_t T, int64_t D) {
  return gate_ws_bytes(B, T, D);
}

int mg_mingru_gate_scan_fwd(const float* k, const float* hpre, const float* log_h0, float* h,
                            int64_t B, int64_t T, int64_t D, void* ws, size_t ws_bytes,
                            hipStream_t stream) {
  if (!k || !hpre || !log_h0 || !h || !ws || !geometry_ok(B, T, D)) return MG_ERR_ARG;
  return gate_fwd_launch<GATE_MINGRU, false>(k, hpre, nullptr, log_h0, h, GateDecay{}, B, T, D,
                                             ws, ws_bytes, stream);
}

int mg_mingru_gate_scan_bwd(const float* k, const float* hpre, const float* log_h0,
                            const float* h, const float* gh, float* dk, float* dhpre,
                            float* dlog_h0, int64_t B, int64_t T, int64_t D, void* ws,
                            size_t ws_bytes, hipStream_t stream) {
  if (!k || !hpre || !log_h0 || !h || !gh || !dk || !dhpre || !dlog_h0 || !ws ||
      !geometry_ok(B, T, D))
    return MG_ERR_ARG;
  return gate_bwd_launch<GATE_MINGRU, false>(k, hpre, nullptr, log_h0, h, gh, dk, dhpre, nullptr,
                                             dlog_h0, GateDecay{}, B, T, D, ws, ws_bytes, stream);
}

int mg_mingru_gate_scan_decay_fwd(const float* k, const float* hpre, const float* log_h0,
                                  const float* dt, const float* lam, float* h, int64_t B,
                                  int64_t T, int64_t D, void* ws, size_t ws_bytes,
                                  hipStream_t stream) {
  if (!k || !hpre || !log_h0 || !dt || !lam || !h || !ws || !geometry_ok(B, T, D))
    return MG_ERR_ARG;
  return gate_fwd_launch<GATE_MINGRU, true>(k, hpre, nullptr, log_h0, h,
                                            GateDecay{dt, lam, nullptr, nullptr}, B, T, D, ws,
                                            ws_bytes, stream);
}

int mg_mingru_gate_scan_decay_bwd(const float* k, const float* hpre, const float* log_h0,
                                  const float* dt, const float* lam, const float* h,
                                  const float* gh, float* dk, float* dhpre, float* dlog_h0,
                                  float* dlam, float* ddt, int64_t B, int64_t T, int64_t D,
                                  void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!k || !hpre || !log_h0 || !dt || !lam || !h || !gh || !dk || !dhpre || !dlog_h0 || !ws ||
      !geometry_ok(B, T, D))
    return MG_ERR_ARG;
  return gate_bwd_launch<GATE_MINGRU, true>(k, hpre, nullptr, log_h0, h, gh, dk, dhpre, nullptr,
                                            dlog_h0, GateDecay{dt, lam, dlam, ddt}, B, T, D, ws,
                                            ws_bytes, stream);
}

int64_t mg_gate_decay_dlam_rows(int64_t B, int64_t T, int64_t D) {
  if (B <= 0 || T <= 0 || D <= 0) return 0;
  return B * ((T + GATE_WAVES_BWD * GATE_TSUB_BWD - 1) / (GATE_WAVES_BWD * GATE_TSUB_BWD));
}

int64_t mg_gate_decay_ddt_rows(int64_t B, int64_t T, int64_t D) {
  if (B <= 0 || T <= 0 || D <= 0) return 0;
  return (D + MG_WAVE - 1) / MG_WAVE;
}

int mg_log_scan_fwd(const float* lc, const float* lv, float* h, float* hstate, int64_t B,
                    int64_t T, int64_t D, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!lc || !lv || !h || !ws || !geometry_ok(B, T, D)) return MG_ERR_ARG;
  const int vec = log_vec(B, T, D, {lc, lv, h, hstate});
  auto run = [&](auto v) {
    constexpr int V = decltype(v)::value;
    EwPlan p = ew_plan(B, T, D, V, LOG_TSUB, LOG_WAVES, 3);
    if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
    return ew_run(ew_two_launch(p, B, T, D, 2), log_fwd_kernel<V, LOG_WAVES>,
                  log_fwd_kernel<V, LOG_WAVES, EW_REDUCE>, log_fwd_kernel<V, LOG_WAVES, EW_FINAL>,
                  log_fwd_kernel<V, LOG_WAVES, EW_AGG>,
                  p, ws, stream, lc, lv, h, hstate);
  };
  return vec == 2 ? run(std::integral_constant<int, 2>{}) : run(std::integral_constant<int, 1>{});
}

int mg_log_scan_bwd(const float* lc, const float* lv, const float* h, const float* hstate,
                    const float* gh, float* dlc, float* dlv, int64_t B, int64_t T, int64_t D,
                    void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!lc || !lv || !h || !gh || !dlc || !dlv || !ws || !geometry_ok(B, T, D)) return MG_ERR_ARG;
  const int vec = log_vec(B, T, D, {lc, lv, h, hstate, gh, dlc, dlv});
  auto run = [&](auto v) {
    constexpr int V = decltype(v)::value;
    EwPlan p = ew_plan(B, T, D, V, LOG_TSUB, LOG_WAVES, 3);
    if (ws_bytes < p.total) return MG_ERR_WORKSPACE;
    return ew_run(ew_two_launch(p, B, T, D, 3), log_bwd_kernel<V, LOG_WAVES>,
                  log_bwd_kernel<V, LOG_WAVES, EW_REDUCE>, log_bwd_kernel<V, LOG_WAVES, EW_FINAL>,
                  log_bwd_kernel<V, LOG_WAVES, EW_AGG>,
                  p, ws, stream, lc, lv, h, hstate, gh, dlc, dlv);
  };
  return vec == 2 ? run(std::integral_constant<int, 2>{}) : run(std::integral_constant<int, 1>{});
}

}  // extern "C"

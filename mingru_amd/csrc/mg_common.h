// Shared device helpers for the mingru_amd HIP kernels (gfx950, wave64).
//
// Decoupled look-back across workgroups
// -------------------------------------
// The scans split the time axis into chunks processed by independent
// workgroups.  A workgroup takes a ticket from a global counter, so tickets
// follow dispatch order; the ticket -> (lane group, chunk) map keeps chunk
// order monotone in ticket order within each lane group.  Every predecessor
// of a workgroup therefore already runs, and it publishes its local
// aggregate before it waits on anything, so the look-back always terminates.
// Each spin is still bounded (MG_SPIN_LIMIT polls); on overflow the kernel
// records an error in the workspace header and carries on instead of hanging.
//
// Published values are self-validating 64-bit words {fp32 value, tag}
// written and read with relaxed agent-scope atomics (single-copy atomic,
// coherent across XCDs without any cache-wide maintenance).  A reader uses a
// word only once its tag equals the current launch's epoch, so no
// release/acquire fences -- which on gfx950 write back / invalidate the whole
// L2 of an XCD -- are needed.
//
// Workspace protocol (no per-launch clearing)
// -------------------------------------------
// The workspace is zero-filled once by its owner and then reused, unchanged,
// by launches that are ordered on one stream.  Header words (first 256 bytes):
//   [MG_H_TICKET0], [MG_H_TICKET1]  ticket counters, used by alternate epochs
//   [MG_H_ERROR]                    spin-limit overflows (diagnostic)
//   [MG_H_EPOCH]                    epoch of the last completed launch
//   [4], [5]                        one 64-bit {count, epoch} word of the
//                                   elementwise scans' one-launch aggregate form
//                                   (scan_elementwise.hip, EW_AGG)
// Every workgroup reads the epoch (previous + 1, never 0 on a zeroed
// workspace), takes its ticket from the counter of the epoch's parity, and the
// workgroup holding ticket 0 resets the other counter for the next launch.
// The workgroup holding the last ticket publishes the new epoch.  Slots of earlier
// launches carry older tags and never validate, so stale contents are
// harmless.  The epoch lives on the device, so graph replays advance it too.
// Launches that may overlap (different streams) need different workspaces.
// The elementwise scans, the thread-per-plane block-matrix backward and its
// forward for small held inputs run the persistent form (mg_persistent's
// protocol): resident workgroups take tickets until the work runs out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#define MG_WAVE 64
#define MG_HEADER_BYTES 256
#define MG_SPIN_LIMIT (1u << 22)

// Status codes returned by every extern "C" entry point.
#define MG_OK 0
#define MG_ERR_ARG 1
#define MG_ERR_LAUNCH 2
#define MG_ERR_WORKSPACE 3
#define MG_ERR_TOO_LARGE 4  // problem needs more than a fixed static scratch holds
#define MG_ERR_RUNTIME 5    // a HIP runtime call (not a launch) failed
#define MG_ERR_CAPTURE 6    // a one-time device set-up was asked for under stream capture

typedef unsigned long long mg_slot_t;

enum : int { MG_H_TICKET0 = 0, MG_H_TICKET1 = 1, MG_H_ERROR = 2, MG_H_EPOCH = 3 };

__device__ __forceinline__ void mg_count_error(unsigned* header) {
  __hip_atomic_fetch_add(header + MG_H_ERROR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A value every lane of the wave holds (an LDS word all lanes read, a wave index),
// marked as such: the compiler keeps it and what is derived from it in scalar
// registers.
__device__ __forceinline__ unsigned mg_uniform(unsigned x) {
  return (unsigned)__builtin_amdgcn_readfirstlane((int)x);
}

struct MgTicket {
  unsigned ticket;  // dispatch-ordered index of this workgroup within the launch
  unsigned epoch;   // tag of every slot this launch publishes
};

// Workspace protocol entry for a 1-D grid; see the header comment.  The ticket
// counter's address depends on the loaded epoch, so every ticket is taken only
// after its workgroup has read the epoch; the holder of the last ticket can
// therefore publish the next epoch without racing any reader of this launch.
__device__ __forceinline__ MgTicket mg_take_ticket(unsigned* header) {
  __shared__ unsigned s_ticket, s_epoch;
  if (threadIdx.x == 0) {
    const unsigned e =
        __hip_atomic_load(header + MG_H_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const unsigned t = __hip_atomic_fetch_add(header + MG_H_TICKET0 + (e & 1u), 1u,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == 0u)  // the previous launch, which used the other counter, has completed
      __hip_atomic_store(header + MG_H_TICKET0 + ((e + 1u) & 1u), 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (t == gridDim.x - 1u)
      __hip_atomic_store(header + MG_H_EPOCH, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // A ticket beyond the grid can only come from a workspace that broke the
    // protocol (not zero-filled, or shared by overlapping launches): record it;
    // the caller retires the workgroup instead of indexing past its slots.
    if (t >= gridDim.x) mg_count_error(header);
    s_ticket = t;
    s_epoch = e;
  }
  __syncthreads();
  return MgTicket{s_ticket, s_epoch};
}

// Persistent form of the protocol: a 1-D grid of at most as many workgroups as
// the chip holds at once, and `chunks` tickets of work.  Thread 0 of every
// workgroup reads the epoch once, then takes tickets from that epoch's counter
// until one lies past the work; so each workgroup ends on exactly one such ticket
// and a launch hands out chunks + gridDim.x tickets in all.  The holder of the
// final one -- taken after every workgroup has read the epoch -- publishes the new
// epoch, and the holder of ticket 0 resets the other counter, as above.  A ticket
// past the final one can only come from a workspace that broke the protocol: it
// is counted as an error and, lying past the work, ends its workgroup.
__device__ __forceinline__ unsigned mg_next_ticket(unsigned* header, unsigned epoch,
                                                   unsigned chunks) {
  const unsigned t = __hip_atomic_fetch_add(header + MG_H_TICKET0 + (epoch & 1u), 1u,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (t == 0u)  // the previous launch, which used the other counter, has completed
    __hip_atomic_store(header + MG_H_TICKET0 + ((epoch + 1u) & 1u), 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const unsigned last = chunks + gridDim.x - 1u;
  if (t == last)
    __hip_atomic_store(header + MG_H_EPOCH, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else if (t > last)
    mg_count_error(header);
  return t;
}

// Runs body(ticket, epoch) over this workgroup's tickets below `chunks`.  The next
// ticket's atomic is issued before the current body, so its round trip overlaps
// the body's work instead of delaying the next chunk's first loads.  Tickets stay
// monotone in time, so every predecessor of a chunk is held by a running
// workgroup, as in the one-ticket form.
// UNIFORM marks the ticket and epoch, which every lane reads from the same LDS
// words, as wave-uniform (mg_uniform), so that what the body derives from them
// (chunk, lane group, row bases) stays in scalar registers.  It is a per-kernel
// choice: it frees vector registers where a kernel is at the cap (the linear
// backward: 38 spilled registers -> 5), and it was slower by 1-2% in kernels that
// are not.
template <bool UNIFORM = false, typename Body>
__device__ __forceinline__ void mg_persistent(unsigned* header, unsigned chunks, Body&& body) {
  __shared__ unsigned s_ticket, s_epoch;
  if (threadIdx.x == 0) {
    const unsigned e =
        __hip_atomic_load(header + MG_H_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    s_ticket = mg_next_ticket(header, e, chunks);
    s_epoch = e;
  }
  __syncthreads();
  unsigned t = UNIFORM ? mg_uniform(s_ticket) : s_ticket;
  const unsigned e = UNIFORM ? mg_uniform(s_epoch) : s_epoch;
  while (t < chunks) {
    unsigned next = 0u;
    if (threadIdx.x == 0) next = mg_next_ticket(header, e, chunks);
    body(t, e);
    __syncthreads();  // every thread has read s_ticket and finished the body
    if (threadIdx.x == 0) s_ticket = next;
    __syncthreads();
    t = UNIFORM ? mg_uniform(s_ticket) : s_ticket;
  }
}

// Workgroups of kernel `k` (blocks of `threads`) the current device holds at once,
// the grid of a persistent launch.  Cached per (kernel, device, block) in a fixed
// table: no allocation, so allocation-free entry points may call it.
inline unsigned mg_resident(const void* k, int threads) {
  struct Entry {
    const void* k;
    int dev, threads;
    unsigned n;
  };
  constexpr int CAP = 256;
  static Entry cache[CAP];
  static int used = 0;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].k == k && cache[i].dev == dev && cache[i].threads == threads) return cache[i].n;
  int per = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, threads, 0) != hipSuccess || per < 1)
    per = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 1;
  const unsigned n = (unsigned)per * (unsigned)cus;
  if (used < CAP) cache[used++] = Entry{k, dev, threads, n};
  return n;
}

__device__ __forceinline__ void mg_slot_put(mg_slot_t* p, float v, unsigned epoch) {
  const mg_slot_t w = ((mg_slot_t)epoch << 32) | (mg_slot_t)__float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true and the value if the slot has been published in this epoch.
__device__ __forceinline__ bool mg_slot_get(const mg_slot_t* p, float& v, unsigned epoch) {
  const mg_slot_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v = __uint_as_float((unsigned)(w & 0xffffffffull));
  return (unsigned)(w >> 32) == epoch;
}

// Streaming (non-temporal) global accesses for data read or written exactly
// once: the hint keeps single-use lines from displacing the look-back slots
// and the other streams in the caches, which raises sustained HBM bandwidth
// (a 2-in/2-out stream measured 5.5 -> 6.2 TB/s on MI355X).  Use the streaming
// stores only where one store instruction of a wave covers whole contiguous
// lines (consecutive lanes, consecutive vectors): partial-line streaming stores
// are not merged in L2 and cost several times their size.
typedef float mg_v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 mg_ld_stream4(const float* p) {
  const mg_v4f v = __builtin_nontemporal_load(reinterpret_cast<const mg_v4f*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void mg_st_stream4(float* p, float4 x) {
  const mg_v4f v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<mg_v4f*>(p));
}
typedef float mg_v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float2 mg_ld_stream2(const float* p) {
  const mg_v2f v = __builtin_nontemporal_load(reinterpret_cast<const mg_v2f*>(p));
  return make_float2(v.x, v.y);
}
__device__ __forceinline__ void mg_st_stream2(float* p, float2 x) {
  const mg_v2f v = {x.x, x.y};
  __builtin_nontemporal_store(v, reinterpret_cast<mg_v2f*>(p));
}
__device__ __forceinline__ float mg_ld_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void mg_st_stream(float* p, float x) { __builtin_nontemporal_store(x, p); }

static inline size_t mg_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// x of the lane N places further along this lane's DPP row of 16 lanes, cyclically
// (DPP row_ror:N, a VALU operand modifier: no LDS crossbar round trip).
template <int N>
__device__ __forceinline__ float mg_row_ror(float x) {
  static_assert(N >= 1 && N <= 15, "row_ror takes 1..15");
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// x + x of lane ^ 16 (S = 16) or lane ^ 32 (S = 32), in every lane, by gfx950's
// v_permlane16_swap / v_permlane32_swap of x with itself: one copy ends up with the
// lower rows (halves) of each pair, the other with the upper ones, so their sum is
// the pair's sum in every lane, whichever copy the builtin returns first.
template <int S>
__device__ __forceinline__ float mg_pair_sum(float x) {
  static_assert(S == 16 || S == 32, "row pairs (16) or wave halves (32)");
  const unsigned u = __float_as_uint(x);
  if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Sum of x over each group of N consecutive lanes (N = 16, 32 or 64), in every lane
// of the group; the whole wave must be active.  Rotations by 8, 4, 2, 1 within a
// row leave every lane of it the row's total; wider groups add the other rows'
// totals by lane swaps.  No LDS crossbar is used, and the association is fixed, so
// results are reproducible.
template <int N>
__device__ __forceinline__ float mg_group_sum(float x) {
  static_assert(N == 16 || N == 32 || N == 64, "groups of 16, 32 or 64 lanes");
  x += mg_row_ror<8>(x);
  x += mg_row_ror<4>(x);
  x += mg_row_ror<2>(x);
  x += mg_row_ror<1>(x);
  if constexpr (N >= 32) x = mg_pair_sum<16>(x);
  if constexpr (N >= 64) x = mg_pair_sum<32>(x);
  return x;
}

// DPP move with the lanes whose source lies outside the pattern's range receiving 0.
template <int CTRL>
__device__ __forceinline__ float mg_dpp0(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Inclusive prefix (lane l: x[0] + ... + x[l]) and suffix (x[l] + ... + x[63]) sums
// over the wave without the LDS crossbar: Hillis-Steele steps of 1, 2, 4 and 8 lanes
// within each 16-lane row (DPP row_shr / row_shl), then the other rows' totals read
// with v_readlane.  Each lane's sum holds only its own range's terms (no difference of
// running sums).  The whole wave must be active.
__device__ __forceinline__ float mg_wave_prefix_sum(float x) {
  x += mg_dpp0<0x111>(x);  // row_shr:1
  x += mg_dpp0<0x112>(x);
  x += mg_dpp0<0x114>(x);
  x += mg_dpp0<0x118>(x);
  const int row = (threadIdx.x & (MG_WAVE - 1)) >> 4;
  const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 15));
  const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 31));
  const float t2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 47));
  return x + ((row > 0 ? t0 : 0.f) + ((row > 1 ? t1 : 0.f) + (row > 2 ? t2 : 0.f)));
}
__device__ __forceinline__ float mg_wave_suffix_sum(float x) {
  x += mg_dpp0<0x101>(x);  // row_shl:1
  x += mg_dpp0<0x102>(x);
  x += mg_dpp0<0x104>(x);
  x += mg_dpp0<0x108>(x);
  const int row = (threadIdx.x & (MG_WAVE - 1)) >> 4;
  const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float t2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float t3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return x + ((row < 1 ? t1 : 0.f) + ((row < 2 ? t2 : 0.f) + (row < 3 ? t3 : 0.f)));
}
// x of lane l + 1 (0 in lane 63) and of lane l - 1 (0 in lane 0): DPP wave_shl / wave_shr.
__device__ __forceinline__ float mg_wave_next(float x) { return mg_dpp0<0x130>(x); }
__device__ __forceinline__ float mg_wave_prev(float x) { return mg_dpp0<0x138>(x); }

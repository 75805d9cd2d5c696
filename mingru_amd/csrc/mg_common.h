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
// word only once its tag is non-zero, so no release/acquire fences -- which on
// gfx950 write back / invalidate the whole L2 of an XCD -- are needed.
//
// Workspace header (first 256 bytes of every workspace):
//   word 0: ticket counter, word 1: error counter (spin-limit overflows).
// The host clears the header and every look-back slot with mg_clear_kernel
// before each scan launch, so the caller may pass uninitialised memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MG_WAVE 64
#define MG_HEADER_BYTES 256
#define MG_SPIN_LIMIT (1u << 22)

// Status codes returned by every extern "C" entry point.
#define MG_OK 0
#define MG_ERR_ARG 1
#define MG_ERR_LAUNCH 2
#define MG_ERR_WORKSPACE 3

typedef unsigned long long mg_slot_t;

__device__ __forceinline__ unsigned mg_take_ticket(unsigned* header) {
  __shared__ unsigned s_ticket;
  if (threadIdx.x == 0) {
    s_ticket = __hip_atomic_fetch_add(header, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return s_ticket;
}

__device__ __forceinline__ void mg_slot_put(mg_slot_t* p, float v) {
  const mg_slot_t w = (1ull << 32) | (mg_slot_t)__float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true and the value if the slot has been published.
__device__ __forceinline__ bool mg_slot_get(const mg_slot_t* p, float& v) {
  const mg_slot_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v = __uint_as_float((unsigned)(w & 0xffffffffull));
  return (w >> 32) != 0ull;
}

__device__ __forceinline__ void mg_count_error(unsigned* header) {
  __hip_atomic_fetch_add(header + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Streaming (non-temporal) global accesses for data read or written exactly
// once: the hint keeps single-use lines from displacing the look-back slots
// and the other streams in the caches, which raises sustained HBM bandwidth
// (a 2-in/2-out stream measured 5.5 -> 6.2 TB/s on MI355X).
typedef float mg_v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 mg_ld_stream4(const float* p) {
  const mg_v4f v = __builtin_nontemporal_load(reinterpret_cast<const mg_v4f*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void mg_st_stream4(float* p, float4 x) {
  const mg_v4f v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<mg_v4f*>(p));
}
__device__ __forceinline__ float mg_ld_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void mg_st_stream(float* p, float x) { __builtin_nontemporal_store(x, p); }

// Zeroes `n16` 16-byte units (workspace header and look-back slots).
__global__ void mg_clear_kernel(uint4* p, size_t n16);

static inline size_t mg_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

static inline int mg_clear(void* ws, size_t bytes, hipStream_t stream) {
  const size_t n16 = (bytes + 15) / 16;
  const int threads = 256;
  size_t blocks = (n16 + threads - 1) / threads;
  if (blocks == 0) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(mg_clear_kernel, dim3((unsigned)blocks), dim3(threads), 0, stream,
                     (uint4*)ws, n16);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

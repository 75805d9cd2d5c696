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
// records an error in the workspace header and carries on with an identity
// carry instead of hanging.
//
// Workspace header (first 256 bytes of every workspace):
//   word 0: ticket counter, word 1: error counter (spin-limit overflows).
// The host clears the header and the flag array with mg_clear_kernel before
// each scan launch, so the caller may pass uninitialised memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MG_WAVE 64
#define MG_HEADER_BYTES 256
#define MG_SPIN_LIMIT (1u << 22)

enum : unsigned { MG_FLAG_NONE = 0u, MG_FLAG_AGG = 1u, MG_FLAG_INCL = 2u };

// Status codes returned by every extern "C" entry point.
#define MG_OK 0
#define MG_ERR_ARG 1
#define MG_ERR_LAUNCH 2
#define MG_ERR_WORKSPACE 3

__device__ __forceinline__ unsigned mg_take_ticket(unsigned* header) {
  __shared__ unsigned s_ticket;
  if (threadIdx.x == 0) {
    s_ticket = __hip_atomic_fetch_add(header, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return s_ticket;
}

// Release: called by the publishing wave after its data stores.
__device__ __forceinline__ void mg_publish_flag(unsigned* flag, unsigned value) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if ((threadIdx.x & (MG_WAVE - 1)) == 0) {
    __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Acquire: poll until the flag is non-zero or the spin limit is reached.
// Returns the flag value (MG_FLAG_NONE on overflow, after counting an error).
__device__ __forceinline__ unsigned mg_wait_flag(const unsigned* flag, unsigned* header) {
  unsigned v = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned spins = 0;
  while (v == MG_FLAG_NONE) {
    __builtin_amdgcn_s_sleep(1);
    v = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (++spins >= MG_SPIN_LIMIT) {
      if ((threadIdx.x & (MG_WAVE - 1)) == 0) {
        __hip_atomic_fetch_add(header + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return MG_FLAG_NONE;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return v;
}

// Clears n 32-bit words (the workspace header and flag array).
__global__ void mg_clear_kernel(unsigned* p, size_t n);

static inline size_t mg_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

static inline int mg_clear(void* ws, size_t words, hipStream_t stream) {
  const int threads = 256;
  size_t blocks = (words + threads - 1) / threads;
  if (blocks == 0) blocks = 1;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(mg_clear_kernel, dim3((unsigned)blocks), dim3(threads), 0, stream,
                     (unsigned*)ws, words);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

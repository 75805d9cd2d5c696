// DeltaMinGRU bf16 backward preparation kernel (both forms), in a translation
// unit of its own.  Instantiated beside the gradient kernel, it changed the
// compiler's register allocation of the ungated gradient kernel: 12 spilled
// registers instead of 5, 337 against 311 us at C5.
#include "mg_delta_bf16.h"

namespace mgd {

int dwb_bwd_prep_launch(bool gated, const void* Q, const void* K, const void* V, const void* beta,
                        const float* lg, const void* dy, const float* Hb, float* Um, float* Em,
                        float* G0m, float* Apm, float* bpm, float* vm, int64_t BH,
                        const DwGeom& g, hipStream_t stream) {
  const dim3 pgrid(g.nc, (unsigned)BH);
  const u16 *q = (const u16*)Q, *k = (const u16*)K, *v = (const u16*)V, *b = (const u16*)beta,
            *d = (const u16*)dy;
  const float* Tin = dw_inv_slots(Hb, BH, g);
  if (gated)
    hipLaunchKernelGGL(dwb_bwd_prep<true>, pgrid, dim3(NTB), 0, stream, q, k, v, b, lg, d, Hb, Tin,
                       Um, Em, G0m, Apm, bpm, vm, g);
  else
    hipLaunchKernelGGL(dwb_bwd_prep<false>, pgrid, dim3(NTB), 0, stream, q, k, v, b, nullptr, d,
                       Hb, Tin, Um, Em, G0m, Apm, bpm, nullptr, g);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

}  // namespace mgd

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
#include "mg_delta_bf16.h"

namespace mgd {

int dw_fwd_bf16(const void* Q, const void* K, const void* V, const void* beta, const float* H0,
                void* y, float* HT, float* Hb, int64_t BH, const DwGeom& g, void* ws,
                size_t ws_bytes, hipStream_t stream) {
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 4 * mb) return MG_ERR_WORKSPACE;
  float* Am = (float*)ws;  // split pair
  float* Bm = (float*)((char*)ws + mb);
  float* Qem = (float*)((char*)ws + 2 * mb);  // split pair
  float* Pum = (float*)((char*)ws + 3 * mb);
  hipLaunchKernelGGL(dwb_fwd_prep<false>, dim3(g.nc, (unsigned)BH), dim3(NTB), 0, stream,
                     (const u16*)Q, (const u16*)K, (const u16*)V, (const u16*)beta, nullptr, Am,
                     Bm, Qem, Pum, nullptr, dw_inv_slots(Hb, BH, g), g);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dwb_fwd_chain<false>, dim3(chain_grid(BH, g)), dim3(NT), 0, stream, H0, Am,
                     Bm, Qem, Pum, nullptr, (u16*)y, HT, Hb, g, BH);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

int dw_bwd_bf16(const void* Q, const void* K, const void* V, const void* beta, const float* Hb,
                const void* dy, const float* dHT, void* dQ, void* dK, void* dV, void* dbeta,
                float* dH0, int64_t BH, const DwGeom& g, void* ws, size_t ws_bytes,
                hipStream_t stream) {
  const size_t mb = dw_mat_bytes(BH, g);
  if (ws_bytes < 6 * mb) return MG_ERR_WORKSPACE;
  float* Um = (float*)ws;
  float* Em = (float*)((char*)ws + mb);  // split pair
  float* G0m = (float*)((char*)ws + 2 * mb);
  float* Apm = (float*)((char*)ws + 3 * mb);  // split pair
  float* bpm = (float*)((char*)ws + 4 * mb);
  float* dHn = (float*)((char*)ws + 5 * mb);
  const dim3 pgrid(g.nc, (unsigned)BH);
  const u16 *q = (const u16*)Q, *k = (const u16*)K, *b = (const u16*)beta, *d = (const u16*)dy;
  const int rc = dwb_bwd_prep_launch(false, Q, K, V, beta, nullptr, dy, Hb, Um, Em, G0m, Apm, bpm,
                                     nullptr, BH, g, stream);
  if (rc != MG_OK) return rc;
  hipLaunchKernelGGL(dwb_bwd_chain<false>, dim3(chain_grid(BH, g)), dim3(NT), 0, stream, dHT, Apm,
                     bpm, nullptr, dHn, dH0, g, BH);
  if (hipGetLastError() != hipSuccess) return MG_ERR_LAUNCH;
  hipLaunchKernelGGL(dwb_bwd_grads<false>, pgrid, dim3(NTB), 0, stream, q, k, b, nullptr, d, Hb, dHn,
                     Um, Em, G0m, (u16*)dQ, (u16*)dK, (u16*)dV, (u16*)dbeta, nullptr, g);
  return hipGetLastError() == hipSuccess ? MG_OK : MG_ERR_LAUNCH;
}

}  // namespace mgd

/*
 * mingru_hip.h -- C ABI of libmingru_hip.so, the MI355X (gfx950) kernels behind
 * the MINGRU_SCAN seam of mingru_amd.
 *
 * Conventions (every entry point):
 *   - pointers are device pointers to contiguous row-major fp32 (bf16 where
 *     stated) tensors; sizes are int64 element counts;
 *   - `ws`/`ws_bytes` is a caller-provided device workspace of at least the
 *     size returned by the matching *_workspace_bytes query.
 *     Look-back scan entry points (linear, log, affine): the workspace must be
 *     zero-filled once before its first use and may then be passed, unchanged,
 *     to any sequence of scan calls ordered on one stream (of any op or size up
 *     to its capacity); nothing is cleared between calls, because each launch
 *     tags its look-back slots with a fresh epoch kept in the workspace header.
 *     Calls that can run concurrently (different streams) need different
 *     workspaces.  Angle and delta entry points: contents on entry are
 *     irrelevant;
 *   - work is enqueued asynchronously on `stream`; nothing allocates, throws or
 *     synchronises;
 *   - the return value is a status: 0 ok, 1 invalid argument / outside the
 *     envelope, 2 kernel launch failed, 3 workspace too small, 4 problem too
 *     large for a fixed static scratch, 5 a HIP runtime call failed, 6 a
 *     one-time device set-up was asked for while `stream` was being captured.
 *
 * Each declaration cites the reference interface it replaces
 * (chris-santiago/minGRU, paths relative to the repository root).
 */
#ifndef MINGRU_HIP_H
#define MINGRU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mg_stream_t; /* == hipStream_t */

/* ---- linear_scan: h_t = a_t h_{t-1} + b_t, (B, T, D) ------------------------
 * Replaces linear_scan_fwd / linear_scan_bwd
 * (src/mingru/triton_scans.py:1318-1334, 1392-1417; kernels :703-751, :962-1036)
 * behind SCAN_IMPLS["linear_scan"] (src/mingru/triton_scans.py:2449-2465). */
size_t mg_linear_scan_workspace_bytes(int64_t B, int64_t T, int64_t D);
/* a, b -> A (running product), Bc (zero-start solution). */
int mg_linear_scan_fwd(const float* a, const float* b, float* A, float* Bc, int64_t B, int64_t T,
                       int64_t D, void* ws, size_t ws_bytes, mg_stream_t stream);
/* Grads gA, gB of (A, Bc) -> da, db.  A, Bc are the forward outputs; the kernels
 * read Bc and the row of A before each sub-chunk, not b (kept for the interface). */
int mg_linear_scan_bwd(const float* a, const float* b, const float* A, const float* Bc,
                       const float* gA, const float* gB, float* da, float* db, int64_t B,
                       int64_t T, int64_t D, void* ws, size_t ws_bytes, mg_stream_t stream);

/* Allocation-free variant of mg_linear_scan_fwd.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * look-back workspace is a static device array of MG_NOALLOC_SCRATCH_BYTES per
 * GPU, held from the library's first call on that GPU until the process ends
 * and zero-filled once by that call (on `stream`).  That first call on a GPU
 * must not be made under stream capture (it returns 6 and does nothing); later
 * calls may be captured.  Problems whose forward workspace exceeds the array
 * (about B*T*D > 2^27 elements) return MG_ERR_TOO_LARGE (4) without touching
 * the device.  Every call on one GPU shares the array: calls must be ordered on
 * one stream; calls that can overlap on one GPU race.  Allocates nothing, never
 * synchronises. */
#define MG_NOALLOC_SCRATCH_BYTES (64u << 20)
int mg_linear_scan_fwd_noalloc(const float* a, const float* b, float* A, float* Bc, int64_t B,
                               int64_t T, int64_t D, mg_stream_t stream);
/* Failed look-back waits recorded by mg_linear_scan_fwd_noalloc on the current
 * GPU since its static array was zeroed (as mg_scan_workspace_errors reports for
 * a caller workspace); 0 when the entry point has not run on this GPU.  No
 * counterpart in the reference.  Synchronises `stream`, allocates nothing. */
int mg_linear_scan_noalloc_errors(unsigned* count, mg_stream_t stream);

/* ---- fused SignedMinGRU gates + linear_scan, (B, T, D) -----------------------
 * No reference kernel fuses these: replaces the mixer's coefficient code and
 * its scan call (SignedMinGRU._coeffs / forward, src/mingru/min_gru.py:1788-1857):
 * a = tanh(s) (times 1 - sigmoid(z) when `coupled`), b = sigmoid(z) * hpre,
 * h = A * h0 + Bc with (A, Bc) = linear_scan(a, b).  One pass reads the three
 * pre-activations and writes h; h0 / dh0 are (B, D).  Workspace as for
 * linear_scan (its own size query). */
size_t mg_signed_gate_scan_workspace_bytes(int64_t B, int64_t T, int64_t D);
int mg_signed_gate_scan_fwd(const float* s, const float* z, const float* hpre, const float* h0,
                            float* h, int64_t B, int64_t T, int64_t D, int coupled, void* ws,
                            size_t ws_bytes, mg_stream_t stream);
/* h = forward output, gh = dL/dh -> ds, dz, dhpre (B,T,D) and dh0 (B,D). */
int mg_signed_gate_scan_bwd(const float* s, const float* z, const float* hpre, const float* h0,
                            const float* h, const float* gh, float* ds, float* dz, float* dhpre,
                            float* dh0, int64_t B, int64_t T, int64_t D, int coupled, void* ws,
                            size_t ws_bytes, mg_stream_t stream);

/* ---- time decay of the fused gate scans ---------------------------------------------
 * No reference kernel: the decay-active forms of the two fused gate scans, replacing
 * the mixers' eager decay (DecayMixin._decay_gamma folded into a,
 * src/mingru/min_gru.py:1807-1813 for SignedMinGRU, and MinGRU's log coefficient
 * minus lam dt, :1383-1393).  The coefficient a is multiplied by
 * gamma = exp(-lam[d] dt[b, t]) in the kernel: dt (B, T) is the normalised delta_t,
 * lam (D) the per-channel rate (a fixed rate repeated).  The backward also writes,
 * where the pointer is not NULL, row-wise partial sums of
 *   dlam: mg_gate_decay_dlam_rows(B, T, D) rows of D floats (dL/dlam = their sum),
 *   ddt:  mg_gate_decay_ddt_rows(B, T, D) rows of B*T floats (dL/ddt = their sum);
 * every row is written.  Workspace as the matching undecayed entry point. */
int mg_signed_gate_scan_decay_fwd(const float* s, const float* z, const float* hpre,
                                  const float* h0, const float* dt, const float* lam, float* h,
                                  int64_t B, int64_t T, int64_t D, int coupled, void* ws,
                                  size_t ws_bytes, mg_stream_t stream);
int mg_signed_gate_scan_decay_bwd(const float* s, const float* z, const float* hpre,
                                  const float* h0, const float* dt, const float* lam,
                                  const float* h, const float* gh, float* ds, float* dz,
                                  float* dhpre, float* dh0, float* dlam, float* ddt, int64_t B,
                                  int64_t T, int64_t D, int coupled, void* ws, size_t ws_bytes,
                                  mg_stream_t stream);
int mg_mingru_gate_scan_decay_fwd(const float* k, const float* hpre, const float* log_h0,
                                  const float* dt, const float* lam, float* h, int64_t B,
                                  int64_t T, int64_t D, void* ws, size_t ws_bytes,
                                  mg_stream_t stream);
int mg_mingru_gate_scan_decay_bwd(const float* k, const float* hpre, const float* log_h0,
                                  const float* dt, const float* lam, const float* h,
                                  const float* gh, float* dk, float* dhpre, float* dlog_h0,
                                  float* dlam, float* ddt, int64_t B, int64_t T, int64_t D,
                                  void* ws, size_t ws_bytes, mg_stream_t stream);
int64_t mg_gate_decay_dlam_rows(int64_t B, int64_t T, int64_t D);
int64_t mg_gate_decay_ddt_rows(int64_t B, int64_t T, int64_t D);

/* ---- fused MinGRU gates + parallel_scan_log, (B, T, D) -------------------------
 * No reference kernel fuses these: replaces MinGRU.forward's coefficient code and
 * its scan call (src/mingru/min_gru.py:1366-1397): log(1 - z) = -softplus(k),
 * log z = -softplus(-k), log h~ = log_g(hpre) and
 * h = exp(parallel_scan_log(log(1 - z), [log h0, log z + log h~])).  The kernel
 * runs the same recurrence in linear space (every term is positive):
 * h_t = sigmoid(-k) h_{t-1} + sigmoid(k) g(hpre), h_0 = exp(log_h0).  One pass
 * reads k and hpre and writes h; log_h0 / dlog_h0 are (B, D).  Workspace from its
 * own size query. */
size_t mg_mingru_gate_scan_workspace_bytes(int64_t B, int64_t T, int64_t D);
int mg_mingru_gate_scan_fwd(const float* k, const float* hpre, const float* log_h0, float* h,
                            int64_t B, int64_t T, int64_t D, void* ws, size_t ws_bytes,
                            mg_stream_t stream);
/* h = forward output, gh = dL/dh -> dk, dhpre (B,T,D) and dlog_h0 (B,D). */
int mg_mingru_gate_scan_bwd(const float* k, const float* hpre, const float* log_h0,
                            const float* h, const float* gh, float* dk, float* dhpre,
                            float* dlog_h0, int64_t B, int64_t T, int64_t D, void* ws,
                            size_t ws_bytes, mg_stream_t stream);

/* ---- parallel_scan_log: log-space inputs, (B, T, D) and (B, T+1, D) ---------
 * Replaces parallel_scan_log_fwd (src/mingru/triton_scans.py:1336-1357, kernel
 * :754-821) and its eager-recompute backward (:1489-1552) behind
 * SCAN_IMPLS["parallel_scan_log"] (:2467-2490).  Inputs anywhere in fp32's
 * range: the kernels hold every product and sum as an fp32 significand with a
 * separate exponent, so e^lc, e^lv and the backward's adjoint never overflow or
 * underflow before the result is formed (the reference evaluates in log space,
 * src/mingru/min_gru.py:804-807).  `hstate` (mg_log_scan_state_bytes, fp32)
 * receives extended-range forward states at every 8-step boundary for the
 * backward; it may be NULL in both calls, and the backward then restarts from
 * the fp32 outputs h (exact unless h under- or overflowed). */
size_t mg_log_scan_workspace_bytes(int64_t B, int64_t T, int64_t D);
size_t mg_log_scan_state_bytes(int64_t B, int64_t T, int64_t D);
/* lc = log a (B,T,D), lv = [log h0, log b] (B,T+1,D) -> h (B,T,D) [, hstate]. */
int mg_log_scan_fwd(const float* lc, const float* lv, float* h, float* hstate, int64_t B,
                    int64_t T, int64_t D, void* ws, size_t ws_bytes, mg_stream_t stream);
/* h = forward output, hstate = the forward's record (or NULL), gh = dL/dh
 * -> dlc (B,T,D), dlv (B,T+1,D). */
int mg_log_scan_bwd(const float* lc, const float* lv, const float* h, const float* hstate,
                    const float* gh, float* dlc, float* dlv, int64_t B, int64_t T, int64_t D,
                    void* ws, size_t ws_bytes, mg_stream_t stream);

/* ---- look-back workspace diagnostics ----------------------------------------
 * No reference counterpart (the reference's kernels have no look-back).  Copies
 * the count of failed look-back waits recorded in a linear / log / affine / fused
 * gate scan workspace to *count, after the work queued on `stream`.  Every wait
 * is bounded: a wait that gives up (or a workspace that broke the protocol)
 * increments the count and the kernel finishes with a partial carry, so a
 * nonzero count means results since the workspace was zeroed are not to be
 * trusted.  The one entry point that synchronises (`stream`). */
int mg_scan_workspace_errors(const void* ws, unsigned* count, mg_stream_t stream);

/* ---- matrix_scan / matrix_affine_scan: k x k blocks, (B, T, n, k, k) -------
 * Replaces affine_scan_fwd / affine_scan_bwd (src/mingru/triton_scans.py:
 * 1293-1316, 1359-1390; kernels :630-700, :824-959) behind
 * SCAN_IMPLS["matrix_scan"] / ["matrix_affine_scan"] (:2492-2563).
 * k, v in {1,2,4,8,16} (k <= 4 one plane per thread, k = 8 and 16 on the
 * matrix cores); pointers 16-byte aligned. */
size_t mg_affine_scan_workspace_bytes(int64_t B, int64_t T, int64_t n, int k, int v);
/* A (B,T,n,k,k), Bm (B,T,n,k,v) -> Abar = A_t..A_1, Bbar (zero-start solution). */
int mg_affine_scan_fwd(const float* A, const float* Bm, float* Abar, float* Bbar, int64_t B,
                       int64_t T, int64_t n, int k, int v, void* ws, size_t ws_bytes,
                       mg_stream_t stream);
/* Grads of (Abar, Bbar) -> dA, dBm.  Abar, Bbar are the forward outputs; the kernels
 * read them, not Bm (kept for the interface). */
int mg_affine_scan_bwd(const float* A, const float* Bm, const float* Abar, const float* Bbar,
                       const float* gAbar, const float* gBbar, float* dA, float* dBm, int64_t B,
                       int64_t T, int64_t n, int k, int v, void* ws, size_t ws_bytes,
                       mg_stream_t stream);

/* ---- angle-fused block-rotation scan (RotationMinGRU / GivensMinGRU) --------
 * Replaces angle_scan_fwd / angle_scan_bwd (src/mingru/triton_scans.py:1579-1703;
 * kernels :1039-1291) behind angle_scan_impl (:1743-1812).
 * theta (B,T,n,NA) with NA angles per token, scale/gamma (B,T,n), b/h (B,T,n,k),
 * h0 (B,n,k); k in {2,4,8}.  sched 0: brick-wall rounds (NA = rounds*k/2),
 * sched 1: all pairs i<j in lexicographic order, one plane per round
 * (rounds = k(k-1)/2 = NA).  flags bit 0: scale coordinate 1 by `scale`,
 * bit 1: decay by `gamma`.  The forward writes the per-chunk transition
 * products (and, past 16 chunks of 16 tokens, the products over groups of 8
 * chunks) to `chunk_prod` (mg_angle_scan_state_bytes); the backward reads
 * them.  The workspace's contents on entry are irrelevant (no look-back). */
size_t mg_angle_scan_workspace_bytes(int64_t B, int64_t T, int64_t n, int k);
size_t mg_angle_scan_state_bytes(int64_t B, int64_t T, int64_t n, int k);
int mg_angle_scan_fwd(const float* theta, const float* scale, const float* gamma, const float* b,
                      const float* h0, float* h, float* chunk_prod, int64_t B, int64_t T,
                      int64_t n, int k, int sched, int rounds, int flags, void* ws,
                      size_t ws_bytes, mg_stream_t stream);
/* h = forward output, chunk_prod = the forward's chunk products, gh = dL/dh
 * -> dtheta, dscale, dgamma (written when the flag is set), db, dh0. */
int mg_angle_scan_bwd(const float* theta, const float* scale, const float* gamma, const float* h0,
                      const float* h, const float* chunk_prod, const float* gh, float* dtheta,
                      float* dscale, float* dgamma, float* db, float* dh0, int64_t B, int64_t T,
                      int64_t n, int k, int sched, int rounds, int flags, void* ws,
                      size_t ws_bytes, mg_stream_t stream);

/* ---- angle-fused scan with the mixers' gated prologue (brick-wall schedules) --------
 * No reference kernel fuses these: the same scan as mg_angle_scan_fwd/bwd with
 * sched 0 (brick-wall rounds, k in {2,4,8}), but with the heads of RotationMinGRU /
 * GivensMinGRU formed inside the kernel instead of by eager ops
 * (src/mingru/min_gru.py:2261-2262, 2719): b = sigmoid(z) * hpre from z, hpre
 * (B,T,n,k), and, when flags bit 0 is set, the scale tanh(u) from u (B,T,n).  The
 * backward writes dz, dhpre in place of db and du in place of dscale.  flags: bit 0
 * scale, bit 1 decay (gamma (B,T,n) as in mg_angle_scan_fwd).  State and workspace
 * sizes as mg_angle_scan_state_bytes / mg_angle_scan_workspace_bytes. */
int mg_angle_scan_gated_fwd(const float* theta, const float* u, const float* gamma,
                            const float* z, const float* hpre, const float* h0, float* h,
                            float* chunk_prod, int64_t B, int64_t T, int64_t n, int k, int rounds,
                            int flags, void* ws, size_t ws_bytes, mg_stream_t stream);
int mg_angle_scan_gated_bwd(const float* theta, const float* u, const float* gamma,
                            const float* z, const float* hpre, const float* h0, const float* h,
                            const float* chunk_prod, const float* gh, float* dtheta, float* du,
                            float* dgamma, float* dz, float* dhpre, float* dh0, int64_t B,
                            int64_t T, int64_t n, int k, int rounds, int flags, void* ws,
                            size_t ws_bytes, mg_stream_t stream);

/* ---- angle-fused scan driven by run-time plane tables -------------------------
 * Replaces the same reference kernels as mg_angle_scan_fwd/bwd
 * (src/mingru/triton_scans.py:1039-1291, angle_scan_impl :1743-1812), taking
 * their plane metadata as the reference kernel does: perm/p2p (R,k) int32 and
 * sgn (R,k) fp32 on the device, theta (B,T,n,R,half).  k in {2,4,8,16},
 * half <= 64, R <= 128; the tables must describe disjoint plane rotations (perm
 * an involution, partners sharing an angle that no other plane of the round
 * uses, signs -1/+1; a position whose partner is itself is untouched).  flags as
 * mg_angle_scan_fwd.  The forward writes the per-chunk transition products to
 * `chunk_prod` (mg_angle_scan_tables_state_bytes), which the backward reads;
 * the workspace (mg_angle_scan_tables_workspace_bytes) needs no initialisation.
 * The backward writes dtheta only for angles some plane uses. */
size_t mg_angle_scan_tables_state_bytes(int64_t B, int64_t T, int64_t n, int k);
size_t mg_angle_scan_tables_workspace_bytes(int64_t B, int64_t T, int64_t n, int k);
int mg_angle_scan_tables_fwd(const float* theta, const float* scale, const float* gamma,
                             const float* b, const float* h0, const int* perm, const float* sgn,
                             const int* p2p, float* h, float* chunk_prod, int64_t B, int64_t T,
                             int64_t n, int k, int R, int half, int flags, void* ws,
                             size_t ws_bytes, mg_stream_t stream);
/* h = forward output, chunk_prod = the forward's chunk products, gh = dL/dh
 * -> dtheta, dscale, dgamma (when flagged), db, dh0. */
int mg_angle_scan_tables_bwd(const float* theta, const float* scale, const float* gamma,
                             const float* h0, const float* h, const float* chunk_prod,
                             const float* gh, const int* perm, const float* sgn, const int* p2p,
                             float* dtheta, float* dscale, float* dgamma, float* db, float* dh0,
                             int64_t B, int64_t T, int64_t n, int k, int R, int half, int flags,
                             void* ws, size_t ws_bytes, mg_stream_t stream);

/* ---- DeltaMinGRU chunked-WY delta rule ----------------------------------------
 * Replaces the reference's three forward kernels (_delta_prepass_kernel,
 * _delta_state_kernel, _delta_readout_kernel, src/mingru/triton_scans.py:
 * 1859-2193, launched by _delta_forward_launch :2195-2322) and its torch
 * backward (_delta_backward_torch :473-605, wired by _DeltaScanFn :2324-2401)
 * behind delta_scan_impl (:2403-2447).
 * Layouts: Q (B,H,T,dk), K (B,H,T,nh,dk), V (B,H,T,nh,dv), beta (B,H,T,nh),
 * y (B,H,T,dv), all of element type `dtype` (0 = fp32, 1 = bf16);
 * H0 / HT / dHT / dH0 (B,H,dk,dv) fp32.  Envelope: 1 <= dk, dv <= 64,
 * chunk >= 1, nh * chunk <= 64.
 * `Hbound` (mg_delta_state_bytes) receives the chunk-entry states and each chunk's
 * inverse (I + L)^-1 in a layout private to the library (it differs between dtypes)
 * and is read back only by mg_delta_bwd with the same shape and dtype; `ws` needs
 * mg_delta_workspace_bytes. */
size_t mg_delta_workspace_bytes(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv,
                                int chunk);
size_t mg_delta_state_bytes(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv, int chunk);
int mg_delta_fwd(const void* Q, const void* K, const void* V, const void* beta, const float* H0,
                 void* y, float* HT, float* Hbound, int64_t B, int64_t H, int64_t T, int nh,
                 int dk, int dv, int chunk, int dtype, void* ws, size_t ws_bytes,
                 mg_stream_t stream);
/* dy (dtype), dHT -> dQ, dK, dV, dbeta (dtype) and dH0. */
int mg_delta_bwd(const void* Q, const void* K, const void* V, const void* beta,
                 const float* Hbound, const void* dy, const float* dHT, void* dQ, void* dK,
                 void* dV, void* dbeta, float* dH0, int64_t B, int64_t H, int64_t T, int nh,
                 int dk, int dv, int chunk, int dtype, void* ws, size_t ws_bytes,
                 mg_stream_t stream);

/* ---- DeltaMinGRU decay-gated chunked-WY delta rule ------------------------------------
 * No reference kernel: replaces the eager decay-active forward
 * (DeltaMinGRU._forward_chunked_gated, src/mingru/min_gru.py:3257-3448, guarded by
 * _delta_decay_dispatch_guard :612-668) and its autograd backward.  Per token t the
 * state decays by gamma_t = exp(log_gamma[b,h,t]) before the token's nh micro-steps.
 * Layouts and dtype tag as mg_delta_fwd (dtype 1 = bf16, any nh), plus
 * log_gamma / dlog_gamma (B,H,T) fp32.  `Hbound` takes mg_delta_state_bytes; `ws`
 * mg_delta_gated_workspace_bytes (forward and backward). */
size_t mg_delta_gated_workspace_bytes(int64_t B, int64_t H, int64_t T, int nh, int dk, int dv,
                                      int chunk);
int mg_delta_gated_fwd(const void* Q, const void* K, const void* V, const void* beta,
                       const float* log_gamma, const float* H0, void* y, float* HT,
                       float* Hbound, int64_t B, int64_t H, int64_t T, int nh, int dk, int dv,
                       int chunk, int dtype, void* ws, size_t ws_bytes, mg_stream_t stream);
/* dy (dtype), dHT -> dQ, dK, dV, dbeta (dtype), dlog_gamma and dH0 (fp32). */
int mg_delta_gated_bwd(const void* Q, const void* K, const void* V, const void* beta,
                       const float* log_gamma, const float* Hbound, const void* dy,
                       const float* dHT, void* dQ, void* dK, void* dV, void* dbeta,
                       float* dlog_gamma, float* dH0, int64_t B, int64_t H, int64_t T, int nh,
                       int dk, int dv, int chunk, int dtype, void* ws, size_t ws_bytes,
                       mg_stream_t stream);

/* ---- streaming decode: one recurrent step (inference) -----------------------------
 * No reference kernels: these replace the eager bodies of the mixers' step()
 * (src/mingru/min_gru.py:1399-1448 MinGRU, SignedMinGRU.step, 3611-3688
 * DeltaMinGRU.step).  No workspace.
 * mg_gate_step: h = gamma * a * h_prev + b over n elements, kind 0 SignedMinGRU
 * (p0, p1, p2 = s, z, hpre), 1 SignedMinGRU coupled, 2 MinGRU (p0, p1 = k, hpre;
 * p2 unused, may be NULL); gamma may be NULL (no decay). */
int mg_gate_step(int kind, const float* p0, const float* p1, const float* p2, const float* gamma,
                 const float* h_prev, float* h, int64_t n, mg_stream_t stream);
/* mg_delta_step: per head of BH, H (dk,dv) -> H_out = H after exp(log_gamma)
 * decay (log_gamma (BH) may be NULL) and nh micro-steps H += beta k (v - H^T k)^T;
 * y (dv) = H_out^T q.  q (BH,dk), k (BH,nh,dk), v (BH,nh,dv), beta (BH,nh), all
 * fp32; 1 <= dk, dv <= 64.  H_out may equal H (in-place update). */
int mg_delta_step(const float* H, const float* q, const float* k, const float* v,
                  const float* beta, const float* log_gamma, float* H_out, float* y, int64_t BH,
                  int nh, int dk, int dv, mg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MINGRU_HIP_H */

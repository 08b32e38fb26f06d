/* tssm -- C ABI of the MI355X (gfx950) selective-SSM library.
 *
 * Every entry point:
 *   - takes raw device pointers, int64 sizes/strides (in elements) and a
 *     hipStream_t passed as void*; launches asynchronously on that stream;
 *   - never allocates and never synchronises;
 *   - returns 0 on success, a negative TSSM_ERR_* code for an invalid
 *     argument (nothing is launched), or a positive hipError_t.
 * Innermost (channel) strides are 1, exactly as the reference kernels assume
 * (they accept innermost strides but never use them).
 *
 * Reference citations are file:line into Triton-SSM.  "grid_*" arguments give
 * the Triton launch grid the caller used: the library computes exactly the
 * programs of that grid, whatever launch geometry it picks for itself.
 */
#ifndef TSSM_H_
#define TSSM_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define TSSM_OK 0
#define TSSM_ERR_NULL (-1)        /* a required pointer is NULL */
#define TSSM_ERR_SHAPE (-2)       /* a size is negative, zero where not allowed, or inconsistent */
#define TSSM_ERR_STRIDE (-3)      /* a stride is invalid for the access pattern */
#define TSSM_ERR_DTYPE (-4)       /* unknown or unsupported dtype code */
#define TSSM_ERR_WORKSPACE (-5)   /* workspace missing or too small */
#define TSSM_ERR_UNSUPPORTED (-6) /* valid but unsupported configuration */
#define TSSM_ERR_ALIGN (-7)       /* pointer/stride not aligned for vector access */
#define TSSM_ERR_SCRATCH (-8)     /* too large for the no-allocation entry point's scratch */

/* dtype codes */
#define TSSM_F32 0
#define TSSM_BF16 1
#define TSSM_F16 2

/* input discretization of the fused scans */
#define TSSM_DISC_EULER 0 /* Bbar = dt * B           (multihead_ssm_kernel.py:73) */
#define TSSM_DISC_ZOH 1   /* Bbar = expm1(dt a)/a * B (discretize_kernel.py:50-54) */

int tssm_abi_version(void);
const char* tssm_strerror(int status);

/* Workspaces of the single-pass (decoupled look-back) scans are caller-owned
 * device buffers, zero-filled ONCE when allocated and then reused by launches
 * on one stream; nothing else may be written into them (tssm_ssd_scan's
 * workspace in particular is a separate buffer).  A bounded look-back wait
 * that expires (~1 s) sets the workspace's sticky error word and the launch
 * completes with that tile's carry incomplete.  This reads the word
 * (1 = expired) with a synchronous copy -- call it after the stream has
 * finished; with clear=1 a set word is reset to 0.  workspace == NULL reads
 * the word of the current device's tssm_mh_scan_fused_noalloc scratch. */
int tssm_workspace_error(const void* workspace, int clear, int* error_out);

/* Attach a host-visible flag to a look-back workspace (workspace == NULL: the
 * current device's no-allocation scratch), so that an expired wait is seen
 * without synchronising: the kernel that sets the sticky word also stores 1
 * to *host_flag (a system-scope store on that error path only; nothing is
 * written there otherwise).  host_flag must be pinned host memory
 * (hipHostMalloc, or a torch tensor made with pin_memory=True); the caller
 * polls it (e.g. before its next launch on the workspace) and resets it.
 * host_flag == NULL detaches.  A set-up call: one synchronous 8-byte copy into
 * the workspace header.  No reference counterpart (the reference reports no
 * errors at run time). */
int tssm_workspace_attach_host_flag(void* workspace, int* host_flag);

/* ------------------------------------------------------------------ ZOH
 * zoh_discretize_diag_kernel / zoh_discretize_diag_bf16_kernel
 * (discretize_kernel.py:16-57 / :61-94).  Grid (B, T, ceil(H/BLOCK_H)):
 * computes (b < grid_b, t < grid_t, h < min(H, h_cover)).
 * A_log [H] f32, dt [B,T] f32; B, Abar, Bbar in b_dtype / out_dtype. */
int tssm_zoh_discretize(int b_dtype, int out_dtype, const float* A_log, const void* B,
                        const float* dt, void* Abar, void* Bbar, int64_t nbatch, int64_t T,
                        int64_t H, int64_t grid_b, int64_t grid_t, int64_t h_cover,
                        int64_t sB_b, int64_t sB_t, int64_t sdt_b, int64_t sdt_t, int64_t sa_b,
                        int64_t sa_t, int64_t sb_b, int64_t sb_t, void* stream);

/* zoh_discretize_bwd_kernel (discretize_kernel.py:98-162).  Same grid and
 * strides as the forward (dB uses B's strides, dAbar Abar's, dBbar Bbar's,
 * ddt dt's).  dA [H] f32 is ACCUMULATED into (the reference's atomic_add at
 * :156); ddt [B,T] f32 is overwritten with the sum over the covered lanes (the
 * intent of the store/atomic pair at :159-162).  Deterministic: partial sums
 * go through a caller workspace of tssm_zoh_discretize_bwd_workspace_bytes()
 * bytes (no clearing needed) and are reduced in a fixed order.  B, Abar,
 * dAbar, dBbar and dB share `dtype`; A_log, dt, dA and ddt are f32. */
int64_t tssm_zoh_discretize_bwd_workspace_bytes(int64_t grid_b, int64_t grid_t, int64_t h_cover);
int tssm_zoh_discretize_bwd(int dtype, const float* A_log, const void* B, const float* dt,
                            const void* Abar, const void* dAbar, const void* dBbar, float* dA,
                            void* dB, float* ddt, int64_t nbatch, int64_t T, int64_t H,
                            int64_t grid_b, int64_t grid_t, int64_t h_cover, int64_t sB_b,
                            int64_t sB_t, int64_t sdt_b, int64_t sdt_t, int64_t sa_b,
                            int64_t sa_t, int64_t sb_b, int64_t sb_t, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* dt_project_softplus_kernel (discretize_kernel.py:166-213; the scalar index
 * of a block tensor at :203 implemented as its evident intent):
 * dt_out[b,t,h] = clamp(softplus(sum_r dt_raw[b,t,r] W[r,h] + bias[h]),
 * dt_min, dt_max) for b < grid_b, t < grid_t, h < h_cover.  dt_raw [B,T,rank]
 * (strides sr_b, sr_t, unit over r), W [rank,H] (row stride sw_r, unit over h),
 * bias [H], all f32; dt_out in out_dtype with strides so_b, so_t, unit over h. */
int tssm_dt_project_softplus(int out_dtype, const float* dt_raw, const float* W,
                             const float* bias, void* dt_out, int64_t nbatch, int64_t T,
                             int64_t H, int64_t rank, int64_t grid_b, int64_t grid_t,
                             int64_t h_cover, int64_t sr_b, int64_t sr_t, int64_t sw_r,
                             int64_t so_b, int64_t so_t, float dt_min, float dt_max,
                             void* stream);

/* ------------------------------------------------------------------ elementwise scan
 * ssm_scan.py phase kernels; u, A, B, C, D, h, y, loc_*, carry all in `dtype`,
 * contiguous [B, L, H] (the reference computes offsets b*L*H + t*H + h).
 * carry layout [2, B*H, NBLK] (ssm_scan.py:47-50). */
int tssm_ssm_fwd_local(int dtype, const void* u, const void* A, const void* B, void* loc_a,
                       void* loc_x, void* carry, int64_t nbatch, int64_t L, int64_t H,
                       int64_t blk, int64_t nblk, int64_t grid_rows, int64_t grid_blks,
                       void* stream); /* ssm_fwd_local_kernel, ssm_scan.py:18-50 */
int tssm_carry_scan(int dtype, void* carry, int64_t nrows, int64_t nblk, int reverse,
                    int64_t grid_rows, void* stream);
/* ssm_carry_scan_kernel (ssm_scan.py:54-65), ssm_bwd_carry_scan_kernel (:174-185,
 * reverse=1), multihead_ssm_carry_scan_kernel (multihead_ssm_kernel.py:106-117) */
int tssm_ssm_fwd_apply(int dtype, const void* loc_a, const void* loc_x, const void* carry,
                       void* h_out, int64_t nbatch, int64_t L, int64_t H, int64_t blk,
                       int64_t nblk, int64_t grid_rows, int64_t grid_blks,
                       void* stream); /* ssm_fwd_apply_kernel, ssm_scan.py:69-98 */
int tssm_ssm_output(int dtype, const void* h, const void* C, const void* D, const void* u,
                    void* y, int64_t nbatch, int64_t L, int64_t H, int64_t blk,
                    int64_t grid_rows, int64_t grid_blks,
                    void* stream); /* ssm_output_kernel, ssm_scan.py:102-124 */
int tssm_ssm_bwd_local(int dtype, const void* A, const void* C, const void* dY, void* loc_a,
                       void* loc_dh, void* carry, int64_t nbatch, int64_t L, int64_t H,
                       int64_t blk, int64_t nblk, int64_t grid_rows, int64_t grid_blks,
                       void* stream); /* ssm_bwd_local_kernel, ssm_scan.py:136-170 */
int tssm_ssm_bwd_apply(int dtype, const void* loc_a, const void* loc_dh, const void* carry,
                       const void* u, const void* A, const void* B, const void* h,
                       const void* dY, void* du, void* dA, void* dB, void* dC, int64_t nbatch,
                       int64_t L, int64_t H, int64_t blk, int64_t nblk, int64_t grid_rows,
                       int64_t grid_blks,
                       void* stream); /* ssm_bwd_apply_kernel, ssm_scan.py:189-231 */

/* ------------------------------------------------------------------ multihead DIAG scan
 * multihead_ssm_fwd_local_kernel (multihead_ssm_kernel.py:20-102): Euler input
 * term, loc_a/loc_x f32 [B,L,nh,hd], carry f32 [2, B*nh*hd, NBLK].
 * u/B in `dtype`; A_log [nh, *] f32 with row stride sal_h; dt f32. */
int tssm_mh_fwd_local(int dtype, const void* u, const float* A_log, const void* B,
                      const float* dt, float* loc_a, float* loc_x, float* carry,
                      int64_t nbatch, int64_t L, int64_t H, int64_t n_heads, int64_t head_dim,
                      int64_t su_b, int64_t su_l, int64_t sal_h, int64_t sB_b, int64_t sB_l,
                      int64_t sB_h, int64_t sdt_b, int64_t sdt_l, int64_t sdt_h, int64_t blk_l,
                      int64_t nblk, int64_t grid_rows, int64_t grid_blks, void* stream);
/* multihead_ssm_output_kernel (multihead_ssm_kernel.py:121-187): y contiguous
 * [B, L, H] in `dtype`; C/u in `dtype`; D [H] f32. */
int tssm_mh_output(int dtype, const float* loc_a, const float* loc_x, const float* carry,
                   const void* C, const float* D, const void* u, void* y, int64_t nbatch,
                   int64_t L, int64_t H, int64_t n_heads, int64_t head_dim, int64_t su_b,
                   int64_t su_l, int64_t sC_b, int64_t sC_l, int64_t sC_h, int64_t blk_l,
                   int64_t nblk, int64_t grid_rows, int64_t grid_blks, void* stream);

/* Fused single-pass DIAG multihead scan (a9 -> a11 in one launch, with the
 * discretization fused into the load stage and a decoupled look-back across
 * chunks).  u [B,L,nh*hd], B/C [B,L,nh,hd], y [B,L,nh*hd] in `dtype`;
 * A_log f32 [nh,hd] (a_per_head=0) or [nh] (a_per_head=1); dt f32 [B,L,nh];
 * D f32 [nh*hd] or NULL; h0 f32 [B,nh,hd] or NULL; h_last f32 [B,nh,hd] or
 * NULL.  head_dim must be a multiple of 8 and <= 128; channel rows must be
 * 16-byte aligned.  `chunk` selects the time tile (64, 128 or 256). */
int64_t tssm_mh_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t n_heads,
                                     int64_t head_dim, int64_t chunk);
int tssm_mh_scan_fused(int dtype, int disc, const void* u, const float* A_log, const void* B,
                       const void* C, const float* dt, const float* D, const float* h0,
                       void* y, float* h_last, int64_t nbatch, int64_t L, int64_t n_heads,
                       int64_t head_dim, int a_per_head, int64_t su_b, int64_t su_l,
                       int64_t sB_b, int64_t sB_l, int64_t sB_h, int64_t sC_b, int64_t sC_l,
                       int64_t sC_h, int64_t sdt_b, int64_t sdt_l, int64_t sdt_h, int64_t sy_b,
                       int64_t sy_l, int64_t chunk, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* No-allocation variant of tssm_mh_scan_fused.  No reference counterpart: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernel and results as tssm_mh_scan_fused, without the workspace:
 * the look-back words live in a fixed device array of
 * TSSM_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends), whose
 * address is resolved on the first call on each device -- make that first
 * call outside graph capture.  Each call enqueues two kernels: a one-thread
 * kernel that advances the scratch's epoch (the tag of the call's look-back
 * words) on the device, then the scan, which reads it; so a call captured in
 * a HIP graph takes a fresh tag on every replay, and nothing is cleared with
 * a memset.  Problems needing more than the array
 * (tssm_mh_scan_workspace_bytes() > the maximum) return TSSM_ERR_SCRATCH;
 * `stream` must belong to the current device.  Every call on a GPU shares its
 * array: calls (or graph replays) that overlap on one GPU race.  Its sticky
 * look-back error word is read with tssm_workspace_error(NULL, ...). */
#define TSSM_NOALLOC_SCRATCH_BYTES (16ll << 20)
int tssm_mh_scan_fused_noalloc(int dtype, int disc, const void* u, const float* A_log,
                               const void* B, const void* C, const float* dt, const float* D,
                               const float* h0, void* y, float* h_last, int64_t nbatch,
                               int64_t L, int64_t n_heads, int64_t head_dim, int a_per_head,
                               int64_t su_b, int64_t su_l, int64_t sB_b, int64_t sB_l,
                               int64_t sB_h, int64_t sC_b, int64_t sC_l, int64_t sC_h,
                               int64_t sdt_b, int64_t sdt_l, int64_t sdt_h, int64_t sy_b,
                               int64_t sy_l, int64_t chunk, void* stream);

/* ------------------------------------------------------------------ interpolation
 * fused_time_aware_interp_kernel / fused_interp_bf16_kernel /
 * fused_interp_fp16_kernel (fused_interp_kernel.py:10-100 / :104-181 /
 * :187-257).  V, Vhat in v_dtype; M and tau in any float dtype.  Grid
 * (B, T, ceil(F/FTILE)): computes b < grid_b, t < grid_t, tiles < grid_f.
 * K (search window; bounded by the 64 KiB of LDS one workgroup stages the
 * window's flags in: K <= 32352 here, TSSM_ERR_UNSUPPORTED beyond) and FTILE
 * (tile of the "any observed" aggregate) are semantic: they change results.  The per-(b, t, tile) "any observed"
 * flags go through a caller workspace of
 * tssm_time_aware_interp_workspace_bytes() bytes (no clearing needed). */
int64_t tssm_time_aware_interp_workspace_bytes(int64_t T, int64_t F, int64_t K, int64_t FTILE,
                                               int64_t grid_b, int64_t grid_t, int64_t grid_f);
int tssm_time_aware_interp(int v_dtype, int m_dtype, int tau_dtype, const void* V, const void* M,
                           const void* tau, void* Vhat, int64_t nbatch, int64_t T, int64_t F,
                           int64_t svb, int64_t svt, int64_t smb, int64_t smt, int64_t stb,
                           int64_t stt, int64_t sob, int64_t sot, int64_t K, int64_t FTILE,
                           int64_t grid_b, int64_t grid_t, int64_t grid_f, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* Opt-in "corrected" interpolation (no reference counterpart: the intent
 * stated at fused_interp_kernel.py:49-50, not the reference's behaviour, which
 * tssm_time_aware_interp keeps).  Per (b, t, f): an observed value (M > 0.5)
 * is kept; otherwise the nearest steps within K on each side where that
 * feature is observed give the value with the reference's weights, clipping
 * and one-sided fills.  Whole tensors, no workspace. */
int tssm_time_aware_interp_corrected(int v_dtype, int m_dtype, int tau_dtype, const void* V,
                                     const void* M, const void* tau, void* Vhat, int64_t nbatch,
                                     int64_t T, int64_t F, int64_t svb, int64_t svt, int64_t smb,
                                     int64_t smt, int64_t stb, int64_t stt, int64_t sob,
                                     int64_t sot, int64_t K, void* stream);

/* fused_interp_ssm_step_kernel (fused_ssm_interp.py:12-101): interpolates
 * step t_cur into Vhat[:, t_cur] and writes h_out = A_bar*h_in + B_bar*vhat.
 * A_bar, B_bar [F], h_in, h_out f32.  Grid (B, ceil(F/FTILE)). */
int tssm_interp_ssm_step(int v_dtype, int m_dtype, int tau_dtype, const void* V, const void* M,
                         const void* tau, const float* A_bar, const float* B_bar,
                         const float* h_in, void* Vhat, float* h_out, int64_t nbatch, int64_t T,
                         int64_t F, int64_t svb, int64_t svt, int64_t smb, int64_t smt,
                         int64_t stb, int64_t stt, int64_t sob, int64_t sot, int64_t s_hib,
                         int64_t s_hob, int64_t t_cur, int64_t K, int64_t FTILE, int64_t grid_b,
                         int64_t grid_f, void* stream);

/* Interpolation + Mamba-1 scan over a whole sequence (the sequence form of
 * fused_interp_ssm_step_kernel, fused_ssm_interp.py:12-101, with the
 * interpolation of fused_interp_kernel.py:29-100 and the scan of
 * tssm_selective_scan with dt_t = tau_t - tau_{t-1}, dt_0 = tau_0): Vhat is
 * formed inside the scan's first pass, written once and consumed there as x;
 * three launches on `stream` (five when few lanes carry many chunks: the
 * carry scan then folds 32-chunk segments first).  V, Vhat, B, C, y in
 * `dtype` (f32 or bf16), M
 * and tau f32; V/M/Vhat [B,T,F], tau [B,T], B/C [B,T,N], y [B,T,F]; A_log
 * f32 [F,N]; D f32 [F] or NULL; h0/h_last f32 [B,F,N] or NULL.  K and FTILE as
 * in tssm_time_aware_interp (semantic).  Returns TSSM_ERR_UNSUPPORTED before
 * any launch unless tssm_interp_selective_scan_supported() holds (f32 masks in
 * 16-byte rows, FTILE a power of two in [16, 256], 1 <= K <= 64, F a multiple
 * of 4, N 8 or 16, a problem of at least 512 blocks of 64 channels x 32
 * steps); callers then run tssm_time_aware_interp and tssm_selective_scan.
 * The workspace (raw fp32 chunk states, not look-back words) holds
 * tssm_interp_selective_scan_workspace_bytes() bytes.  No reference
 * counterpart as one entry point. */
int64_t tssm_interp_selective_scan_workspace_bytes(int64_t nbatch, int64_t T, int64_t F,
                                                   int64_t N);
int tssm_interp_selective_scan_supported(int dtype, int m_dtype, int tau_dtype, int64_t nbatch,
                                         int64_t T, int64_t F, int64_t N, int64_t K,
                                         int64_t FTILE, const void* M, int64_t sm_b,
                                         int64_t sm_t, int64_t sv_t);
int tssm_interp_selective_scan(int dtype, int disc, const void* V, const float* M,
                               const float* tau, const float* A_log, const void* B,
                               const void* C, const float* D, const float* h0, void* Vhat,
                               void* y, float* h_last, int64_t nbatch, int64_t T, int64_t F,
                               int64_t N, int64_t sv_b, int64_t sv_t, int64_t sm_b, int64_t sm_t,
                               int64_t stau_b, int64_t stau_t, int64_t sB_b, int64_t sB_l,
                               int64_t sC_b, int64_t sC_l, int64_t so_b, int64_t so_t,
                               int64_t sy_b, int64_t sy_t, int64_t K, int64_t FTILE,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ streaming
 * streaming_ssm_inplace_kernel / streaming_ssm_inplace_bf16_kernel
 * (streaming_inference_kernel.py:7-37 / :41-71).  All tensors in `dtype`;
 * h updated in place; y uses vhat's batch stride svb.  Grid
 * (B, ceil(H/BLOCK_H)): computes b < grid_b, lanes < min(H, h_cover). */
int tssm_stream_step(int dtype, const void* vhat, void* h, const void* Abar, const void* Bbar,
                     const void* C, const void* D, void* y, int64_t nbatch, int64_t H,
                     int64_t grid_b, int64_t h_cover, int64_t svb, int64_t shb, int64_t scb,
                     void* stream);

/* streaming_interp_then_ssm_kernel (streaming_inference_kernel.py:75-156),
 * f32 tensors and int32 ring_head.  One workgroup per stream makes the ring
 * head update race-free; BLOCK_H stays the tile of the "any observed" test. */
int tssm_stream_interp_step(float* ring_V, float* ring_M, float* ring_tau, int32_t* ring_head,
                            const float* v_new, const float* m_new, const float* tau_new,
                            float* h, const float* Abar, const float* Bbar, const float* C,
                            const float* D, float* y, int64_t nbatch, int64_t H, int64_t srb,
                            int64_t srk, int64_t svb, int64_t shb, int64_t scb, int64_t BLOCK_H,
                            int64_t KRING, int64_t grid_b, void* stream);

/* Opt-in corrected streaming step (no reference counterpart): the insert and
 * race-free head update of tssm_stream_interp_step, then per feature an
 * observed new value is kept and an unobserved one is forward-filled from the
 * most recent of the previous KRING-1 slots where that feature was observed. */
int tssm_stream_interp_step_corrected(float* ring_V, float* ring_M, float* ring_tau,
                                      int32_t* ring_head, const float* v_new, const float* m_new,
                                      const float* tau_new, float* h, const float* Abar,
                                      const float* Bbar, const float* C, const float* D, float* y,
                                      int64_t nbatch, int64_t H, int64_t srb, int64_t srk,
                                      int64_t svb, int64_t shb, int64_t scb, int64_t KRING,
                                      void* stream);

/* ------------------------------------------------------------------ SSD (new fused entry points)
 * Selective scan with one decay per head and a P x N state per (batch, head):
 *   h_t[p,n] = exp(dt_t a_h) h_{t-1}[p,n] + Bbar_t x_t[p] B_t[n],
 *   y_t[p] = sum_n C_t[n] h_t[p,n] + D[h,p] x_t[p]
 * (the recurrence of ssm_scan.py:5-10 with discretize_kernel.py:44-54's ZOH
 * or multihead_ssm_kernel.py:73's Euler input term).  No reference kernel
 * covers this family; the reference's elementwise kernels can express it only
 * lane by lane.  Chunk states pass through the workspace (raw fp32, no
 * clearing needed); it must NOT be a workspace of the look-back scans, whose
 * tagged words it would overwrite.  x, B, C, y in `dtype` ([B,L,H,P] / [B,L,H,N]); dt f32
 * [B,L,H]; A_log f32 [H]; D f32 [H*P] or NULL; h0/h_last f32 [B,H,P,N] or
 * NULL.  P <= 64, N in {8, 16, 32, 64}; innermost strides 1. */
int64_t tssm_ssd_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t H, int64_t P,
                                      int64_t N, int64_t chunk);
int tssm_ssd_scan(int dtype, int disc, const void* x, const float* dt, const float* A_log,
                  const void* B, const void* C, const float* D, const float* h0, void* y,
                  float* h_last, int64_t nbatch, int64_t L, int64_t H, int64_t P, int64_t N,
                  int64_t sx_b, int64_t sx_l, int64_t sx_h, int64_t sdt_b, int64_t sdt_l,
                  int64_t sdt_h, int64_t sB_b, int64_t sB_l, int64_t sB_h, int64_t sC_b,
                  int64_t sC_l, int64_t sC_h, int64_t sy_b, int64_t sy_l, int64_t sy_h,
                  int64_t chunk, void* workspace, int64_t workspace_bytes, void* stream);

/* tssm_ssd_scan in one launch for bf16 x/B/C/y, P = 64, N = 16 and 256-step
 * chunks (the matrix-core tile passes' case): a wave takes one segment of a
 * (batch, head) row (one or two 256-step tiles), sweeps it last sub-chunk
 * first for its end state (x, B, dt through the caches), publishes its carry
 * as tagged look-back words, resolves its entry state by a decoupled
 * look-back over the row's earlier segments (a decay product of exactly zero
 * ends a walk), and sweeps the segment again forward for the outputs, so
 * that what it reads a second time is still in the last-level cache.  Same
 * arguments and results as tssm_ssd_scan (D f32 [H*P] or NULL; h0/h_last f32
 * [B,H,P,N] contiguous or NULL); the workspace is a look-back workspace
 * (zero-filled once, epoch-tagged words, tssm_workspace_error reads its
 * sticky word) of tssm_ssd_scan_fused_workspace_bytes() bytes.
 * tssm_ssd_scan_fused_supported() says whether these operands take it (else
 * the call returns TSSM_ERR_UNSUPPORTED before any launch). */
int64_t tssm_ssd_scan_fused_workspace_bytes(int64_t nbatch, int64_t L, int64_t H, int64_t P,
                                            int64_t N, int64_t chunk);
int tssm_ssd_scan_fused_supported(int dtype, const void* x, const float* dt, const float* A_log,
                                  const void* B, const void* C, const float* D, const float* h0,
                                  void* y, float* h_last, int64_t nbatch, int64_t L, int64_t H,
                                  int64_t P, int64_t N, int64_t sx_b, int64_t sx_l, int64_t sx_h,
                                  int64_t sdt_b, int64_t sdt_l, int64_t sdt_h, int64_t sB_b,
                                  int64_t sB_l, int64_t sB_h, int64_t sC_b, int64_t sC_l,
                                  int64_t sC_h, int64_t sy_b, int64_t sy_l, int64_t sy_h,
                                  int64_t chunk);
int tssm_ssd_scan_fused(int dtype, int disc, const void* x, const float* dt, const float* A_log,
                        const void* B, const void* C, const float* D, const float* h0, void* y,
                        float* h_last, int64_t nbatch, int64_t L, int64_t H, int64_t P,
                        int64_t N, int64_t sx_b, int64_t sx_l, int64_t sx_h, int64_t sdt_b,
                        int64_t sdt_l, int64_t sdt_h, int64_t sB_b, int64_t sB_l, int64_t sB_h,
                        int64_t sC_b, int64_t sC_l, int64_t sC_h, int64_t sy_b, int64_t sy_l,
                        int64_t sy_h, int64_t chunk, void* workspace, int64_t workspace_bytes,
                        void* stream);

/* One streaming SSD step for S independent streams with the state
 * [S,H,P,N] f32 resident in HBM and updated in place (the per-stream,
 * per-head generalisation of streaming_ssm_inplace_kernel,
 * streaming_inference_kernel.py:7-37).  x [S,H,P], B/C [S,H,N] (16-byte
 * aligned rows), y [S,H,P], dt [S,H] via strides (sdt_h = 0 for one dt per
 * stream), A_log [H], D [H*P] or NULL; all f32.  N in {16,...,256} (powers of 2). */
int tssm_ssd_stream_step(int disc, const float* x, const float* dt, const float* A_log,
                         const float* B, const float* C, const float* D, float* state, float* y,
                         int64_t S, int64_t H, int64_t P, int64_t N, int64_t sdt_s,
                         int64_t sdt_h, int64_t sx_s, int64_t sx_h, int64_t sB_s, int64_t sB_h,
                         int64_t sC_s, int64_t sC_h, int64_t sy_s, int64_t sy_h, void* stream);

/* ------------------------------------------------------------------ Mamba-1 selective scan
 * Lanes (channel d, state n) of a diagonal selective SSM:
 *   h_t[d,n] = exp(dt_t a[d,n]) h_{t-1}[d,n] + Bbar_t[d,n] B_t[n] x_t[d],
 *   y_t[d] = sum_n C_t[n] h_t[d,n] + D[d] x_t[d]
 * -- what the reference computes with zoh_discretize_diag_kernel over lanes
 * (d,n) followed by ssm_forward and a sum over n (discretize_kernel.py:16-57,
 * ssm_scan.py:239-264), fused: one single-pass launch (same kernel as
 * tssm_mh_scan_fused with the channel input broadcast over the states), or,
 * for N = 8 or 16 with f32/bf16 I/O and at least 512 blocks of 64 channels x
 * 32 steps, three launches on `stream` (chunk end states, a carry scan over
 * the chunks, the outputs; the carry scan takes three launches of its own
 * when few lanes carry many chunks) with lanes = channels; `chunk` then does
 * not apply.  The workspace size covers either.
 * x, B, C, y in `dtype` ([B,L,Dc] / [B,L,N]); A_log f32 [Dc,N]; dt f32 with
 * strides (b, l, d) -- sdt_d = 0 for one dt per (b,t); with dt_is_tau=1 dt
 * holds timestamps tau and dt_t = tau_t - tau_{t-1}, dt_0 = tau_0.
 * D f32 [Dc] or NULL; h0/h_last f32 [B,Dc,N] or NULL.  N a multiple of 8,
 * <= 128; B/C rows 16-byte aligned. */
int64_t tssm_selective_scan_workspace_bytes(int64_t nbatch, int64_t L, int64_t Dc, int64_t N,
                                            int64_t chunk);
int tssm_selective_scan(int dtype, int disc, const void* x, const float* dt, int dt_is_tau,
                        const float* A_log, const void* B, const void* C, const float* D,
                        const float* h0, void* y, float* h_last, int64_t nbatch, int64_t L,
                        int64_t Dc, int64_t N, int64_t sx_b, int64_t sx_l, int64_t sdt_b,
                        int64_t sdt_l, int64_t sdt_d, int64_t sB_b, int64_t sB_l, int64_t sC_b,
                        int64_t sC_l, int64_t sy_b, int64_t sy_l, int64_t chunk, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* tssm_selective_scan with the dt producer fused into the scan: per
 * (b, t, d), dt = clamp(softplus(sum_k dt_raw[b,t,k] W[k,d] + bias[d]),
 * dt_min, dt_max) -- dt_project_softplus_kernel (discretize_kernel.py:166-213,
 * the scalar block index at :203 taken as its evident intent) feeding the
 * scan, without a caller-side [B,L,Dc] dt tensor or a projection launch.
 * dt_raw f32 [B,L,rank] (strides sr_b, sr_l, unit over k), W f32 [rank, Dc]
 * (row stride sw_r, unit over d), bias f32 [Dc]; rank <= 64.  Everything else
 * as tssm_selective_scan.  Large problems (the three-pass scan) form dt on
 * the matrix cores inside the passes, bit-identical to the projection
 * kernel's values, when rank, Dc and the row strides are multiples of 4 and
 * dt_raw, W, bias are 16-byte aligned.  The workspace may be
 * tssm_selective_scan_workspace_bytes() bytes (pass 3 then produces dt again)
 * or tssm_selective_scan_dtproj_workspace_bytes() (pass 1 also stores the dt
 * it produced there and pass 3 reads it back, the faster form). */
int64_t tssm_selective_scan_dtproj_workspace_bytes(int64_t nbatch, int64_t L, int64_t Dc,
                                                   int64_t N, int64_t chunk);

/* 1 if tssm_selective_scan (W == NULL: dt given, dt_raw its pointer, sdt_d
 * its channel stride) or tssm_selective_scan_dtproj (W != NULL) takes the
 * three-pass path for these operands, else 0 (the single-pass look-back
 * kernel).  The three passes write raw fp32 chunk states (and the produced
 * dt) into the workspace, not tagged look-back words: a workspace that served
 * them must be zero-filled before any look-back launch uses it, so callers
 * keep separate workspaces for the two paths (tssm/workspace.py does).  No
 * reference counterpart. */
int tssm_selective_scan_takes_passes(int dtype, int64_t nbatch, int64_t L, int64_t Dc, int64_t N,
                                     int64_t sdt_d, int dt_is_tau, const float* dt_raw,
                                     const float* W, const float* bias, int64_t rank,
                                     int64_t sr_b, int64_t sr_l, int64_t sw_r);
int tssm_selective_scan_dtproj(int dtype, int disc, const void* x, const float* dt_raw,
                               const float* W, const float* bias, float dt_min, float dt_max,
                               const float* A_log, const void* B, const void* C, const float* D,
                               const float* h0, void* y, float* h_last, int64_t nbatch,
                               int64_t L, int64_t Dc, int64_t N, int64_t rank, int64_t sx_b,
                               int64_t sx_l, int64_t sr_b, int64_t sr_l, int64_t sw_r,
                               int64_t sB_b, int64_t sB_l, int64_t sC_b, int64_t sC_l,
                               int64_t sy_b, int64_t sy_l, int64_t chunk, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* tssm_selective_scan with B and C produced from x in the scan: B_t = x_t W_B,
 * C_t = x_t W_C (Mamba-1's input projection columns for B and C, the step
 * before ssm_scan.py:239-264 in a selective model; the reference has no
 * kernel for it), so no B/C tensors and no projection launch.  W_bc f32
 * [Dc, 2N]: columns 0..N-1 W_B, N..2N-1 W_C, row stride sw_d (>= 2N), unit
 * column stride (a column slice of a wider x_proj weight works).  fp32 x/y,
 * Dc <= 256 and a multiple of 4, N 8 or 16, x rows 16-byte aligned; dt as in
 * tssm_selective_scan (shared, with or without timestamps, or per channel).
 * Three launches (five when few lanes carry many chunks): pass 1 stages
 * each 32-step chunk's x tile in LDS, forms the chunk's B/C rows on the fp32 matrix cores and runs the recurrence from
 * that tile; pass 3 reads the C rows pass 1 stored in the workspace
 * (tssm_selective_scan_bcproj_workspace_bytes() bytes: raw fp32, not
 * look-back words).  No reference counterpart. */
int64_t tssm_selective_scan_bcproj_workspace_bytes(int64_t nbatch, int64_t L, int64_t Dc,
                                                   int64_t N);
int tssm_selective_scan_bcproj(int disc, const float* x, const float* dt, int dt_is_tau,
                               const float* A_log, const float* W_bc, int64_t sw_d,
                               const float* D, const float* h0, float* y, float* h_last,
                               int64_t nbatch, int64_t L, int64_t Dc, int64_t N, int64_t sx_b,
                               int64_t sx_l, int64_t sdt_b, int64_t sdt_l, int64_t sdt_d,
                               int64_t sy_b, int64_t sy_l, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* tssm_selective_scan with the whole selective input projection in the
 * scan, x -> (dt, B, C): x_dbl_t = x_t W_x (Mamba-1's x_proj; the reference
 * has no kernel for it), dt_raw = x_dbl[:, :rank], B = x_dbl[:, rank:rank+N],
 * C = x_dbl[:, rank+N:rank+2N], and dt = clamp(softplus(dt_raw W_dt + bias),
 * dt_min, dt_max) as dt_project_softplus_kernel computes it
 * (discretize_kernel.py:166-213).  W_x f32 [Dc, rank + 2N], row stride swx_d
 * (>= rank + 2N), unit column stride; W_dt f32 [rank][Dc], row stride sw_r
 * (>= Dc, a multiple of 4), bias [Dc]; rank 16, 32, 48 or 64.  fp32 x/y,
 * Dc <= 256 and a multiple of 4, N 8 or 16, x rows and W_dt, bias, A_log
 * 16-byte aligned.  Three launches (five when few lanes carry many chunks):
 * pass 1 stages each 32-step chunk's x tile in LDS, forms its dt_raw/B/C rows on the fp32 matrix cores, then every
 * channel's dt (stored to a dt table in the workspace) and runs the
 * recurrence; pass 3 reads the dt table and the C rows.  Workspace of
 * tssm_selective_scan_xproj_workspace_bytes() bytes (raw fp32, not look-back
 * words).  No reference counterpart. */
int64_t tssm_selective_scan_xproj_workspace_bytes(int64_t nbatch, int64_t L, int64_t Dc,
                                                  int64_t N);
int tssm_selective_scan_xproj(int disc, const float* x, const float* A_log, const float* W_x,
                              int64_t swx_d, int64_t rank, const float* W_dt, int64_t sw_r,
                              const float* bias, float dt_min, float dt_max, const float* D,
                              const float* h0, float* y, float* h_last, int64_t nbatch, int64_t L,
                              int64_t Dc, int64_t N, int64_t sx_b, int64_t sx_l, int64_t sy_b,
                              int64_t sy_l, void* workspace, int64_t workspace_bytes,
                              void* stream);

/* ------------------------------------------------------------------ elementwise scan, single pass
 * The host functions ssm_forward / ssm_backward (ssm_scan.py:239-289) as one
 * launch each over contiguous [B, L, H] tensors of `dtype` (D [H]): every
 * input read once, every output written once; the state crosses chunks by a
 * decoupled look-back.  forward: y, h.  backward: du = B dh, dA = h_{t-1} dh,
 * dB = u dh, dC = dY h with dh_t = A_{t+1} dh_{t+1} + C_t dY_t.  H % 4 == 0;
 * pointers 16-byte (fp32) / 8-byte (16-bit) aligned.  Workspace: zero-filled
 * once, 256-aligned, tssm_ssm_scan_fused_workspace_bytes(B, L, H) bytes; one
 * stream at a time. */
int64_t tssm_ssm_scan_fused_workspace_bytes(int64_t nbatch, int64_t L, int64_t H);
int tssm_ssm_forward_fused(int dtype, const void* u, const void* A, const void* B, const void* C,
                           const void* D, void* y, void* h, int64_t nbatch, int64_t L, int64_t H,
                           void* workspace, int64_t workspace_bytes, void* stream);
int tssm_ssm_backward_fused(int dtype, const void* u, const void* A, const void* B,
                            const void* C, const void* h, const void* dY, void* du, void* dA,
                            void* dB, void* dC, int64_t nbatch, int64_t L, int64_t H,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ model layers
 * The reference's layers around the scan.  Arithmetic fp32; every float
 * tensor of one call has `dtype` (TSSM_F32/BF16/F16).  Rows are the
 * (grid_b x grid_l) programs of the reference grid; innermost strides 1. */

/* layernorm_kernel (fused_ssm_interp.py:105-129): out = (x-mu)/sqrt(var+eps)*w
 * + bias per row of H (x and out share strides).  block_h >= H is the
 * reference's BLOCK_H: its H..BLOCK_H-1 masked lanes enter var as mu^2. */
int tssm_layernorm_fwd(int dtype, const void* x, const void* w, const void* bias, void* out,
                       int64_t nbatch, int64_t L, int64_t H, int64_t stride_b, int64_t stride_l,
                       float eps, int64_t block_h, int64_t grid_b, int64_t grid_l, void* stream);

/* layernorm_bwd_kernel (fused_ssm_interp.py:134-171): dx per row (dout, x, dx
 * share strides); dw += sum_rows dout*xhat and db += sum_rows dout, summed in a
 * fixed order (the reference adds atomically).  Workspace:
 * tssm_layernorm_bwd_workspace_bytes(grid_b, grid_l, H) bytes, 16-aligned. */
int64_t tssm_layernorm_bwd_workspace_bytes(int64_t grid_b, int64_t grid_l, int64_t H);
int tssm_layernorm_bwd(int dtype, const void* dout, const void* x, const void* w, void* dx,
                       void* dw, void* db, int64_t nbatch, int64_t L, int64_t H, int64_t stride_b,
                       int64_t stride_l, float eps, int64_t block_h, int64_t grid_b,
                       int64_t grid_l, void* workspace, int64_t workspace_bytes, void* stream);

/* swiglu_kernel / swiglu_bwd_kernel (fused_ssm_interp.py:174-217): out =
 * silu(gate)*up; dup = dout*silu(gate), dgate = dout*up*sig*(1+gate*(1-sig)).
 * All tensors of a call share strides. */
int tssm_swiglu_fwd(int dtype, const void* gate, const void* up, void* out, int64_t nbatch,
                    int64_t L, int64_t H, int64_t stride_b, int64_t stride_l, int64_t grid_b,
                    int64_t grid_l, void* stream);
int tssm_swiglu_bwd(int dtype, const void* dout, const void* gate, const void* up, void* dgate,
                    void* dup, int64_t nbatch, int64_t L, int64_t H, int64_t stride_b,
                    int64_t stride_l, int64_t grid_b, int64_t grid_l, void* stream);

/* residual_add_kernel / dropout_residual_kernel (multihead_ssm_kernel.py:191-222)
 * over the first n elements (contiguous): out = x + res, or with a uint8 keep
 * mask out = x*keep/p_keep + res.  keep NULL: plain residual add. */
int tssm_residual_add(int dtype, const void* x, const void* res, const uint8_t* keep, void* out,
                      int64_t n, float p_keep, void* stream);

/* mean_pool_logit_kernel (streaming_inference_kernel.py:160-194): out[b] =
 * sum_{t,h} W[h] h[b,t,h] / (T*H + 1e-9) + bias[0] for b < grid_b; reduced
 * in a fixed order.  Workspace: tssm_mean_pool_logit_workspace_bytes(grid_b,
 * T) bytes. */
int64_t tssm_mean_pool_logit_workspace_bytes(int64_t grid_b, int64_t T);
int tssm_mean_pool_logit(int dtype, const void* h, const void* W, const void* bias, void* out,
                         int64_t nbatch, int64_t nt, int64_t H, int64_t stride_b,
                         int64_t stride_t, int64_t grid_b, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* masked_fill_zero_kernel (streaming_inference_kernel.py:198-214): out[i] =
 * mask[i / H] > 0 ? x[i] : 0 over the first n elements (contiguous [B,T,H],
 * mask [B,T]).  mask_code: 0 f32, 1 bf16, 2 f16, 3 int32, 4 uint8/bool. */
int tssm_masked_fill_zero(int dtype, int mask_code, const void* x, const void* mask, void* out,
                          int64_t n, int64_t H, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TSSM_H_ */

/*
 * kla_hip.h -- C ABI of libkla_hip.so, the MI355X (gfx950) scan kernels behind
 * the "hip" entry of the kla backend registry.
 *
 * Every entry point takes caller-owned device buffers (plain pointers), the
 * problem size and a HIP stream; it validates its arguments on the host,
 * launches on `stream` and returns without synchronising. Nothing here
 * allocates device memory. Status codes are the KLA_* values below; after a
 * non-zero status, kla_hip_last_error() describes it (thread-local string).
 *
 * Layout. A "sequence tensor" is a dense row-major [batch, steps, lanes] array:
 * lanes are contiguous, time stride = lanes, batch stride = steps*lanes. For the
 * reference's [B, L, M, S] scan operands this is lanes = M*S. A "state tensor"
 * is dense [batch, lanes].
 *
 * Workspace. The single-pass scans publish per-chunk carries to one another
 * through a caller-owned device workspace of kla_scan_workspace_bytes() bytes.
 * Zero-fill it ONCE when it is allocated; the kernels keep it consistent from
 * call to call (an epoch-tagged record scheme resets itself at the end of every
 * launch), so it must not be zeroed again between calls, and calls that share
 * one workspace must be ordered on one stream.
 *
 * Reference interfaces replaced (file:line in vaisakh-shaj/kalman-linear-attention):
 *   kla_mobius_scan_fwd  <- TiledMobiusScan.forward / tiled_mobius_lambda
 *                           (src/kla/ops/kernels/triton/tiled_mobius_scan.py:257-264, :113-151)
 *   kla_mobius_scan_bwd  <- TiledMobiusScan.backward
 *                           (src/kla/ops/kernels/triton/tiled_mobius_scan.py:266-279)
 *   kla_affine_scan_fwd  <- TiledAffineScan.forward / tiled_linear_eta
 *                           (src/kla/ops/kernels/triton/tiled_mobius_scan.py:282-289, :205-233)
 *   kla_affine_scan_bwd  <- TiledAffineScan.backward / _reverse_affine
 *                           (src/kla/ops/kernels/triton/tiled_mobius_scan.py:291-298, :247-254)
 *   kla_hip_last_error   <- the TORCH_CHECK messages of the CUDA binding
 *                           (src/kla/ops/kernels/cuda/v2_2/kla_matmul_scan.cu:35-59)
 */
#ifndef KLA_HIP_H_
#define KLA_HIP_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define KLA_OK 0
#define KLA_ERR_INVALID_ARG 1 /* null pointer, negative or oversized shape   */
#define KLA_ERR_WORKSPACE 2   /* workspace null, misaligned or too small     */
#define KLA_ERR_DTYPE 3       /* unsupported element type                    */
#define KLA_ERR_ALIGN 4       /* operand pointer not aligned to its element  */
#define KLA_ERR_HIP 5         /* the HIP runtime refused the launch          */

/* Element types of the affine scan's sequence tensors (state is always fp32). */
#define KLA_DTYPE_F32 0
#define KLA_DTYPE_BF16 1

/* Scan kinds, for kla_scan_workspace_bytes(). */
#define KLA_SCAN_MOBIUS_FWD 0
#define KLA_SCAN_MOBIUS_BWD 1
#define KLA_SCAN_AFFINE_FWD 2
#define KLA_SCAN_AFFINE_BWD 3

/* ABI version of this header; bumped on any signature change. */
int kla_hip_abi_version(void);

/* Message of the last non-zero status returned on the calling thread. */
const char *kla_hip_last_error(void);

/* Bytes of workspace a scan of this kind and size needs (0 on bad arguments). */
size_t kla_scan_workspace_bytes(int kind, int64_t batch, int64_t steps, int64_t lanes);

/* Kernels kla_set_kernel_events can bracket. */
#define KLA_KERNEL_FUSED_FWD 0 /* fused_kla_fwd_kernel (kla_fused_scan*_fwd)  */
#define KLA_KERNEL_FUSED_BWD 1 /* fused_kla_bwd_kernel (kla_fused_scan*_bwd)  */

/* Timing hook, no counterpart in the reference: for a benchmark that times one
 * kernel inside a larger step (the fused backward launches its scan kernel and
 * then the partial-sum reductions). Until called again with NULL events, every
 * launch of `kernel` in the process (from any host thread: torch's autograd
 * launches backwards from a thread of its own) records `start` on its stream
 * right before that kernel and `stop` right after it; hipEventElapsedTime of
 * the pair is then that kernel's duration (of the last launch recorded). Events
 * are the caller's; the hook holds no reference to them beyond the handles. */
int kla_set_kernel_events(int kernel, hipEvent_t start, hipEvent_t stop);

/* Number of look-back waits that gave up since the workspace was zero-filled
 * (0 in every correct run). Reads the workspace header: synchronises `stream`.
 * workspace NULL: the current device's static scratch of
 * kla_mobius_scan_fwd_noalloc (0 if no such call has run on the device). */
int kla_workspace_failures(const void *workspace, hipStream_t stream, uint32_t *failures);

/*
 * Moebius (2x2 linear-fractional) precision scan, forward.
 *   lam[b,t,n] = (A*l + B) / max(C*l + D, 1e-12),  l = lam[b,t-1,n], lam[b,-1,n] = lam0[b,n]
 * A, B, C, D, lam: sequence tensors (fp32). D may be NULL (D == 1).
 * lam0: state tensor (fp32) or NULL (lam0 == 1).
 * Replaces TiledMobiusScan.forward (tiled_mobius_scan.py:257-264).
 */
int kla_mobius_scan_fwd(const float *A, const float *B, const float *C, const float *D,
                        const float *lam0, float *lam, int64_t batch, int64_t steps,
                        int64_t lanes, void *workspace, size_t workspace_bytes,
                        hipStream_t stream);

/*
 * kla_mobius_scan_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. The look-back
 * records live in a static 32 MiB device array (one per GPU, held until the
 * process ends), which fits the scan up to (8, 4096, 2048); a larger call
 * returns KLA_ERR_WORKSPACE and launches nothing. The first call on a device
 * looks the array up, zero-fills it on `stream` and waits for the fill (so make
 * that first call outside a graph capture); the call itself allocates nothing.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on
 * one GPU race. Their results are undefined: the bounded look-back waits still
 * end, but a workgroup whose ticket falls outside its own launch writes nothing,
 * so parts of lam can be left unwritten rather than NaN. A look-back wait that
 * gives up writes NaN and is counted: kla_workspace_failures(NULL, ...) reads the
 * count. Results are bit-identical to kla_mobius_scan_fwd's.
 */
int kla_mobius_scan_fwd_noalloc(const float *A, const float *B, const float *C, const float *D,
                                const float *lam0, float *lam, int64_t batch, int64_t steps,
                                int64_t lanes, hipStream_t stream);

/*
 * Moebius scan, exact scalar-adjoint backward.
 *   den_t = max(C_t*l_{t-1} + D_t, 1e-12), gain_t = (A_t*D_t - B_t*C_t) / den_t^2
 *   nu_t = dlam_t + gain_{t+1}*nu_{t+1}          (reverse scan, nu_T = 0)
 *   dA = nu*l_{t-1}/den, dB = nu/den, dC = -nu*l_t*l_{t-1}/den, dD = -nu*l_t/den
 *   dlam0 = nu_0*gain_0
 * lam: the forward's output. It is read only where a thread's block of steps
 * begins (one row in 24); the values in between are recomputed from A, B, C, D
 * with the forward's own step, which reproduces the forward's lam bit for bit,
 * so lam must be exactly what kla_mobius_scan_fwd wrote for these inputs.
 * D, dD, lam0, dlam0 may be NULL (dD is written only
 * when both D and dD are given); dA, dB, dC may be NULL to skip that output.
 * Replaces TiledMobiusScan.backward (tiled_mobius_scan.py:266-279).
 */
int kla_mobius_scan_bwd(const float *dlam, const float *A, const float *B, const float *C,
                        const float *D, const float *lam0, const float *lam, float *dA,
                        float *dB, float *dC, float *dD, float *dlam0, int64_t batch,
                        int64_t steps, int64_t lanes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/*
 * Affine (first-order linear) scan, forward: h_t = g_t*h_{t-1} + u_t, h_{-1} = h0.
 * g, u, h: sequence tensors of `dtype` (KLA_DTYPE_F32 or KLA_DTYPE_BF16; fp32
 * arithmetic, bf16 stored round-to-nearest-even). h0: fp32 state tensor or NULL (0).
 * Replaces TiledAffineScan.forward (tiled_mobius_scan.py:282-289).
 */
int kla_affine_scan_fwd(int dtype, const void *g, const void *u, const float *h0, void *h,
                        int64_t batch, int64_t steps, int64_t lanes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/*
 * Affine scan, exact backward.
 *   mu_t = dh_t + g_{t+1}*mu_{t+1} (reverse, mu_T = 0), dg_t = mu_t*h_{t-1}, du_t = mu_t,
 *   dh0 = g_0*mu_0.
 * dh, g, h (the forward's output), dg, du: sequence tensors of `dtype`.
 * h0, dh0: fp32 state tensors or NULL; dg, du may be NULL to skip that output.
 * Replaces TiledAffineScan.backward (tiled_mobius_scan.py:291-298).
 */
int kla_affine_scan_bwd(int dtype, const void *dh, const void *g, const void *h,
                        const float *h0, void *dg, void *du, float *dh0, int64_t batch,
                        int64_t steps, int64_t lanes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/*
 * Fused KLA scan: the whole filter of kla_scan_torch in one kernel per direction.
 * Shapes (reference kla_ops.py:23-28): v, lambda_v, y, y_var [batch, steps, M];
 * k, q [batch, steps, S]; a, p [M, S]; lam0, eta0, lam_fin, eta_fin [batch, M, S];
 * all fp32, dense. S <= 256. lam0 / eta0 may be NULL (precision 1, information 0).
 *   phi = lambda_v k^2, r = (v lambda_v) k, a2 = max(a^2, 1e-12), p' = max(p, 1e-12)
 *   lam_t = (A lam_{t-1} + phi) / (C lam_{t-1} + 1), A = (1 + p' phi)/a2, C = p'/a2
 *   eta_t = a / max(a2 + p' lam_{t-1}, 1e-12) * eta_{t-1} + r
 *   var = 1/max(lam_t, 1e-12), mean = eta_t var (decode_from_prior: mean = a mean,
 *   var = a2 var + p'); y = sum_s q mean, y_var = sum_s q^2 var.
 * ck_lam / ck_eta: [batch, kla_fused_checkpoints(steps), M, S] buffers the forward
 * fills for the backward, or both NULL when no backward will follow.
 * y_var may be NULL: the variance read-out is then skipped (a cheaper kernel).
 * Replaces kla_scan_torch (src/kla/ops/kla_ops.py:188-290) / the fused kernels
 * (src/kla/ops/kernels/cuda/v2_2/kla_matmul_fwd_kernel.cuh:89-476,
 * src/kla/ops/kernels/mps/fused_kla_scan.metal:53-131).
 */
int64_t kla_fused_checkpoints(int64_t steps);

int kla_fused_scan_fwd(const float *v, const float *lambda_v, const float *k, const float *q,
                       const float *a, const float *p, const float *lam0, const float *eta0, float *y,
                       float *y_var, float *lam_fin, float *eta_fin, float *ck_lam, float *ck_eta,
                       int decode_from_prior, int64_t batch, int64_t steps, int64_t M, int64_t S,
                       hipStream_t stream);

/* Bytes of workspace kla_fused_scan_bwd needs (partial sums; no zero-fill needed). */
size_t kla_fused_workspace_bytes(int64_t batch, int64_t steps, int64_t M, int64_t S);

/*
 * Exact adjoint of kla_fused_scan_fwd (checkpoint replay). Inputs: the output
 * gradients dy and (optional, NULL = 0) dy_var, dlam_fin, deta_fin, the forward's
 * inputs and its checkpoints. Outputs: dv, dlambda_v [batch, steps, M]; dk, dq
 * [batch, steps, S]; da, dp [M, S]; dlam0, deta0 [batch, M, S] (NULL to skip).
 * Every output is written (not accumulated); sums over channels and batch run in
 * a fixed order, so results are deterministic.
 * Replaces the exact fused backward (src/kla/ops/kernels/mps/fused_kla_scan.metal:135-324)
 * and the CUDA backward (kla_matmul_bwd_kernel.cuh:156-800), whose adjoint is approximate.
 */
int kla_fused_scan_bwd(const float *dy, const float *dy_var, const float *dlam_fin, const float *deta_fin,
                       const float *v, const float *lambda_v, const float *k, const float *q,
                       const float *a, const float *p, const float *ck_lam, const float *ck_eta,
                       float *dv, float *dlambda_v, float *dk, float *dq, float *da, float *dp,
                       float *dlam0, float *deta0, int decode_from_prior, int64_t batch, int64_t steps,
                       int64_t M, int64_t S, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/*
 * The fused scan's sensor inputs as a KLALayer holds them. v and the precision
 * operand `obs` are [batch, steps, M] with rows ld_v / ld_obs elements apart:
 * element (b, t, m) at (b * steps + t) * ld + m, so they may be column slices of
 * the sensor projection. dtype is KLA_DTYPE_F32 or KLA_DTYPE_BF16 (both operands).
 * With log_var = 1, obs holds log sigma^2 and the kernels form
 *   lambda_v = 1 / min(softplus(log sigma^2) + obs_var_min, obs_var_max)
 * (softplus with torch's threshold 20; obs_var_max = +inf for none), which is the
 * tail of KLALayer._project_sensors (reference src/kla/layers/kla_layer.py:224-230).
 * With log_var = 0, obs is lambda_v itself.
 */
typedef struct kla_sensors {
  const void *v;
  int64_t ld_v;
  const void *obs;
  int64_t ld_obs;
  int dtype;
  int log_var;
  float obs_var_min;
  float obs_var_max;
} kla_sensors;

/*
 * kla_fused_scan_fwd with the sensors read as described by `sensors` (the
 * projection read-out and lambda_v formed in the kernel, never stored).
 * Replaces _project_sensors' v / lambda_v tail plus kla_scan_torch
 * (reference src/kla/layers/kla_layer.py:194-231, src/kla/ops/kla_ops.py:188-290).
 */
int kla_fused_scan_sensors_fwd(const kla_sensors *sensors, const float *k, const float *q, const float *a,
                               const float *p, const float *lam0, const float *eta0, float *y, float *y_var,
                               float *lam_fin, float *eta_fin, float *ck_lam, float *ck_eta,
                               int decode_from_prior, int64_t batch, int64_t steps, int64_t M, int64_t S,
                               hipStream_t stream);

/*
 * Exact adjoint of kla_fused_scan_sensors_fwd. dv and dobs are dense
 * [batch, steps, M] of the sensors' dtype (bf16: rounded to nearest even, as
 * autograd's cast back to the projection's dtype rounds); dobs is the gradient
 * of log sigma^2 (log_var, through the reciprocal, the clamp and softplus as torch
 * differentiates them) or of lambda_v. Everything else as kla_fused_scan_bwd;
 * the workspace is kla_fused_workspace_bytes.
 */
int kla_fused_scan_sensors_bwd(const float *dy, const float *dy_var, const float *dlam_fin,
                               const float *deta_fin, const kla_sensors *sensors, const float *k,
                               const float *q, const float *a, const float *p, const float *ck_lam,
                               const float *ck_eta, void *dv, void *dobs, float *dk, float *dq, float *da,
                               float *dp, float *dlam0, float *deta0, int decode_from_prior, int64_t batch,
                               int64_t steps, int64_t M, int64_t S, void *workspace, size_t workspace_bytes,
                               hipStream_t stream);

/*
 * The time-split forward of the fused scan (inference: no checkpoints, no
 * backward), for problems with too few chains (batch * M * S) to fill the GPU.
 * The sequence is cut into `chunks` equal pieces; a [B, L, .] tensor viewed as
 * [B * chunks, L / chunks, .] is the same memory (sequence b's chunk c at
 * b' = b * chunks + c). Three calls:
 *   kla_fused_chunk_maps on the view (batch = B * chunks, steps = L / chunks):
 *     each chunk's steps composed into one map of the state in homogeneous
 *     coordinates (lam = N / D, eta = W / D, where a filter step is linear),
 *     maps [B * chunks, M, S, 8] (n0 n1 d0 d1 w0 w1 w2, one word unused);
 *   kla_chunk_starts (batch = B, chunks): the state entering each chunk,
 *     lam_start, eta_start [B, chunks, M, S], from lam0 (NULL: 1) and eta0
 *     (NULL: 0) through the maps in chunk order, and (lam_end, eta_end, both
 *     or neither) the state after the last chunk, [B, M, S];
 *   kla_fused_scan_sensors_fwd on the view with lam0 / eta0 = the starts: y,
 *     y_var (its final-state outputs are those of every chunk, [B * chunks, M, S]).
 * The sensors are as for kla_fused_scan_sensors_fwd. The chunked forward of the
 * reference's tiled Metal kernel (src/kla/ops/kernels/mps/tiled_kla_scan.metal:1-35,
 * tiled_kla_scan.py:32-60), which composes the precision and the information
 * leaves in two rounds; with kla_fused_scan_sensors_fwd it replaces
 * kla_scan_torch's forward (src/kla/ops/kla_ops.py:188-290).
 */
int kla_fused_chunk_maps(const kla_sensors *sensors, const float *k, const float *a, const float *p, float *maps,
                         int64_t batch, int64_t steps, int64_t M, int64_t S, hipStream_t stream);
int kla_chunk_starts(const float *maps, const float *lam0, const float *eta0, float *lam_start, float *eta_start,
                     float *lam_end, float *eta_end, int64_t batch, int64_t chunks, int64_t M, int64_t S,
                     hipStream_t stream);

/*
 * The time-split backward of the fused scan (training at small batch), the
 * adjoint of the time-split forward: the forward's checkpoints are the same
 * memory on the [B * chunks, L / chunks] view (chunks of a multiple of 16
 * steps). The adjoint of the state (lam_t, eta_t) walks back through an affine
 * map with an upper-triangular linear part per step, so each chunk's steps
 * compose into five numbers per lane. Three calls:
 *   kla_fused_adjoint_maps on the view (batch = B * chunks, steps = L / chunks),
 *     with the backward's dy, dy_var (NULL: no y_var gradient), sensors, k, q,
 *     a, p and checkpoints: maps [B * chunks, M, S, 8] (P Q A u_l u_e, three words
 *     unused), x -> [[P, Q], [0, A]] x + (u_l, u_e) for the adjoint x entering a
 *     chunk from its end;
 *   kla_adjoint_ends (batch = B, chunks): from dlam_fin, deta_fin (NULL: 0)
 *     through the maps in reverse chunk order, the adjoint entering each chunk
 *     from its end, gl_end, ge_end [B, chunks, M, S];
 *   kla_fused_scan_sensors_bwd (or kla_fused_scan_bwd) on the view with
 *     dlam_fin, deta_fin = gl_end, ge_end: every gradient; da, dp summed over
 *     all chunks; the initial-state gradients are chunk 0's, [B * chunks, M, S]
 *     rows b * chunks.
 * The chunked backward of the reference's tiled Metal kernel has no
 * counterpart here (its backward runs through torch autograd,
 * src/kla/ops/mps_backend.py:10-16); with kla_fused_scan_sensors_bwd these
 * replace kla_scan_torch's backward (src/kla/ops/kla_ops.py:188-290).
 */
int kla_fused_adjoint_maps(const float *dy, const float *dy_var, const kla_sensors *sensors, const float *k,
                           const float *q, const float *a, const float *p, const float *ck_lam, const float *ck_eta,
                           float *maps, int decode_from_prior, int64_t batch, int64_t steps, int64_t M, int64_t S,
                           hipStream_t stream);
int kla_adjoint_ends(const float *maps, const float *dlam_fin, const float *deta_fin, float *gl_end, float *ge_end,
                     int64_t batch, int64_t chunks, int64_t M, int64_t S, hipStream_t stream);

/*
 * One O(1) decode step of the filter for every (b, m, s) lane: kla_step
 * (reference src/kla/ops/kla_ops.py:293-331), phi floored at 1e-12 as there.
 * v, lambda_v, y, y_var [batch, M]; k, q [batch, S]; a, p [M, S]; lam, eta,
 * lam_out, eta_out [batch, M, S] (lam_out / eta_out may alias lam / eta). No gradient.
 */
int kla_step_fwd(const float *v, const float *lambda_v, const float *k, const float *q, const float *a,
                 const float *p, const float *lam, const float *eta, float *y, float *y_var, float *lam_out,
                 float *eta_out, int decode_from_prior, int64_t batch, int64_t M, int64_t S, hipStream_t stream);

/*
 * Options of the layer decode step, from KLAConfig (reference configs.py:45-222).
 */
typedef struct kla_decode_config {
  int discretization;     /* 0 = "ou", 1 = "zoh" (kla_layer.py:172-181)                         */
  int zero_process_noise; /* p + 1e-12 instead of max(p, 1e-7) (kla_layer.py:164-170)           */
  int qk_norm;            /* k, q divided by max(||.||_2, 1e-12) over the S states             */
  int has_clip;           /* clip_value set: p <= clip, k and q clamped to [-clip, clip]       */
  float clip_value;
  float obs_var_min;      /* obs_var = softplus(log_var) + obs_var_min                         */
  float obs_var_max;      /* obs_var clamped above by it; +inf when unset                      */
  int decode_from_prior;  /* read out the one-step prior (kla_ops.py:325-328)                   */
  int gate_activation;    /* with a gate: 1 silu, 2 gelu, 3 relu                                */
  int skip_vector;        /* lambda_skip is [M] (1) or a scalar (0)                             */
} kla_decode_config;

/*
 * The whole one-token SSM step of a KLALayer, for inference (fp32, no gradient):
 * replaces KLALayer._run_ssm_step with _compute_aq / _continuous_params /
 * _discretize, the tail of _project_sensors and the lambda-skip and gating lines
 * of forward (reference src/kla/layers/kla_layer.py:164-190, :194-231, :277-293,
 * :295-349), i.e. ~30 torch kernels per layer and token, as one kernel.
 *   (a_bar, p_bar) from delta, lambda_log, process_noise [M, S] (recomputed per call);
 *   k, q [batch, S] rows (stride ld_kq), l2-normalised / clipped per cfg;
 *   Lambda^v = 1 / min(softplus(log_var) + obs_var_min, obs_var_max), log_var and v
 *   [batch, M] rows (strides ld_log_var, ld_v);
 *   the kla_step update of lam, eta [batch, M, S] into lam_out, eta_out (may alias);
 *   y = sum_s q mean (+ lambda_skip * residual), y_var = sum_s q^2 var, both times
 *   act(gate) resp. act(gate)^2 when gate is given. residual and lambda_skip come
 *   together or not at all. y, y_var are dense [batch, M].
 */
int kla_decode_step_fwd(const float *v, int64_t ld_v, const float *log_var, int64_t ld_log_var, const float *k,
                        const float *q, int64_t ld_kq, const float *residual, int64_t ld_residual,
                        const float *lambda_skip, const float *gate, int64_t ld_gate, const float *delta,
                        const float *lambda_log, const float *process_noise, const float *lam, const float *eta,
                        float *lam_out, float *eta_out, float *y, float *y_var, const kla_decode_config *cfg,
                        int64_t batch, int64_t M, int64_t S, hipStream_t stream);

/*
 * One token of the depthwise causal conv with its window state: replaces the
 * one-token path of CausalConv1d.forward (reference src/kla/layers/common.py:70-96).
 *   window = [state[b, c, 0 : K-1], x[b, c]] (x rows of stride ld_x),
 *   y[b, c] = act(sum_j weight[c, j] window[j] + bias[c]), state_out = window[1 : K];
 *   weight [channels, K], bias [channels] or NULL, state / state_out [batch, channels, K-1]
 *   (may alias), activation 0 none, 1 silu, 2 gelu, 3 relu. fp32.
 */
int kla_conv_step_fwd(const float *x, int64_t ld_x, const float *state, float *state_out, const float *weight,
                      const float *bias, int activation, float *y, int64_t batch, int64_t channels,
                      int64_t kernel_size, hipStream_t stream);

/*
 * The layer's short depthwise causal conv over a sequence, with autograd's
 * backward: replaces CausalConv1d.forward for L >= 1 (reference
 * src/kla/layers/common.py:58-96: transpose, torch.cat of the state in front,
 * F.conv1d(groups=D), activation) and its backward through autograd.
 *   xpad = [state (K-1), x (steps)] per (b, c); y[b, t, c] = act(bias[c] + sum_j w[c, j] xpad[t + j]);
 *   state_out = xpad[steps : steps + K - 1].
 * x [batch, steps, channels] with element strides ld_t (time) and ld_b (batch),
 * channels contiguous; y dense [batch, steps, channels]; state, state_out
 * [batch, channels, K-1] (state NULL = zeros, state_out NULL = not wanted);
 * weight [channels, K] fp32, bias [channels] fp32 or NULL; K <= 8; activation
 * 0 none, 1 silu, 2 gelu, 3 relu. dtype KLA_DTYPE_F32 or KLA_DTYPE_BF16 for x,
 * y and the states; with bf16 the weight and bias are rounded to bf16 and the
 * conv output is rounded before the activation (torch autocast's numerics).
 */
int kla_causal_conv_fwd(int dtype, const void *x, int64_t ld_t, int64_t ld_b, const void *state, const float *weight,
                        const float *bias, int activation, void *y, void *state_out, int64_t batch, int64_t steps,
                        int64_t channels, int64_t kernel_size, hipStream_t stream);

/* Bytes of workspace kla_causal_conv_bwd needs (partial sums; no zero-fill needed). */
size_t kla_causal_conv_workspace_bytes(int64_t batch, int64_t steps, int64_t channels, int64_t kernel_size);

/*
 * Exact adjoint of kla_causal_conv_fwd given dy (gradient of y, dense) and
 * optionally dstate_out (gradient of state_out, NULL = 0): dx (dense
 * [batch, steps, channels]), dstate (NULL to skip), dweight [channels, K] and
 * dbias [channels] (fp32; dbias may be NULL when bias is). Weight and bias
 * gradients are summed in a fixed order (deterministic).
 */
int kla_causal_conv_bwd(int dtype, const void *dy, const void *x, int64_t ld_t, int64_t ld_b, const void *state,
                        const float *weight, const float *bias, int activation, const void *dstate_out, void *dx,
                        void *dstate, float *dweight, float *dbias, int64_t batch, int64_t steps, int64_t channels,
                        int64_t kernel_size, void *workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * The KLALayer output tail after the scan (reference src/kla/layers/kla_layer.py:333-337):
 *   t = y + lambda_skip * residual,  out = t * act(gate)
 * y, dy: fp32 [rows, M] dense. out, dout: [rows, M] dense of `out_dtype`
 * (KLA_DTYPE_F32, or KLA_DTYPE_BF16 where the consumer of out -- the output
 * projection under autocast -- rounds it to bf16 anyway). residual, gate:
 * [rows, M] of `dtype` (KLA_DTYPE_F32 or KLA_DTYPE_BF16) with rows ld_res /
 * ld_gate elements apart, or NULL when the layer has no skip / no gate.
 * lambda_skip: fp32 [M] (lambda_vector = 1) or one value (0-dim: with bf16
 * residuals lambda * residual is rounded to bf16, as torch's type promotion
 * leaves it). activation: 0 none, 1 silu, 2 gelu, 3 relu; act(gate) is rounded
 * to `dtype`.
 */
int kla_gate_skip_fwd(int dtype, int out_dtype, const float *y, const void *residual, int64_t ld_res,
                      const void *gate, int64_t ld_gate, const float *lambda_skip, int lambda_vector, int activation,
                      void *out, int64_t rows, int64_t M, hipStream_t stream);

/* Bytes of workspace kla_gate_skip_bwd needs (column partial sums; no zero-fill needed). */
size_t kla_gate_skip_workspace_bytes(int64_t rows, int64_t M);

/*
 * Backward of kla_gate_skip_fwd, with torch autograd's roundings: dy (fp32),
 * dres and dgate (dense [rows, M] of `dtype`, NULL to skip), dlambda ([M], or one
 * value for a 0-dim lambda, summed in a fixed order; required with a residual).
 * Replaces the autograd backward of those lines (MulBackward0, AddBackward0 and
 * the activation's backward).
 */
int kla_gate_skip_bwd(int dtype, int out_dtype, const void *dout, const float *y, const void *residual,
                      int64_t ld_res, const void *gate, int64_t ld_gate, const float *lambda_skip, int lambda_vector,
                      int activation, float *dy, void *dres, void *dgate, float *dlambda, int64_t rows, int64_t M,
                      void *workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Inference kernels of the sequence model around the KLA layers (no gradient):
 * RMSNorm, y = ((x * rsqrt(mean(x^2) + eps)) * weight) in x's dtype, over rows
 * of `dim` (x, y dense [rows, dim] of `dtype`, weight fp32 [dim]); replaces
 * RMSNorm.forward (reference src/kla/layers/common.py:45-55).
 */
int kla_rms_norm_fwd(int dtype, const void *x, const float *weight, float eps, void *y, int64_t rows, int64_t dim,
                     hipStream_t stream);

/*
 * SwiGLU activation: out = silu(h[:, :hidden]) * h[:, hidden:2 hidden] (h rows
 * ld_h elements apart, out dense [rows, hidden], both of `dtype`); replaces the
 * `F.silu(gate) * up` of MLP.forward (reference src/kla/layers/common.py:120-123).
 */
int kla_swiglu_fwd(int dtype, const void *h, int64_t ld_h, void *out, int64_t rows, int64_t hidden,
                   hipStream_t stream);

/*
 * Embedding rows of one decode step: out[r, :] = table[ids[r], :] for r < rows
 * (table rows ld_table elements apart, vocab of them; out rows ld_out apart;
 * both of `dtype`, ids int64). An id outside [0, vocab) reads nothing and
 * writes a row of NaN. Replaces nn.Embedding in SequenceModel.forward
 * (reference src/kla/models/sequence_model.py:157) for a one-token step.
 */
int kla_gather_rows(int dtype, const void *table, int64_t ld_table, int64_t vocab, const int64_t *ids, void *out,
                    int64_t ld_out, int64_t rows, int64_t dim, hipStream_t stream);

/*
 * Greedy token choice: out[r * ld_out] = argmax_j x[r, j] over n > 0 fp32 values
 * (rows ldx apart), in torch.argmax's order: NaN above every number, ties to
 * the smaller index. Replaces logits.argmax(dim=-1) of SequenceModel._sample
 * with temperature 0 (reference src/kla/models/sequence_model.py, generate).
 */
int kla_argmax_rows(const float *x, int64_t ldx, int64_t rows, int64_t n, int64_t *out, int64_t ld_out,
                    void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes with which kla_argmax_rows splits each row over several
 * workgroups (with a smaller or NULL workspace it runs one workgroup per row). */
size_t kla_argmax_workspace_bytes(int64_t rows, int64_t n);

/*
 * A KLA layer's static dynamics over n = M * S elements, fp32
 * (KLALayer._compute_aq, reference src/kla/layers/kla_layer.py:164-190):
 *   a = -exp(lambda_log);  p = pnoise + 1e-12 (zero_process_noise) or min(max(pnoise, 1e-7), clip)
 *   d = softplus(delta) + 1e-7;  a_bar = exp(d a)
 *   ou: p_bar = (p / (2 rate)) (-expm1(-2 rate d)), rate = max(|a|, 1e-8);  else p_bar = p d
 * has_clip: whether clip applies. The backward takes the gradients of a_bar and
 * p_bar (either may be NULL: zero) and writes those of delta, lambda_log and pnoise.
 */
int kla_discretize_fwd(const float *delta, const float *lambda_log, const float *pnoise, int64_t n, int ou,
                       int zero_process_noise, int has_clip, float clip, float *a_bar, float *p_bar,
                       hipStream_t stream);
int kla_discretize_bwd(const float *delta, const float *lambda_log, const float *pnoise, int64_t n, int ou,
                       int zero_process_noise, int has_clip, float clip, const float *g_a_bar, const float *g_p_bar,
                       float *d_delta, float *d_lambda_log, float *d_pnoise, hipStream_t stream);

/*
 * The k and q sensors of a KLA layer (KLALayer._project_sensors_raw, reference
 * src/kla/layers/kla_layer.py:194-231): per row of S values,
 *   y = clamp(l2_norm(x), -clip, clip) in fp32,  l2_norm(x) = x / max(||x||_2, 1e-12)
 * (norm: whether to normalise; has_clip: whether to clip), rounding to `dtype`
 * after each operation as torch does for that dtype. k, q: [rows, S] of `dtype`
 * with rows ld_k / ld_q elements apart (column slices of the sensor
 * projection); yk, yq: [rows, S] dense fp32. The backward takes the gradients of
 * yk, yq ([rows, S] dense fp32) and writes dk, dq ([rows, S] dense, `dtype`)
 * through torch's autograd chain of the same operations.
 */
int kla_qk_sensors_fwd(int dtype, const void *k, int64_t ld_k, const void *q, int64_t ld_q, float *yk, float *yq,
                       int64_t rows, int64_t S, int norm, int has_clip, float clip, hipStream_t stream);
int kla_qk_sensors_bwd(int dtype, const void *k, int64_t ld_k, const void *q, int64_t ld_q, const float *dyk,
                       const float *dyq, void *dk, void *dq, int64_t rows, int64_t S, int norm, int has_clip,
                       float clip, hipStream_t stream);

/*
 * out[r, :] = [piece_0[r, :], ..., piece_{n-1}[r, :]]: dense out [rows, sum of
 * widths] of `dtype` from n <= 4 pieces, piece i rows of widths[i] elements
 * ld[i] apart (pieces[i] NULL: zeros). The backward of splitting a projection's
 * last dimension (torch.split / chunk in KLALayer, reference
 * src/kla/layers/kla_layer.py:206, :313-316): autograd's concatenation of the
 * pieces' gradients.
 */
int kla_cat_cols(int dtype, int n, const void *const *pieces, const int64_t *ld, const int64_t *widths, void *out,
                 int64_t rows, hipStream_t stream);

/*
 * out[i] = sum_{j < nparts} parts[j * n + i] for i < n: fp32 partials added in
 * j order, rounded once to `dtype` (fp32 or bf16, round to nearest even). The
 * last step of a projection's weight gradient split over the token dimension
 * (dW = sum over token chunks of dY_c^T X_c, each chunk's product an fp32
 * batched GEMM): it replaces the single weight-gradient product of torch's
 * nn.Linear backward for KLALayer's in_proj, sensor_proj and out_proj
 * (reference src/kla/layers/kla_layer.py:61, :88, :127), whose few output
 * tiles leave most CUs idle over a 16384-token reduction.
 */
int kla_sum_parts(int dtype, const float *parts, int64_t nparts, int64_t n, void *out, hipStream_t stream);

/* Epilogues of kla_rows_linear_fwd. */
enum { KLA_ROWS_PLAIN = 0, KLA_ROWS_RESIDUAL = 1, KLA_ROWS_SWIGLU = 2 };

/*
 * A linear layer on a few rows (one-token decode: rows = batch), fp32, with
 * the block's norm and residual or the MLP's activation fused in:
 *   xn  = norm_w ? (x * rsqrt(mean(x^2) + eps)) * norm_w : x      (per row of k)
 *   acc = xn W^T + bias                 W [n_w, k] rows ldw apart, bias [n_w] or NULL
 *   y   = acc                               (KLA_ROWS_PLAIN)
 *         res + acc                         (KLA_ROWS_RESIDUAL, res [rows, n])
 *         silu(acc[:, j]) * acc[:, glu_off + j]  (KLA_ROWS_SWIGLU, j < n)
 * x [rows, k] (ldx), y [rows, n] (ldy), res (ldres). W must hold n rows (n +
 * glu_off for KLA_ROWS_SWIGLU). No gradient; deterministic (fixed-order sums).
 * Replaces, in decode, the nn.Linear calls of KLALayer (in_proj, sensor_proj,
 * out_proj; reference src/kla/layers/kla_layer.py:61, :88, :127, :311, :340),
 * RMSNorm.forward before them (src/kla/layers/common.py:45-55), the block's
 * residual adds (src/kla/models/sequence_model.py:71-87), MLP.forward
 * (common.py:99-123) and the LM head on the final norm (sequence_model.py:169).
 */
int kla_rows_linear_fwd(int epilogue, const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                        const float *norm_w, float eps, const float *res, int64_t ldres, float *y, int64_t ldy,
                        int64_t rows, int64_t n, int64_t k, int64_t glu_off, hipStream_t stream);

/*
 * The k and q sensors of a sequence from the sensor projection's last 2 S rows
 * w [2 S, k] (row stride ldw), bias [2 S] or NULL, for fp32 x [rows, k] (row
 * stride ldx): a = x w^T + bias, k_out[r, :] = a[r, :S], q_out[r, :] = a[r, S:],
 * each row divided by max(||row||_2, 1e-12) when norm, then clamped to
 * [-clip, clip] when has_clip; k_out and q_out [rows, S] dense fp32. S is a power
 * of two in [1, 16]. Replaces the k, q columns of sensor_proj followed by
 * l2_norm and clamp (reference src/kla/layers/kla_layer.py:205-222).
 */
int kla_rows_linear_qk_fwd(const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                           float *k_out, float *q_out, int64_t rows, int64_t k, int64_t S, int norm, int has_clip,
                           float clip, hipStream_t stream);

/*
 * kla_rows_linear_fwd's plain product (same x, w, bias, norm_w, eps, y, rows, n,
 * k) with one token of the depthwise causal conv applied to output columns
 * j < conv_n (in_proj's z half in one-token decode):
 *   y[r, j] = act(sum_{i < conv_k-1} conv_w[j, i] window[r, j, i] + conv_w[j, conv_k-1] a[r, j] + conv_b[j])
 *   window_out[r, j, :] = (window[r, j, 1:], a[r, j])
 * with a the product (plus bias); columns j >= conv_n are y = a. conv_w
 * [conv_n, conv_k] dense, conv_b [conv_n] or NULL, window and window_out
 * [rows, conv_n, conv_k - 1] dense fp32 (window_out may alias window), conv_k
 * in [1, 8], activation 0 identity, 1 silu, 2 gelu (exact erf), 3 relu.
 * Replaces, in decode, in_proj followed by the one-token path of
 * CausalConv1d.forward (reference src/kla/layers/kla_layer.py:311-316,
 * src/kla/layers/common.py:70-96).
 */
int kla_rows_linear_conv_fwd(const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                             const float *norm_w, float eps, float *y, int64_t ldy, int64_t rows, int64_t n,
                             int64_t k, const float *conv_w, const float *conv_b, const float *window,
                             float *window_out, int64_t conv_n, int conv_k, int activation, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KLA_HIP_H_ */

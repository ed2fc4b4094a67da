/*
 * mogt_scan.h — C ABI of the MI355X (gfx950) MOGT scan operator.
 *
 * Plain C: device pointers, sizes, dtype codes and an opaque HIP stream
 * (hipStream_t passed as void*; NULL = the null stream).  No torch types.
 *
 * Conventions shared by every entry point
 *   - Tensors are contiguous row-major device buffers in the layouts named
 *     below (the reference's layouts: U [B,L,R,R], V/H [B,L,R,C]).
 *   - Arithmetic and carried state are fp32; I/O may be fp32 or bf16 (the
 *     generic affine scan also carries an fp64 state and reads / writes fp16
 *     and fp64).
 *   - Work is enqueued on `stream`; calls are asynchronous.
 *   - Return 0 on success, a negative MOGT_E* code on failure; the message is
 *     kept per thread and read with mogt_last_error().
 *   - Nothing here allocates or frees device memory.  Single-pass scans take a
 *     caller-owned `workspace` of at least *_workspace_bytes(...) bytes.  It
 *     must be zero-filled before its FIRST use; each launch leaves it ready for
 *     the next one (no per-call clearing).  Launches that may run concurrently
 *     (different streams) must use different workspaces.
 */
#ifndef MOGT_SCAN_H
#define MOGT_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define MOGT_F32 0
#define MOGT_BF16 1
#define MOGT_F64 2  /* mogt_affine_scan_generic_fwd only */
#define MOGT_F16 3  /* mogt_affine_scan_generic_fwd only */

/* error codes */
#define MOGT_OK 0
#define MOGT_E_INVALID -1   /* bad shape / dtype / argument (reference: ValueError) */
#define MOGT_E_WORKSPACE -2 /* workspace missing or too small */
#define MOGT_E_LAUNCH -3    /* HIP launch error */

/* Last error message of the calling thread ("" if none). */
const char* mogt_last_error(void);

/* ABI version of the loaded library (bumped on incompatible changes). */
int mogt_abi_version(void);

/* Build identity: "name:hash;name:hash;..." — a 12-hex-digit SHA-256 prefix
 * of every source file the library was compiled from (the .hip and .h files
 * of csrc/ and this header) and of the compiler flags (name "flags").  Profiles of a
 * kernel record the hashes of the sources behind it, so a measurement can be
 * matched to the build it came from.  No counterpart in the reference (its
 * kernels are JIT-compiled by Triton from the Python source).              */
const char* mogt_build_manifest(void);

/* Health of a single-pass scan workspace (the diag, coupled and reverse
 * scans' look-back buffer): *count receives the number of bounded waits that
 * gave up in launches on it since it was zero-filled.  It must be 0; a
 * look-back that gives up also writes NaN into its chunk's carry, so the
 * outputs it affected are visibly invalid.  Copies 4 bytes on `stream` and
 * waits for the stream (a debugging / checked-mode query).  The reference has
 * no counterpart: its scans (triton_scan.py:232-311) have no cross-block
 * protocol that could fail.                                                 */
int mogt_workspace_faults(const void* workspace, size_t workspace_bytes, uint32_t* count,
                          void* stream);

/* ------------------------------------------------------------------------- */
/* Diagonal affine scan  h_t = a_t * h_{t-1} + b_t,  h_0 = 0, per feature.
 *
 * Replaces affine_scan_sequential (affine_scan.py:14-62) in the folded R=C=1
 * mapping U=a.transpose(1,2).reshape(B*D,L,1,1) that the reference would need
 * for a per-feature scan, without the fold: a, b, h are [B, L, D].
 * `a_prefix` (nullable) receives prod_{s<=t} a_s, the R=1 case of the
 * reference's return_prefix=True U_prefix output (affine_scan.py:43-55).
 * in_dtype applies to a and b; out_dtype to h and a_prefix.               */
size_t mogt_diag_scan_workspace_bytes(int64_t batch, int64_t length, int64_t features,
                                      int in_dtype);
int mogt_diag_scan_fwd(const void* a, const void* b, void* h, void* a_prefix,
                       int64_t batch, int64_t length, int64_t features,
                       int in_dtype, int out_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Same with an explicit tile configuration, for tuning: `vec` features per
 * lane, `lanes` lanes per row (64, 32 or 16; a row of the chunk is one vector
 * load of `lanes` lanes, so a wave covers 64/lanes rows at once), `steps` steps
 * per lane, `waves` waves per work-group.  A chunk covers lanes*vec features
 * and steps*waves*64/lanes steps.  The workspace query takes the same tile.
 * mogt_diag_scan_tiles lists the compiled tiles of a family (0: fp32 input,
 * 1: bf16 input, 2: coupled scan, 3: coupled reverse scan) as 4 ints each and
 * returns their count.                                                      */
size_t mogt_diag_scan_workspace_bytes_cfg(int64_t batch, int64_t length, int64_t features,
                                          int vec, int lanes, int steps, int waves);
int mogt_diag_scan_fwd_cfg(const void* a, const void* b, void* h, void* a_prefix,
                           int64_t batch, int64_t length, int64_t features,
                           int in_dtype, int out_dtype, int vec, int lanes, int steps, int waves,
                           void* workspace, size_t workspace_bytes, void* stream);
int mogt_diag_scan_tiles(int family, int* out, int max_tiles);

/* mogt_diag_scan_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * look-back state lives in a fixed 8 MiB device array of the library, one per
 * GPU, held until the process ends (problems needing more are rejected with
 * MOGT_E_INVALID; at the default tiles that is about 2.6e8 elements of B*L*D).
 * The first call on a device clears the array on `stream`.  Calls on one GPU
 * share the array: calls that may overlap in time (different streams) race
 * and must not be issued.  Same results as mogt_diag_scan_fwd.               */
int mogt_diag_scan_fwd_noalloc(const void* a, const void* b, void* h, void* a_prefix,
                               int64_t batch, int64_t length, int64_t features,
                               int in_dtype, int out_dtype, void* stream);

/* Reverse-time diagonal scan h_t = a_{t+1} * h_{t+1} + b_t, h_L = 0 (a_L
 * unused), fp32 a, b, h [B, L, D]: with b = dH it is the gradient
 * G_t = dH_t + a_{t+1} G_{t+1} of the diagonal scan, the R = C = 1 case of
 * affine_scan_sequential_backward (affine_scan.py:65-124) and of the reverse
 * scan of _triton_affine_scan_hybrid_backward (triton_scan.py:359-426); then
 * db = G and da_t = G_t h_{t-1}.  Workspace:
 * mogt_diag_scan_workspace_bytes(batch, length, features, MOGT_F32).        */
int mogt_diag_scan_rev_fwd(const void* a, const void* b, void* h,
                           int64_t batch, int64_t length, int64_t features,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------- */
/* Coupled write-forget per-rank scan of the MOGT mixer with identity
 * connection (model_mogt.py:166-203 with connection_impl="identity",
 * phi_value_gate of width r, couple_forget_to_value_gate=True):
 *   g = sigmoid(z[b,t,i]),  a = damping * (1 - g),  v' = v[b,t,i*C+j] * g
 *   h[b,t,i*C+j] = a * h[b,t-1,i*C+j] + v'
 * z: gate logits [B, L, R] (fp32 or bf16); v: [B, L, R*C]; h: [B, L, R*C].
 * When v is bf16, v' is rounded to bf16 exactly as the reference's
 * `V_t_raw * value_gate.to(V_t_raw.dtype)` does (model_mogt.py:180).       */
size_t mogt_coupled_rank_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                              int64_t channels, int v_dtype);
int mogt_coupled_rank_scan_fwd(const void* z, const void* v, void* h,
                               int64_t batch, int64_t length, int64_t rank, int64_t channels,
                               float damping, int z_dtype, int v_dtype, int out_dtype,
                               void* workspace, size_t workspace_bytes, void* stream);
/* mogt_coupled_rank_scan_fwd (fp32 gate logits) that also writes
 * row_stats [B, L, ceil(R*C / 64)] fp32: the sum of squares of the fp32 state
 * h over each group of 64 consecutive features, i.e. the statistics of the
 * RMSNorm norm_out that reads h (model_mogt.py:236-241).  With them h can be
 * written in the read-out GEMM's dtype and normalised after the GEMM, since
 * theta_read(norm_out(h))_t = r_t W diag(w) h_t with r_t =
 * rsqrt(sum(row_stats[t]) / (R*C) + eps) (mogt_add_rmsnorm_rowscale_fwd).
 * Workspace: mogt_coupled_rank_scan_workspace_bytes.                       */
int mogt_coupled_rank_scan_stats_fwd(const void* z, const void* v, void* h, float* row_stats,
                                     int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                     float damping, int v_dtype, int out_dtype,
                                     void* workspace, size_t workspace_bytes, void* stream);
/* mogt_coupled_rank_scan_stats_fwd fed by one projection GEMM: row t of
 * proj [B, L, ld_proj] holds v (columns 0 .. R*C-1, phi_val's output) and, from
 * column gate_col, the value gate's pre-logits for the current token (R
 * columns) and, when gate_prev = 1, for the previous token (the next R
 * columns).  The gate logit is z[t][i] = proj[t][gate_col + i] +
 * (gate_prev && t > 0 ? proj[t-1][gate_col + R + i] : 0) + gate_const[b][i]
 * (gate_const [B, R] fp32: bias + prefix term, nullable) -- phi_value_gate
 * over [x_t, x_{t-1}, prefix] (model_mogt.py:104-122, 166-182) without the
 * concatenated input.  With row_stats (as in mogt_coupled_rank_scan_stats_fwd)
 * h is written in proj's `dtype`; without (nullable), out_dtype must be fp32
 * (the training path, which normalises h separately).  z_out (nullable, fp32
 * [B, L, R]) receives the assembled logits; without it they are kept in the
 * workspace's last 256-byte-aligned B*L*R*4 bytes.  Workspace:
 * mogt_coupled_rank_scan_workspace_bytes (which includes that room).      */
int mogt_coupled_rank_scan_proj_fwd(const void* proj, int64_t ld_proj, int64_t gate_col, int gate_prev,
                                    const float* gate_const, void* h, float* row_stats, float* z_out,
                                    int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                    float damping, int dtype, int out_dtype,
                                    void* workspace, size_t workspace_bytes, void* stream);
/* Gradient epilogue of the projection-fed scan (training): like
 * mogt_coupled_rank_scan_grad with v read from proj (gate_col = R*C, ld_proj =
 * R*C + R*(1 + gate_prev)) and z the logits the forward kept (z_out), written
 * into dproj, the gradient of the projection: dv in columns 0 .. R*C-1, the
 * logit gradient dz[t] in row t's current-token gate columns and in row
 * t-1's previous-token columns (zero in row L-1's), so one GEMM maps it back
 * to x and to [phi_val; W_cur; W_prev].  dz (fp32 [B, L, R], nullable) also
 * receives the logit gradient (for the bias and prefix terms).             */
int mogt_coupled_rank_scan_proj_grad(const float* G, const float* z, const void* proj, int64_t ld_proj,
                                     int gate_prev, const float* h, void* dproj, float* dz,
                                     int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                     float damping, int dtype, void* stream);
/* mogt_coupled_rank_scan_fwd with an explicit tile, one of
 * mogt_diag_scan_tiles(2) whose vector divides `channels` (v and h aligned to
 * it, up to 16 bytes); for sweeps and tile coverage tests.  Workspace:
 * mogt_diag_scan_workspace_bytes_cfg(batch, length, rank * channels, tile). */
int mogt_coupled_rank_scan_fwd_cfg(const void* z, const void* v, void* h,
                                   int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                   float damping, int z_dtype, int v_dtype, int out_dtype,
                                   int vec, int lanes, int steps, int waves,
                                   void* workspace, size_t workspace_bytes, void* stream);
/* Reverse scan of the coupled scan's backward: G_t = dh_t + a_{t+1} G_{t+1},
 * G_L = 0, with a_t = damping * (1 - sigmoid(z[b,t,i])) over rank i's C
 * channels, formed from the gate logits z [B, L, R] (fp32 or bf16) inside the
 * scan; dh, G fp32 [B, L, R*C].  The reverse scan of the reference's backward
 * (_triton_affine_scan_hybrid_backward, triton_scan.py:359-426, and
 * affine_scan_sequential_backward, affine_scan.py:65-124) for the diagonal
 * U_t = damping (1 - g_t) I of the coupled identity connection
 * (model_mogt.py:166-203).  Workspace:
 * mogt_coupled_rank_scan_rev_workspace_bytes.                             */
size_t mogt_coupled_rank_scan_rev_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                  int64_t channels);
int mogt_coupled_rank_scan_rev_fwd(const void* z, const float* dh, float* G,
                                   int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                   float damping, int z_dtype,
                                   void* workspace, size_t workspace_bytes, void* stream);
/* mogt_coupled_rank_scan_rev_fwd with an explicit tile, one of
 * mogt_diag_scan_tiles(3) whose vector divides `channels` (dh and G aligned to
 * it, up to 16 bytes); for sweeps and tile coverage tests.  Workspace:
 * mogt_diag_scan_workspace_bytes_cfg(batch, length, rank * channels, tile). */
int mogt_coupled_rank_scan_rev_fwd_cfg(const void* z, const float* dh, float* G,
                                       int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                       float damping, int z_dtype, int vec, int lanes, int steps, int waves,
                                       void* workspace, size_t workspace_bytes, void* stream);
/* Gradient epilogue of the coupled scan's backward (the autograd of the
 * fused gate + scan; the reference differentiates model_mogt.py:166-203
 * through torch ops): given G (fp32 [B, L, R*C], the reverse scan
 * G_t = dH_t + a_{t+1} G_{t+1}), the gate logits z (fp32 [B, L, R]), v and
 * the forward output h (fp32), writes dv = G * round(sigmoid(z)) in v's dtype
 * and dz = g (1 - g) (sum_c G v - damping sum_c G h_{t-1}) (fp32 [B, L, R]).
 * channels must be a multiple of 4 and rank * channels <= 4096.            */
int mogt_coupled_rank_scan_grad(const void* G, const float* z, const void* v, const float* h, void* dv,
                                float* dz, int64_t batch, int64_t length, int64_t rank,
                                int64_t channels, float damping, int v_dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* Dense affine scan  H_t = U_t H_{t-1} + V_t,  H_0 = 0  (R <= 32, any C).
 *
 * Replaces the forward of triton_affine_scan_hybrid / its
 * _triton_affine_scan_hybrid_forward (triton_scan.py:232-311, :429-477) and
 * the reference scans affine_scan_sequential / _doubling / _block_reference
 * (affine_scan.py:14-278), without the R == 16 restriction (triton_scan.py:200).
 * U: [B, L, R, R] fp32 (the reference up-casts U to fp32, triton_scan.py:203);
 * V: [B, L, R, C] fp32 or bf16; H: [B, L, R, C] in out_dtype.  U_prefix
 * (nullable) receives U_t ... U_1 in out_dtype (return_prefix=True).
 * Three launches on `stream` (chunk summaries, carries, output).            */
size_t mogt_affine_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                        int64_t channels);
int mogt_affine_scan_fwd(const void* U, const void* V, void* H, void* U_prefix,
                         int64_t batch, int64_t length, int64_t rank, int64_t channels,
                         int v_dtype, int out_dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/* The same scan with a rank-1 write V_t = v_t k_t^T, formed in registers
 * (never materialised): the `dense_scan(A, v, k)` form of the matrix scan,
 * i.e. configs[3]'s B_t = v_t k_t^T fed to
 * triton_affine_scan_hybrid (triton_scan.py:429-477) without building the
 * [B, L, R, C] tensor.  v: [B, L, R], k: [B, L, C], both vk_dtype (fp32 or
 * bf16); each element of V_t is the fp32 product v_i * k_j, as a
 * materialised fp32 V.  Workspace: mogt_affine_scan_workspace_bytes.        */
int mogt_affine_scan_vk_fwd(const void* U, const void* v, const void* k, void* H, void* U_prefix,
                            int64_t batch, int64_t length, int64_t rank, int64_t channels,
                            int vk_dtype, int out_dtype,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Generic affine scan  H_t = U_t H_{t-1} + V_t,  H_0 = 0,  for any rank
 * R <= 1024 and any C, with the state carried in fp32 or fp64.
 *
 * Replaces affine_scan_sequential / _doubling / _block_reference
 * (affine_scan.py:14-62, :127-172, :175-278) for what the MFMA pipeline above
 * does not take: their state_dtype argument (affine_scan.py:18; float64 in the
 * reference's own sanity check, sanity_affine_scan.py:19-61), ranks above 32,
 * and fp16 / fp64 inputs and outputs.  U: [B, L, R, R] in state_dtype
 * (MOGT_F32 or MOGT_F64; the reference casts U to state_dtype,
 * affine_scan.py:35); V: [B, L, R, C] in v_dtype; H: [B, L, R, C] and U_prefix
 * (nullable, U_t ... U_1, return_prefix=True, affine_scan.py:43-55): out_dtype.
 * v_dtype / out_dtype: MOGT_F32, MOGT_BF16, MOGT_F64 or MOGT_F16; narrow
 * outputs round the state through fp32, as torch's float64 -> bf16 cast does.
 * reverse = 1 runs the total-gradient recursion of the backward instead
 * (affine_scan_sequential_backward, affine_scan.py:110-118):
 * H_t = V_t + U_{t+1}^T H_{t+1}, H_{L-1} = V_{L-1}, with U_prefix NULL.
 * Up to three launches on `stream` (chunk summaries, carries, output); the
 * workspace (query with the same prefix flag and state dtype) needs no
 * clearing.                                                                 */
size_t mogt_affine_scan_generic_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                int64_t channels, int with_prefix, int state_dtype);
int mogt_affine_scan_generic_fwd(const void* U, const void* V, void* H, void* U_prefix,
                                 int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                 int v_dtype, int state_dtype, int out_dtype, int reverse,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* Block-local scan on the generic kernel, for what mogt_affine_local_scan
 * does not take (R > 32, float64): per block of `block_size` steps, from the
 * identity / zero state, every step's U_prefix [B, L, R, R] and H_prefix
 * [B, L, R, C] in out_dtype (the per-step outputs of triton_affine_local_scan,
 * triton_scan.py:54-148, :178-229; its per-block summaries are the prefixes at
 * each block's last step, which the caller gathers).  U in state_dtype, V in
 * v_dtype, as mogt_affine_scan_generic_fwd.  No workspace; one launch.      */
int mogt_affine_local_scan_generic(const void* U, const void* V, void* U_prefix, void* H_prefix,
                                   int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                   int64_t block_size, int v_dtype, int state_dtype, int out_dtype,
                                   void* stream);

/* Transport-only prefix product Y_t = U_t Y_{t-1}, Y_0 = I.
 * Replaces triton_fused_scan / _fused_scan_kernel (triton_scan.py:13-51,
 * :151-175), which hard-codes R = 16; here any R <= 32.  U fp32, Y out_dtype. */
size_t mogt_fused_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank);
int mogt_fused_scan_fwd(const void* U, void* Y, int64_t batch, int64_t length, int64_t rank,
                        int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Reverse-time scan of the backward, G_t = X_t + U_{t+1}^T G_{t+1},
 * G_{L-1} = X_{L-1}: the carry recursion of affine_scan_sequential_backward
 * (affine_scan.py:110-118) and of _triton_affine_scan_hybrid_backward
 * (triton_scan.py:397-416), on the matrix-core pipeline of
 * mogt_affine_scan_fwd walking time backwards and reading U_{t+1} transposed
 * (no reversed or transposed copy is built).  U [B,L,R,R], X, G [B,L,R,C]
 * fp32; R <= 32, C > 0; workspace of mogt_affine_scan_workspace_bytes.     */
int mogt_affine_scan_rev_fwd(const void* U, const void* X, void* G, int64_t batch, int64_t length,
                             int64_t rank, int64_t channels, void* workspace, size_t workspace_bytes,
                             void* stream);

/* dU_t = G_t M_{t-1}^T of the backward (affine_scan.py:119-124 and
 * triton_scan.py:417-418), M the forward state: M = H [B,L,R,C], or with P
 * (the prefix products [B,L,R,R], when G carries their gradient too) the
 * augmented M = [H | P]; M_{-1} = [0 | I].  G [B,L,R,C (+R)], dU [B,L,R,R];
 * all fp32, R <= 32.  No workspace.                                        */
int mogt_affine_scan_grad_u(const void* G, const void* H, const void* P, void* dU, int64_t batch,
                            int64_t length, int64_t rank, int64_t channels, void* stream);

/* Block-local affine scan: per block of `block_size` steps, the local prefixes
 * U_prefix/H_prefix [B, L, ...] and the per-block summaries U_summary
 * [B, nb, R, R] / H_summary [B, nb, R, C], nb = ceil(L / block_size); all
 * outputs fp32.  Replaces triton_affine_local_scan / _affine_local_scan_kernel
 * (triton_scan.py:54-148, :178-229).  No workspace; one launch.             */
int mogt_affine_local_scan(const void* U, const void* V, void* U_prefix, void* H_prefix,
                           void* U_summary, void* H_summary, int64_t batch, int64_t length,
                           int64_t rank, int64_t channels, int64_t block_size, int v_dtype,
                           void* stream);

/* ------------------------------------------------------------------------- */
/* Rank-1 coupled write-forget scan with readout:
 *   S_t = f_t S_{t-1} + (1 - f_t) v_t k_t^T,  y_t = S_t q_t,  S_0 = 0
 * i.e. affine_scan_sequential (affine_scan.py:14-62) with U_t = f_t I and
 * V_t = (1 - f_t) v_t k_t^T, read out through q_t, without materialising S_t.
 * f: [B, L, H]; k, v, q, y: [B, L, H, head_dim]; head_dim = 64.  Products run
 * on bf16 MFMA with fp32 accumulation and fp32 carried state (inputs are
 * rounded to bf16).  With bf16 k, v, q, sequences of at most 64
 * super-chunks of 256 steps (L <= 16384) and at most three work-groups per
 * compute unit (B * H * ceil(L / 256) <= 3 * CUs, i.e. all resident at once)
 * it runs as one launch whose work-groups exchange the carried states
 * through the workspace; otherwise as three launches (chunk states, carries,
 * outputs).  The workspace query covers both.
 * The one-launch form needs every super-chunk of a sequence resident at
 * once (in-order dispatch guarantees it on an otherwise idle GPU); if a
 * kernel on another stream holds the compute units its bounded waits give
 * up, the affected outputs are NaN and mogt_workspace_faults counts them.
 * mogt_rank1_coupled_scan_fwd_cfg: the same with the path forced (0 = by
 *   shape as above, 1 = one launch, 2 = three launches, 3 = a test of the
 *   give-up handling: the one-launch kernel with super-chunk 0 withholding
 *   its aggregate, and each work-group's wait on it giving up after 64 polls,
 *   so every super-chunk after the first comes back NaN and the count grows by
 *   exactly B * H * ceil(L / 256); needs L > 256); no counterpart in the
 *   reference -- for tests and
 *   benchmarks of both paths.
 * mogt_rank1_check_ranges: host-only self-check, no device work: evaluates
 *   every buffer range the rank-1 kernels build over a [B, L, H, 64] tensor of
 *   `elem_bytes` elements (2 or 4) -- each lies inside the tensor, covers the
 *   rows before L of its 64-row tile and none after -- and returns 0, or
 *   MOGT_E_INVALID naming the first violation.  No counterpart in the
 *   reference.                                                              */
size_t mogt_rank1_coupled_scan_workspace_bytes(int64_t batch, int64_t length, int64_t heads,
                                               int64_t head_dim);
int mogt_rank1_coupled_scan_fwd(const void* f, const void* k, const void* v, const void* q,
                                void* y, int64_t batch, int64_t length, int64_t heads,
                                int64_t head_dim, int f_dtype, int kvq_dtype, int out_dtype,
                                void* workspace, size_t workspace_bytes, void* stream);
int mogt_rank1_coupled_scan_fwd_cfg(const void* f, const void* k, const void* v, const void* q,
                                    void* y, int64_t batch, int64_t length, int64_t heads,
                                    int64_t head_dim, int f_dtype, int kvq_dtype, int out_dtype,
                                    void* workspace, size_t workspace_bytes, int path, void* stream);
int mogt_rank1_check_ranges(int64_t batch, int64_t length, int64_t heads, int elem_bytes);

/* ------------------------------------------------------------------------- */
/* Row-wise kernels of the MOGT block (one wave per row, rows of `dim`
 * contiguous elements, dim a multiple of 4 and <= 4096; weight fp32 [dim]).
 *
 * mogt_rmsnorm_fwd: out = (x * rsqrt(mean(x^2) + eps)).type_as(x) * weight
 *   -- RMSNorm.forward, model_mogt.py:9-20 (statistics in fp32).
 * mogt_add_rmsnorm_fwd: x_out = x + (scale * z) [the product rounded to z's
 *   dtype], out = rmsnorm(x_out) -- the residual update followed by the next
 *   RMSNorm (model_mogt.py:243-256), x and x_out fp32; x_out may be null when
 *   only the normalised row is needed (the backbone's final norm_f).
 * mogt_silu_mul_fwd: y = [rows, 2*hidden] (w1 | w2 outputs), out = silu(y1) *
 *   y2 [rows, hidden] -- SwiGLU.forward, model_mogt.py:29-30 (silu result
 *   rounded to the tensor dtype before the product, as torch does).          */
int mogt_rmsnorm_fwd(const void* x, const float* weight, void* out, int64_t rows, int64_t dim,
                     float eps, int x_dtype, int out_dtype, void* stream);
int mogt_add_rmsnorm_fwd(const float* x, const void* z, float scale, const float* weight,
                         float* x_out, void* out, int64_t rows, int64_t dim, float eps,
                         int z_dtype, int out_dtype, void* stream);
int mogt_silu_mul_fwd(const void* y, void* out, int64_t rows, int64_t hidden, int dtype,
                      void* stream);
/* mogt_swiglu_gate_fwd: y = silu(x w_gate^T) * (x w_up^T) as one bf16 GEMM
 *   with the gate in its epilogue -- SwiGLU.forward's silu(w1(x)) * w2(x),
 *   model_mogt.py:29-30, without the [rows, 2*hidden] pre-activations.  x
 *   [rows, d_in] (row stride ldx), w_gate / w_up [hidden, d_in] (nn.Linear
 *   weights, contiguous), y [rows, hidden] (row stride ldy); dtype MOGT_BF16
 *   only; fp32 accumulation, each linear output and the silu rounded to bf16
 *   as in the unfused path.  d_in % 32 == 0, hidden % 128 == 0, ldx % 8 == 0,
 *   ldy % 4 == 0; x and weights 16-byte aligned, y 8-byte aligned.           */
int mogt_swiglu_gate_fwd(const void* x, const void* w_gate, const void* w_up, void* y, int64_t rows,
                         int64_t d_in, int64_t hidden, int64_t ldx, int64_t ldy, int dtype, void* stream);
/* mogt_swiglu_gate_fwd_cfg: the same (model_mogt.py:29-30) with the schedule
 *   forced: 0 = by shape (as mogt_swiglu_gate_fwd: persistent when d_in % 128
 *   == 0 and d_in >= 640, else one tile per work-group), 1 = one tile per
 *   work-group, 2 = persistent (MOGT_E_INVALID when d_in does not allow it).
 *   Outputs are bit-identical across schedules; for tests and the bench.      */
int mogt_swiglu_gate_fwd_cfg(const void* x, const void* w_gate, const void* w_up, void* y, int64_t rows,
                             int64_t d_in, int64_t hidden, int64_t ldx, int64_t ldy, int dtype, int path,
                             void* stream);
/* mogt_swiglu_check_schedule: host-only self-check, no device work: walks the
 *   persistent schedule's tile assignment for `rows` x `hidden` outputs on a
 *   grid of `grid` work-groups (the CU count on a GPU) and returns 0 when every
 *   tile, and every (row block, output block) it maps to, is taken by exactly
 *   one work-group, else MOGT_E_INVALID naming the first violation.  No
 *   counterpart in the reference.                                            */
int mogt_swiglu_check_schedule(int64_t rows, int64_t hidden, int grid);
/* mogt_linear_wgrad: dW = dY^T X, the weight gradient of a bias-free
 *   nn.Linear (model_mogt.py:25-27 w1, w2, w3, :57 phi_val, :61 theta_read;
 *   the grad_weight torch's linear backward forms), as a split-K GEMM on the
 *   matrix cores: the tokens are cut into `splits` slices, fp32 partials of
 *   every slice go to the workspace, and a second kernel sums them in slice
 *   order (deterministic) and rounds once.  dY [tokens, d_out] (row stride
 *   ldd) and X [tokens, d_in] (row stride ldx) bf16; dW [d_out, d_in] (row
 *   stride ldw) in out_dtype (MOGT_BF16 or MOGT_F32); fp32 accumulation.
 *   d_out, d_in and the strides multiples of 8; dY, X, dW and the workspace
 *   16-byte aligned.  splits <= 0 picks enough slices to give each CU one
 *   work-group.  tokens == 0 writes zeros.  A slice's bytes (slice tokens x
 *   row stride x 2) must stay under 2 GiB (MOGT_E_INVALID asks for more
 *   splits).
 * mogt_linear_wgrad_splits: the slice count a launch with these arguments
 *   uses (cus: the device's CU count, or <= 0 to query the current device);
 *   -1 for a bad shape.
 * mogt_linear_wgrad_workspace_bytes: splits x d_out x d_in x 4 for that
 *   count (0 without tokens).                                                 */
int mogt_linear_wgrad(const void* dy, const void* x, void* dw, int64_t tokens, int64_t d_out, int64_t d_in,
                      int64_t ldd, int64_t ldx, int64_t ldw, int64_t splits, int out_dtype, void* workspace,
                      size_t workspace_bytes, void* stream);
int64_t mogt_linear_wgrad_splits(int64_t tokens, int64_t d_out, int64_t d_in, int64_t splits, int64_t cus);
size_t mogt_linear_wgrad_workspace_bytes(int64_t tokens, int64_t d_out, int64_t d_in, int64_t splits,
                                         int64_t cus);
/* mogt_add_rmsnorm_fwd for a read-out of an unnormalised row: z = W diag(w) h
 * (theta_read with norm_out's weight folded in), row_stats [rows, n_stats] the
 * partial sums of squares of h (mogt_coupled_rank_scan_stats_fwd).  With r =
 * rsqrt(sum(row_stats[row]) / dim + stat_eps):  Z = round(r z) (the
 * reference's theta_read(norm_out(h)) in z's dtype), x_out = x + round(scale
 * Z), out = rmsnorm(x_out) * weight -- model_mogt.py:236-256.             */
int mogt_add_rmsnorm_rowscale_fwd(const float* x, const void* z, const float* row_stats,
                                  int64_t n_stats, float stat_eps, float scale, const float* weight,
                                  float* x_out, void* out, int64_t rows, int64_t dim, float eps,
                                  int z_dtype, int out_dtype, void* stream);

/* Backward of the row kernels (the autograd of RMSNorm and SwiGLU,
 * model_mogt.py:15-20, 29-30, as torch differentiates the reference's
 * expressions).
 * mogt_rmsnorm_bwd: dx = r (dy*w - n mean(dy*w*n)) [+ dres], n = x r,
 *   r = rsqrt(mean(x^2) + eps); dx has x's dtype, dy fp32 or bf16; dres
 *   (fp32 [rows, dim], may be null) is the residual stream's own gradient of
 *   add_rmsnorm (x fp32).  Each wave covers rows_per_wave rows and each
 *   work-group 4 waves; dw_partial: fp32 [dim, G], G = ceil(ceil(rows /
 *   rows_per_wave) / 4) work-groups: per feature, each work-group's partial
 *   sum of dy * n.type_as(x) (its waves' sums added in a fixed order); the
 *   caller sums each feature's G partials (a contiguous row).
 *   dz (may be null): also writes dz = dx * dz_scale in dz_dtype, the
 *   gradient of add_rmsnorm's scaled residual term x + scale * z.
 * mogt_silu_mul_bwd: y = [rows, 2*hidden] (forward input), dout = [rows,
 *   hidden]; dy = [rows, 2*hidden] = [dout*b*silu'(a) | dout*silu(a)],
 *   rounded where torch's bf16 autograd rounds.                            */
int mogt_rmsnorm_bwd(const void* x, const float* weight, const void* dy, const float* dres, void* dx,
                     float* dw_partial, int64_t rows, int64_t dim, float eps, int rows_per_wave,
                     int x_dtype, int dy_dtype, void* dz, float dz_scale, int dz_dtype, void* stream);
int mogt_silu_mul_bwd(const void* y, const void* dout, void* dy, int64_t rows, int64_t hidden,
                      int dtype, void* stream);

/* Backward of the token embedding (nn.Embedding in MOGTModel.forward,
 * model_mogt.py:262, 270, which torch differentiates by sorting the ids):
 * dweight[v] = the sum of the grad rows of every position holding token v,
 * summed in position order (deterministic).  The caller sorts the
 * n token ids stably (sorted_ids, int64) with the positions in that order
 * (positions, int64), zero-fills dweight (fp32 [vocab, dim]) and passes
 * partials: fp32 [ceil(n / 16) * 2, dim] scratch.  Position p < n_first is
 * row p of grad (row stride ld_grad), position p >= n_first row p - n_first
 * of grad2 (stride ld_grad2; nullable when n_first = n): two lookups into one
 * table (the tokens and the prefix-condition rows) share one dweight.  fp32
 * or bf16 rows; dim % 4 == 0, <= 4096.  Ids outside [0, vocab) are
 * skipped.                                                                 */
int mogt_embedding_bwd(const void* grad, int64_t ld_grad, const void* grad2, int64_t ld_grad2,
                       int64_t n_first, int grad_dtype, const int64_t* sorted_ids,
                       const int64_t* positions, int64_t n, int64_t dim, int64_t vocab, float* dweight,
                       float* partials, void* stream);

/* ------------------------------------------------------------------------- */
/* Connection map of the transport, U = damping * f(scale * A) for a batch of
 * skew-symmetric r x r generators A (fp32 [count, r, r], r <= 32), replacing
 * MOGTBlock._build_transport (model_mogt.py:79-102):
 *   impl MOGT_CONN_EXP:    f = matrix exponential (torch.matrix_exp, :83-85)
 *   impl MOGT_CONN_CAYLEY: f(S) = (I - S/2)^{-1} (I + S/2)
 *                          (torch.linalg.solve(I - A/2, I + A/2), :86-90)
 * The reference passes A / r, i.e. scale = 1 / r.  U: [count, r, r] in
 * out_dtype.  A must be skew-symmetric (the kernels rely on A^T = -A).      */
#define MOGT_CONN_EXP 0
#define MOGT_CONN_CAYLEY 1
int mogt_connection_map_fwd(const void* A, void* U, int64_t count, int64_t rank, float scale,
                            float damping, int impl, int out_dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* Cross-entropy rows of the chunked tied-head loss, replacing the per-chunk
 * F.cross_entropy of _ChunkedLinearCrossEntropy.forward and the softmax /
 * one-hot / scale steps of its backward (chunked_lm_loss.py:29-35, 61-64).
 * logits: [rows, vocab] with row stride `ld` elements (fp32 or bf16, the
 * caller's GEMM output); labels: int64 [rows].
 *
 * mogt_lm_ce_fwd: lse_rows[r] = log sum_j exp(logits[r][j]) and
 *   loss_rows[r] = lse_rows[r] - logits[r][labels[r]] (fp32).  A row whose
 *   label equals ignore_index gets loss 0 (F.cross_entropy's ignore_index,
 *   -100 by default); any other label outside [0, vocab) gets NaN.
 * mogt_lm_ce_bwd: grad[r][j] = s * (exp(logits[r][j] - lse_rows[r]) -
 *   [j == labels[r]]) with s = *scale (one fp32 in device memory: the
 *   caller's grad_output / tokens, read by the kernel, so no host sync),
 *   row stride ld_grad, fp32 or bf16; ignored rows are zero.  grad may be
 *   the logits buffer itself (same dtype and stride).                      */
int mogt_lm_ce_fwd(const void* logits, int64_t ld, int logits_dtype, const int64_t* labels,
                   int64_t rows, int64_t vocab, int64_t ignore_index, float* loss_rows,
                   float* lse_rows, void* stream);
int mogt_lm_ce_bwd(const void* logits, int64_t ld, int logits_dtype, const int64_t* labels,
                   const float* lse_rows, int64_t rows, int64_t vocab, int64_t ignore_index,
                   const float* scale, void* grad, int64_t ld_grad, int grad_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOGT_SCAN_H */

/*
 * mm_scan.h -- C ABI of the MI355X (gfx950) selective-scan library `libmm_scan.so`.
 *
 * Three entry points replace the native calls on the Mamba selective-scan hot path:
 *
 *   mm_scan_fwd      replaces the pybind call `selective_scan_cuda.fwd(u, delta, A, B, C, D, z,
 *                    delta_bias, P, Q, gamma, delta_softplus)` bound at
 *                    csrc/selective_scan/selective_scan.cpp:620-627, i.e. selective_scan_fwd
 *                    (selective_scan.cpp:270-413) -> selective_scan_fwd_cuda
 *                    (selective_scan_fwd_kernel.cuh:593-623) for real A, including the
 *                    MotifMamba low-rank P/Q coupling (selective_scan.cpp:342-369,
 *                    selective_scan_interface.py:237-350). The parameter block mirrors
 *                    SSMParamsBase (selective_scan.h:26-82) but with int64 element strides
 *                    instead of uint32.
 *
 *   mm_scan_bwd      replaces `selective_scan_cuda.bwd(u, delta, A, B, C, D, z, delta_bias, P, Q,
 *                    gamma, dout, x, out, dz, dP_out, dQ_out, delta_softplus, recompute_out_z)`
 *                    (selective_scan.cpp:415-612, pybind :628-637) for real A, with the exact
 *                    gradients of the P/Q coupling (dense kernel selective_scan_bwd_kernel.cuh:
 *                    166-345; autograd through selective_scan_interface.py:262-350 for dP/dQ).
 *
 *   mm_state_update  replaces `selective_state_update(state, x, dt, A, B, C, D, z, dt_bias,
 *                    dt_softplus)` as called at mamba_ssm/modules/mamba_simplemotif.py:397-399
 *                    (upstream mamba_ssm.ops.triton.selective_state_update, not vendored in the
 *                    reference; its in-tree math is mamba_simplemotif.py:369-376).
 *
 * Conventions
 *   - All pointers are device pointers (HBM) except the parameter blocks themselves, which are
 *     read on the host during the call and may be freed as soon as the call returns.
 *   - Strides are in elements, not bytes. The innermost (sequence) dimension of u, delta, z,
 *     out, out_z and of variable B/C must be contiguous (stride 1), as the reference requires
 *     (selective_scan.cpp:304-305, 321, 326, 350).
 *   - The library never allocates, frees or synchronises. Every call enqueues its kernels on
 *     `stream` (a hipStream_t; NULL = the null stream of the current device) and returns.
 *     Scratch memory, where a shape benefits from it, is provided by the caller (`workspace`).
 *   - Return value: 0 on success. MM_ERR_INVALID_ARGUMENT (-1) when the parameter block fails
 *     validation (nothing is launched), MM_ERR_UNSUPPORTED (-2) for a valid request this build
 *     does not implement, otherwise the positive hipError_t of the failed launch.
 *     mm_last_error() returns a message for the most recent failure on the calling thread.
 */
#ifndef MM_SCAN_H_
#define MM_SCAN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MM_SCAN_ABI_VERSION 10

#define MM_OK 0
#define MM_ERR_INVALID_ARGUMENT (-1)
#define MM_ERR_UNSUPPORTED (-2)

/* Element types of the activations (u, delta, z, out, out_z, variable B/C). A, D, delta_bias,
 * constant B/C, last_state and chunk_states are always float32, as in the reference
 * (selective_scan.cpp:282-292, 332-346). */
typedef enum mm_dtype {
    MM_FLOAT32 = 0,
    MM_FLOAT16 = 1,
    MM_BFLOAT16 = 2
} mm_dtype;

/* Largest state dimension accepted by mm_scan_fwd (the reference limit, selective_scan.cpp:313). */
#define MM_SCAN_MAX_DSTATE 256
/* Sequence-chunk length of the chunk_states wire format (selective_scan.cpp:383). */
#define MM_SCAN_CHUNK 2048

/* Forward selective scan (real A only):
 *   delta' = softplus(delta + delta_bias)            (softplus only when delta_softplus != 0)
 *   h_t[n] = exp(delta'_t * A[d,n]) * h_{t-1}[n] + delta'_t * u_t * B[b, g(d), n, t],  h_{-1} = 0
 *   y_t    = sum_n h_t[n] * C[b, g(d), n, t]
 *   out_t  = y_t + D[d] * u_t ;  out_z_t = out_t * silu(z_t)
 * with g(d) = d / (dim / n_groups). Constant B/C (is_variable_* == 0) are (dim, dstate) float32
 * and use B[d, n] / C[d, n] instead. */
typedef struct mm_scan_fwd_params {
    int64_t batch, dim, seqlen, dstate, n_groups;
    mm_dtype itype;          /* dtype of u, delta, z, out, out_z and variable B/C */
    int32_t is_variable_B;   /* 1: B is (batch, n_groups, dstate, seqlen) of itype; 0: (dim, dstate) f32 */
    int32_t is_variable_C;
    int32_t delta_softplus;

    const void *u;           /* (batch, dim, seqlen) */
    const void *delta;       /* (batch, dim, seqlen) */
    const float *A;          /* (dim, dstate) */
    const void *B;
    const void *C;
    const float *D;          /* (dim,) or NULL */
    const void *z;           /* (batch, dim, seqlen) or NULL */
    const float *delta_bias; /* (dim,) or NULL */

    void *out;               /* (batch, dim, seqlen) pre-gate output, or NULL (not written) */
    void *out_z;             /* (batch, dim, seqlen) gated output; required iff z != NULL */
    float *last_state;       /* (batch, dim, dstate) contiguous, or NULL */
    float *chunk_states;     /* (batch, dim, ceil(seqlen/2048), 2*dstate) contiguous, or NULL:
                                per chunk the running (prod a, h) pair of the reference's `x`
                                (selective_scan_fwd_kernel.cuh:492-495) */

    int64_t u_batch_stride, u_d_stride;
    int64_t delta_batch_stride, delta_d_stride;
    int64_t z_batch_stride, z_d_stride;
    int64_t out_batch_stride, out_d_stride;
    int64_t out_z_batch_stride, out_z_d_stride;
    int64_t A_d_stride, A_dstate_stride;
    int64_t B_batch_stride, B_group_stride, B_dstate_stride, B_d_stride;
    int64_t C_batch_stride, C_group_stride, C_dstate_stride, C_d_stride;

    /* Optional device scratch of `workspace_bytes` bytes (16-byte aligned), owned by the caller.
     * Shapes with few (batch, channel) rows and long sequences scan the sequence in parallel
     * segments and need mm_scan_fwd_workspace_size() bytes for the segment carries; with a NULL or
     * smaller workspace the same results come from the single-pass kernels. No counterpart in
     * SSMParamsBase: the reference scans each row with one thread block. */
    void *workspace;
    int64_t workspace_bytes;

    /* MotifMamba low-rank coupling (SSMParamsBase::has_pq / pq_rank / P_* / Q_* / gamma_*,
     * selective_scan.h:36-37, 58-65, 80-82; checks of selective_scan.cpp:342-369). With P and Q
     * set, the recurrence becomes
     *   h_t = exp(delta'_t A[d,:]) * h_{t-1} + delta'_t P_d (Q_d h_{t-1}) + delta'_t u_t B_t
     * (selective_scan_interface.py:320-337), P_d = P[d] (dstate, pq_rank) and Q_d = Q[d]
     * (pq_rank, dstate), float32; a pair shared by every channel has P_d_stride = Q_d_stride = 0.
     * pq_rank is 0..8 (0: no coupling). chunk_states then holds (1, h) per chunk, as the
     * reference's dense forward writes it (selective_scan_fwd_kernel.cuh:244-249). gamma
     * ((dstate,) or (dim, dstate)) is carried for interface parity and, as in both reference
     * forward paths, not read. NULL P and Q: the diagonal scan above. */
    const float *P;
    const float *Q;
    const float *gamma;
    int64_t pq_rank;
    int64_t P_d_stride, P_dstate_stride, P_r_stride;
    int64_t Q_d_stride, Q_r_stride, Q_dstate_stride;
    int64_t gamma_d_stride, gamma_dstate_stride;

    /* Checkpoints for the backward (ABI version 8, 9 without P/Q; no counterpart in the reference,
     * whose backward keeps only `chunk_states`). When non-NULL: the state before every 16-step
     * tile, float32 [ceil(seqlen / 16)][batch][dim][16], states past dstate written as 0 --
     * B * dim * seqlen * 4 bytes, about one float32 copy of u. Passed to mm_scan_bwd as
     * `tile_states`, they spare it the recompute of the whole forward. Written with P/Q and
     * dstate <= 16, and without P/Q together with chunk_states (the training forward) by the
     * dstate-16 kernels or, below dstate 16, the P/Q kernels run with a zero coupling
     * (mm_scan_fwd_tile_states_size() is non-zero exactly when this request can write them).
     * NULL: not written. */
    float *tile_states;
} mm_scan_fwd_params;

/* Backward of the diagonal forward scan: the gradients of every input for a given gradient `dout`
 * of the returned output (out_z when z is given, else out), as selective_scan_cuda.bwd computes them
 * (selective_scan.cpp:415-612, selective_scan_bwd_kernel.cuh:405-880), for real A (P/Q: below):
 *   g_t   = dout_t * silu(z_t)                      dz_t = dout_t * out_t * silu'(z_t)
 *   gh_t  = C_t g_t + exp(delta'_{t+1} A) gh_{t+1}  (reverse scan per state, gh after L = 0)
 *   du_t  = D g_t + delta'_t sum_n gh_t B_t          ddelta'_t = sum_n gh_t (u_t B_t + A (h_t - delta'_t u_t B_t))
 *   dB_t += gh_t delta'_t u_t ;  dC_t += g_t h_t ;   dA += gh_t delta'_t (h_t - delta'_t u_t B_t)
 *   ddelta_t = ddelta'_t * sigmoid(delta_t + bias) with softplus (1 past the threshold 20)
 *   dD += g_t u_t ;  ddelta_bias += ddelta_t
 * The forward states are recomputed from h_{-1} = 0 (the chunk states of the forward are not
 * needed). dA, dB, dC, dD and ddelta_bias are sums over rows and steps: the call overwrites them
 * (it clears them on `stream` first) and accumulates in float32 with device atomics, so their
 * low-order bits depend on the order in which workgroups finish, as in the reference. */
typedef struct mm_scan_bwd_params {
    int64_t batch, dim, seqlen, dstate, n_groups;
    mm_dtype itype;          /* dtype of u, delta, z, out, dout, du, ddelta, dz and variable B/C */
    int32_t is_variable_B;
    int32_t is_variable_C;
    int32_t delta_softplus;

    const void *u;           /* (batch, dim, seqlen) */
    const void *delta;       /* (batch, dim, seqlen) */
    const float *A;          /* (dim, dstate) */
    const void *B;           /* as in mm_scan_fwd_params */
    const void *C;
    const float *D;          /* (dim,) or NULL */
    const void *z;           /* (batch, dim, seqlen) or NULL */
    const float *delta_bias; /* (dim,) or NULL */
    const void *dout;        /* (batch, dim, seqlen) */
    const void *out;         /* (batch, dim, seqlen) pre-gate forward output; required iff z != NULL */

    void *du;                /* (batch, dim, seqlen) */
    void *ddelta;            /* (batch, dim, seqlen) */
    void *dz;                /* (batch, dim, seqlen); required iff z != NULL */
    void *out_z;             /* (batch, dim, seqlen) out * silu(z) recomputed, or NULL */
    float *dA;               /* (dim, dstate) */
    float *dB;               /* float32, the shape of B: (batch, n_groups, dstate, seqlen) or (dim, dstate) */
    float *dC;               /* float32, the shape of C */
    float *dD;               /* (dim,); required iff D != NULL */
    float *ddelta_bias;      /* (dim,); required iff delta_bias != NULL */

    int64_t u_batch_stride, u_d_stride;
    int64_t delta_batch_stride, delta_d_stride;
    int64_t z_batch_stride, z_d_stride;
    int64_t out_batch_stride, out_d_stride;
    int64_t dout_batch_stride, dout_d_stride;
    int64_t du_batch_stride, du_d_stride;
    int64_t ddelta_batch_stride, ddelta_d_stride;
    int64_t dz_batch_stride, dz_d_stride;
    int64_t out_z_batch_stride, out_z_d_stride;
    int64_t A_d_stride, A_dstate_stride;
    int64_t B_batch_stride, B_group_stride, B_dstate_stride, B_d_stride;
    int64_t C_batch_stride, C_group_stride, C_dstate_stride, C_d_stride;
    int64_t dA_d_stride, dA_dstate_stride;
    int64_t dB_batch_stride, dB_group_stride, dB_dstate_stride, dB_d_stride;
    int64_t dC_batch_stride, dC_group_stride, dC_dstate_stride, dC_d_stride;

    /* Device scratch of mm_scan_bwd_workspace_size() bytes (16-byte aligned), owned by the caller:
     * the recomputed forward states at every 16-step tile start (and, for dstate 16 and for P/Q,
     * the per-16-channel-block partial sums of dB and dC -- per-workgroup partial sums for the
     * general kernels of the other shapes; for dstate 16 with tile_states, the adjoint carries of
     * the sequence segments its last round of workgroups is cut into). Required.
     * With tile_states at dstate 16, a workspace without room for the carries (sized for another
     * device or round size) is accepted too: the call then scans every row whole, without segments. */
    void *workspace;
    int64_t workspace_bytes;

    /* MotifMamba low-rank coupling (ABI version 7). With P and Q set (as in mm_scan_fwd_params:
     * P_d (dstate, pq_rank), Q_d (pq_rank, dstate), float32, d strides 0 for a pair shared by all
     * channels), the gradients are those of the coupled recurrence
     *   h_t = exp(delta'_t A) h_{t-1} + delta'_t P (Q h_{t-1}) + delta'_t u_t B_t
     * -- what the reference's dense backward kernel (selective_scan_bwd_kernel.cuh:166-345) and
     * torch autograd through selective_scan_full_matrix_cuda (selective_scan_interface.py:262-350,
     * its path for P/Q calls with z and for dP/dQ) both compute -- with the state adjoint running through the transposed transition matrix exp(delta' A) + delta' P Q,
     * plus dP and dQ (float32, the shapes of P and Q; overwritten: the call clears them first).
     * Supported: variable B and C, dstate <= 16, pq_rank 1..8, dim and dim / n_groups multiples of
     * 16, seqlen a multiple of 8; other requests return MM_ERR_UNSUPPORTED. */
    const float *P;
    const float *Q;
    int64_t pq_rank;
    int64_t P_d_stride, P_dstate_stride, P_r_stride;
    int64_t Q_d_stride, Q_r_stride, Q_dstate_stride;
    float *dP;
    float *dQ;
    int64_t dP_d_stride, dP_dstate_stride, dP_r_stride;
    int64_t dQ_d_stride, dQ_r_stride, dQ_dstate_stride;

    /* Optional (ABI version 8, 9 without P/Q): the `tile_states` mm_scan_fwd wrote for the same
     * inputs; the P/Q backward (also serving diagonal requests below dstate 16 with a zero
     * coupling) and the dstate-16 backward then read their checkpoints there instead of
     * recomputing them (and need a smaller workspace); the general backward ignores them. The
     * contents are trusted: stale states give wrong gradients. */
    const float *tile_states;
} mm_scan_bwd_params;

/* Single-token decode update, in place on `state`:
 *   dt' = softplus(dt + dt_bias) (softplus only when dt_softplus != 0)
 *   state[b,d,n] = state[b,d,n] * exp(dt' * A[d,n]) + dt' * B[b,g(d),n] * x[b,d]
 *   out[b,d] = (sum_n state[b,d,n] * C[b,g(d),n] + D[d] * x[b,d]) * silu(z[b,d])
 * x, dt, z, out, B, C are itype; A is float32. The state is state_type, D and dt_bias are D_type
 * and dt_bias_type (ABI version 10; all three float32 when left zero): every value is widened to
 * float32, the arithmetic is float32, the updated state is rounded to state_type (round to nearest
 * even) when stored, and out is read from the float32 state before that rounding -- the semantics
 * of the upstream Triton kernel (mamba_ssm 2.2.x selective_state_update), which loads each operand
 * `.to(tl.float32)` and stores the state back in its own dtype. A bfloat16 or float16 model's
 * decode passes the state in dt_proj.weight.dtype and D / dt_proj.bias uncast
 * (mamba_simplemotif.py:397-399, 410-414, 428-435). */
typedef struct mm_state_update_params {
    int64_t batch, dim, dstate, n_groups;
    mm_dtype itype;
    int32_t dt_softplus;

    void *state;             /* (batch, dim, dstate) of state_type, updated in place */
    const void *x;           /* (batch, dim) */
    const void *dt;          /* (batch, dim) */
    const float *A;          /* (dim, dstate) */
    const void *B;           /* (batch, n_groups, dstate) */
    const void *C;           /* (batch, n_groups, dstate) */
    const void *D;           /* (dim,) contiguous, of D_type, or NULL */
    const void *z;           /* (batch, dim) or NULL */
    const void *dt_bias;     /* (dim,) contiguous, of dt_bias_type, or NULL */
    void *out;               /* (batch, dim) */

    int64_t state_batch_stride, state_d_stride, state_dstate_stride;
    int64_t x_batch_stride, x_d_stride;
    int64_t dt_batch_stride, dt_d_stride;
    int64_t z_batch_stride, z_d_stride;
    int64_t out_batch_stride, out_d_stride;
    int64_t A_d_stride, A_dstate_stride;
    int64_t B_batch_stride, B_group_stride, B_dstate_stride;
    int64_t C_batch_stride, C_group_stride, C_dstate_stride;

    /* ABI version 10: element types of state, D and dt_bias (MM_FLOAT32 = 0 when zeroed). */
    mm_dtype state_type, D_type, dt_bias_type;
} mm_state_update_params;

/* Forward scan. Replaces selective_scan_cuda.fwd (selective_scan.cpp:270-413, pybind :620-627),
 * the diagonal kernels and the dense P/Q kernel (selective_scan_fwd_kernel.cuh:159-251, 587-598). */
int mm_scan_fwd(const mm_scan_fwd_params *params, void *stream);

/* Bytes of `workspace` that let mm_scan_fwd use sequence-parallel segments for this request
 * (0: the single-pass kernels are used anyway). Reads only sizes, flags and strides of `params`,
 * and the current device's compute-unit count (the segment count targets about 5 waves per SIMD):
 * query it with the call's device current. Returns 0 for a request mm_scan_fwd would reject. No counterpart in the reference (its forward
 * allocates nothing beyond the outputs, selective_scan.cpp:383-389). */
int64_t mm_scan_fwd_workspace_size(const mm_scan_fwd_params *params);

/* Bytes of `tile_states` mm_scan_fwd writes for this request, 0 when it cannot write them (no
 * counterpart in the reference: the checkpoints the backward would otherwise recompute). */
int64_t mm_scan_fwd_tile_states_size(const mm_scan_fwd_params *params);

/* Size of the static device scratch behind mm_scan_fwd_noalloc (4 MiB per GPU, held from the
 * library's load until the process ends). */
#define MM_SCAN_FWD_NOALLOC_SCRATCH_BYTES (4 << 20)

/* mm_scan_fwd for callers that cannot allocate device memory: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. No counterpart in the reference. Same results
 * as mm_scan_fwd with a workspace of mm_scan_fwd_workspace_size() bytes; params->workspace and
 * workspace_bytes are ignored: the sequence-segment scratch is a static device array of
 * MM_SCAN_FWD_NOALLOC_SCRATCH_BYTES per GPU. The segment heuristic asks for at most about 3,456
 * bytes per SIMD of the device (batch * dim * segments * 72 bytes with segments ~ 5 * SIMDs * 8 /
 * (batch * dim)): up to ~3.4 MiB on the 1,024-SIMD MI355X (for instance, needs
 * 2,949,120 bytes). A request that needs more than the static buffer (a device with more SIMDs, or
 * MM_SCAN_SEGMENTS forcing more segments) runs the single-pass kernels, with the results of
 * mm_scan_fwd given no workspace. The call allocates and frees nothing. All calls on one GPU share
 * that GPU's scratch: calls that overlap in time on one GPU (other streams, other threads) race and
 * must be serialised by the caller. */
int mm_scan_fwd_noalloc(const mm_scan_fwd_params *params, void *stream);

/* Backward scan. Replaces selective_scan_cuda.bwd (selective_scan.cpp:415-612, pybind :628-637). */
int mm_scan_bwd(const mm_scan_bwd_params *params, void *stream);

/* Bytes of `workspace` mm_scan_bwd needs for `params` (0 for a request it would reject or that has
 * nothing to do). Reads sizes and, for dstate 16 with tile_states, the current device's compute-unit
 * count (the size of one round of workgroups). No counterpart in the reference (its backward recomputes each
 * 2048-step chunk inside one thread block). */
int64_t mm_scan_bwd_workspace_size(const mm_scan_bwd_params *params);

/* Decode step. Replaces selective_state_update (call site mamba_simplemotif.py:397-399). */
int mm_state_update(const mm_state_update_params *params, void *stream);

/* Message for the last non-zero return on this thread ("" if none). */
const char *mm_last_error(void);

/* MM_SCAN_ABI_VERSION of the loaded library; lets a binding refuse a stale build. */
int mm_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MM_SCAN_H_ */

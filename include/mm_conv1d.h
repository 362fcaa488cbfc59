/*
 * mm_conv1d.h -- C ABI of the causal depthwise conv1d of libmm_scan.so (gfx950), the step before the
 * selective scan in every Mamba block.
 *
 *   mm_causal_conv1d_fwd     replaces `causal_conv1d_fn(x, weight, bias, seq_idx=None,
 *                            initial_states, return_final_states, final_states_out, activation)`
 *                            (call sites mamba_ssm/modules/mamba_simplemotif.py:301-306,
 *                            mamba_ssm/ops/selective_scan_interface.py:482-484 and :672) from the
 *                            third-party package causal-conv1d (>= 1.2.0, pyproject.toml:33-34; not
 *                            vendored), whose in-tree fallback is mamba_simplemotif.py:298-299:
 *                                out[b,d,t] = act(bias[d] + sum_{k<W} weight[d,k] * x[b,d,t-(W-1)+k])
 *                            with x before t = 0 taken from initial_states (or 0).
 *   mm_causal_conv1d_bwd     replaces causal_conv1d_bwd_function (selective_scan_interface.py:635-637),
 *                            the backward MambaInnerFn calls.
 *   mm_causal_conv1d_update  replaces `causal_conv1d_update(x, conv_state, weight, bias, activation)`
 *                            (call site mamba_simplemotif.py:352-358; fallback :353-358): each new
 *                            token is appended to conv_state (shifting it left) and the output is the
 *                            dot of the state's last W entries with the weights.
 *
 * Conventions as in mm_scan.h: device pointers, element strides, the seqlen dimension of the
 * forward's x/out contiguous, no allocation or synchronisation, 0 / MM_ERR_INVALID_ARGUMENT /
 * MM_ERR_UNSUPPORTED / hipError_t returns, message in mm_last_error(). Arithmetic in float32.
 */
#ifndef MM_CONV1D_H_
#define MM_CONV1D_H_

#include <stdint.h>

#include "mm_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest kernel width accepted (the package supports 2 to 4; Mamba uses d_conv = 4). */
#define MM_CONV1D_MAX_WIDTH 8

typedef struct mm_conv1d_fwd_params {
    int64_t batch, dim, seqlen, width;
    mm_dtype itype;              /* x, out, initial_states, final_states */
    mm_dtype wtype;              /* weight, bias */
    int32_t silu;                /* activation "silu" / "swish" */

    const void *x;               /* (batch, dim, seqlen) */
    const void *weight;          /* (dim, width) */
    const void *bias;            /* (dim,) or NULL */
    const void *initial_states;  /* (batch, dim, width - 1) or NULL */
    void *out;                   /* (batch, dim, seqlen) */
    void *final_states;          /* (batch, dim, width - 1) or NULL: the last width - 1 inputs */

    int64_t x_batch_stride, x_d_stride;
    int64_t out_batch_stride, out_d_stride;
    int64_t weight_d_stride, weight_w_stride;
    int64_t bias_stride;
    int64_t init_batch_stride, init_d_stride, init_w_stride;
    int64_t final_batch_stride, final_d_stride, final_w_stride;
} mm_conv1d_fwd_params;

typedef struct mm_conv1d_update_params {
    int64_t batch, dim, seqlen, width, state_len;   /* state_len >= width - 1 */
    mm_dtype itype;              /* x, out */
    mm_dtype wtype;              /* weight, bias */
    mm_dtype stype;              /* conv_state */
    int32_t silu;

    const void *x;               /* (batch, dim, seqlen) new tokens */
    void *conv_state;            /* (batch, dim, state_len), updated in place */
    const void *weight;          /* (dim, width) */
    const void *bias;            /* (dim,) or NULL */
    void *out;                   /* (batch, dim, seqlen) */

    int64_t x_batch_stride, x_d_stride, x_l_stride;
    int64_t state_batch_stride, state_d_stride, state_l_stride;
    int64_t out_batch_stride, out_d_stride, out_l_stride;
    int64_t weight_d_stride, weight_w_stride;
    int64_t bias_stride;
} mm_conv1d_update_params;

/* Backward of the forward above for a gradient `dout` of its output: dx (itype), and dweight,
 * dbias summed over batch and steps (float32, overwritten: one workgroup per channel sums them in a
 * fixed order and stores them, so repeated calls give the same bits). With `silu` the pre-activation is recomputed and dout is taken
 * through silu'. Replaces causal_conv1d_bwd_function(x, weight, bias, dout, seq_idx=None,
 * initial_states=None, dfinal_states=None, dx, return_dinitial_states=False, silu_activation)
 * (call site selective_scan_interface.py:635-637). */
typedef struct mm_conv1d_bwd_params {
    int64_t batch, dim, seqlen, width;
    mm_dtype itype;              /* x, dout, dx */
    mm_dtype wtype;              /* weight, bias */
    int32_t silu;

    const void *x;               /* (batch, dim, seqlen) */
    const void *weight;          /* (dim, width) */
    const void *bias;            /* (dim,) or NULL */
    const void *dout;            /* (batch, dim, seqlen) */
    void *dx;                    /* (batch, dim, seqlen) */
    float *dweight;              /* (dim, width) contiguous */
    float *dbias;                /* (dim,) or NULL */

    int64_t x_batch_stride, x_d_stride;
    int64_t dout_batch_stride, dout_d_stride;
    int64_t dx_batch_stride, dx_d_stride;
    int64_t weight_d_stride, weight_w_stride;
    int64_t bias_stride;
} mm_conv1d_bwd_params;

/* Causal depthwise conv1d forward. */
int mm_causal_conv1d_fwd(const mm_conv1d_fwd_params *params, void *stream);

/* Causal depthwise conv1d backward. */
int mm_causal_conv1d_bwd(const mm_conv1d_bwd_params *params, void *stream);

/* Decode update of the conv state; calls on one state must be ordered (same stream or events). */
int mm_causal_conv1d_update(const mm_conv1d_update_params *params, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MM_CONV1D_H_ */

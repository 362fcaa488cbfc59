/*
 * mm_norm.h -- C ABI of the row RMSNorm of libmm_scan.so (gfx950).
 *
 *   mm_rms_norm_fwd  replaces rms_norm_forward(x, weight, bias=None, eps, is_rms_norm=True)
 *                    (selective_scan_interface.py:217-234), which MambaInnerFn.forward applies to
 *                    B, C and delta when b_rms_weight / c_rms_weight / dt_rms_weight are given
 *                    (selective_scan_interface.py:515-529 and the recomputation at :576-593). The
 *                    reference computes it with the Triton _layer_norm_fwd of mamba_ssm (not
 *                    vendored); its published RMSNorm is
 *                        y[r, c] = x[r, c] * weight[c] / sqrt(mean_c x[r, c]^2 + eps)
 *                    in float32, written in x's dtype.
 *
 * The rows are addressed in the layout the scan reads, so no transposing copy is needed: x is
 * (n0, cols, n2) with element strides, and the norm runs over `cols` for every (i0, i2) -- for B
 * of shape (batch, 1, dstate, seqlen) that is n0 = batch, cols = dstate, n2 = seqlen.
 * Conventions as in mm_scan.h.
 */
#ifndef MM_NORM_H_
#define MM_NORM_H_

#include <stdint.h>

#include "mm_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mm_rms_norm_params {
    int64_t n0, cols, n2;
    mm_dtype itype;              /* x and out */
    mm_dtype wtype;              /* weight */
    float eps;

    const void *x;               /* (n0, cols, n2) */
    const void *weight;          /* (cols,) */
    void *out;                   /* (n0, cols, n2), may not overlap x unless identical */

    int64_t x_stride0, x_stride_c, x_stride2;
    int64_t out_stride0, out_stride_c, out_stride2;
    int64_t weight_stride;
} mm_rms_norm_params;

/* Row RMSNorm over `cols`. */
int mm_rms_norm_fwd(const mm_rms_norm_params *params, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MM_NORM_H_ */

// mm_internal.h -- declarations shared between the translation units of libmm_scan.so.
#pragma once

#include <hip/hip_runtime.h>

#include "mm_scan.h"

namespace mm {

// Records the launch status of the kernel just enqueued (hipGetLastError) and the error text.
int launch_status(const char *what);
// Records `msg` as the thread's last error and returns `code`.
int set_error(int code, const char *msg);

// True when every activation row start (u, delta, z, out, out_z, variable B/C) is 16-byte aligned
// and seqlen is a multiple of 8, so rows can be moved in 16-byte vectors.
bool fwd_vector_ok(const mm_scan_fwd_params *p);

// Tiled forward kernel (mm_scan_tiled.hip). Returns MM_ERR_UNSUPPORTED, without launching,
// when the request falls outside the shapes that kernel covers; the caller then uses the
// lane-per-row kernel.
template <typename T>
int try_launch_tiled(const mm_scan_fwd_params &p, hipStream_t stream);

// Number of sequence segments the dstate-16 kernels use for `p` (1: a single pass), and the
// workspace bytes that takes (mm_scan_tiled.hip).
int64_t segment_count(const mm_scan_fwd_params &p);
bool tile_states_ok(const mm_scan_fwd_params &p);
// The states before every 16-step tile, alone, into p.tile_states (the backward's checkpoints when
// the forward did not save them); MM_ERR_UNSUPPORTED without launching when tile_states_ok fails.
template <typename T>
int launch_states_only(const mm_scan_fwd_params &p, hipStream_t stream);
int64_t segment_workspace_bytes(const mm_scan_fwd_params &p, int64_t n_seg);

// SIMDs of the current device (4 per CU; cached per device), 1024 when it cannot be queried
// (mm_scan_tiled.hip).
int64_t device_simds();

// Forward scan with the low-rank P/Q coupling (mm_scan_pq.hip): the tiled kernel when the request
// fits it, else the lane-per-row kernel.
template <typename T>
int launch_pq(const mm_scan_fwd_params &p, hipStream_t stream, bool diag_x = false);

// The diagonal scan on the P/Q kernels with a zero rank-1 coupling (mm_scan_pq.hip), for diagonal
// requests the dstate-16 kernels do not take: diag_via_pq_fwd / diag_via_pq_bwd tell whether a
// request goes that way (inference forwards with dstate != 16 up to 64; backwards with dstate < 16),
// attach_zero_pair fills a copy of its parameters with the zero pair (and the gradient sink).
bool diag_via_pq_fwd(const mm_scan_fwd_params &p);
int attach_zero_pair(mm_scan_fwd_params &q);
bool diag_via_pq_bwd(const mm_scan_bwd_params &p);
int attach_zero_pair(mm_scan_bwd_params &q);

// Backward (mm_scan_bwd.hip): clears the accumulated gradients and launches the backward kernels
// on `stream`; bwd_workspace_bytes() is the scratch it uses best, bwd_workspace_min_bytes() the
// least it accepts (with tile states: without the segment carries, every unit then a whole row).
template <typename T>
int launch_bwd(const mm_scan_bwd_params &p, hipStream_t stream);
int64_t bwd_workspace_bytes(const mm_scan_bwd_params &p);
int64_t bwd_workspace_min_bytes(const mm_scan_bwd_params &p);

// Backward with the low-rank P/Q coupling (mm_scan_pq_bwd.hip): pq_bwd_ok() tells whether the
// request fits the kernel; launch_pq_bwd() runs it with the checkpoint scratch `ck` and the dB / dC
// partial slabs (the caller clears the accumulated gradients first and reduces the slabs after).
bool pq_bwd_ok(const mm_scan_bwd_params &p);
template <typename T>
int launch_pq_bwd(const mm_scan_bwd_params &p, hipStream_t stream, float *ck, float *partB, float *partC);
// The P/Q backward for the other shapes (dstate up to 256, constant B or C, any length and channel
// count): one lane per state, checkpoints `ck` of pq_general_ck_floats() floats, float32 atomics.
template <typename T>
int launch_pq_general(const mm_scan_bwd_params &p, hipStream_t stream, float *ck, float *partB, float *partC);
int64_t pq_general_ck_floats(const mm_scan_bwd_params &p);
int pq_general_rows_per_block(const mm_scan_bwd_params &p);

// The general backward kernels' dB/dC partial slabs (mm_scan_bwd.hip): when the rows a workgroup
// holds (rpb) all belong to one (batch, group) -- channels per group a multiple of rpb -- and the
// slabs stay under 4 GiB, each workgroup stores its sums over its rows into its own slab
// [block][batch][group][dstate][seqlen] and gen_slab_reduce adds the blocks in order (no atomics);
// gen_slab_floats() is 0 otherwise (the kernels then add with float32 atomics).
int64_t gen_slab_floats(const mm_scan_bwd_params &p, int64_t rpb);
int launch_gen_slab_reduce(const mm_scan_bwd_params &p, hipStream_t stream, const float *partB, const float *partC,
                           int64_t rpb);

}  // namespace mm

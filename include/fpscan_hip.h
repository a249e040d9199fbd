/*
 * fpscan_hip.h -- C ABI of the MI355X (gfx950) first-order linear-recurrence scan.
 *
 *   forward:  y[t] = gates[t] * y[t-1] + tokens[t],   y[-1] = 0
 *   reverse:  y[t] = gates[t] * y[t+1] + tokens[t],   y[L]  = 0
 *   backward: grad_tokens[t] = grad_out[t] + gates[t+1] * grad_tokens[t+1]  (gates[L] = 1)
 *             grad_gates[t]  = grad_tokens[t] * y[t-1]                     (y[-1]   = 0)
 *
 * Tensors are (batch, dim, seqlen) with the seqlen axis contiguous; row (b, d) starts at
 * element offset b*stride_b + d*stride_d. Every tensor passed to one call shares that layout.
 * Element types: fp32, fp16 and bf16; all arithmetic is fp32, outputs are rounded to
 * nearest-even once. seqlen must be a power of two in [32, 65536], as in the reference.
 *
 * All scan entry points are asynchronous on `stream` (a hipStream_t; NULL = the null
 * stream), allocate nothing and are safe to call from several host threads. Pointers are
 * device pointers on the current HIP device; they must be 16-byte aligned and the strides
 * must be multiples of 16 bytes (16/itemsize elements).
 *
 * State the library keeps: (1) process-wide tuning and test hooks -- fpscan_set_tiling,
 * fpscan_set_launch_override, fpscan_set_lookback_test_hook -- which change the path taken
 * (and so fpscan_workspace_bytes' answer and the fp32 rounding order), never the recurrence;
 * they are meant for tests and tuning sweeps and are not synchronised with calls in flight;
 * (2) per device: a count of look-back waits that gave up (fpscan_lookback_overruns), and the
 * static scratch of fpscan_scan_fwd_noalloc.
 *
 * Look-back waits: the tiled paths chain tiles through status words and each wait for an
 * earlier tile is bounded. A wait that gives up -- which a correct launch never does, but a
 * predecessor stalled for tens of milliseconds (preemption, another process) could cause --
 * makes its tile's outputs, and everything computed from them, NaN instead of plausible
 * values, and counts itself in a per-device counter that fpscan_lookback_overruns reads.
 *
 * Workspace: large problems run fastest on the tiled path, which needs
 * fpscan_workspace_bytes() bytes of device memory (one 8-byte word per tile plus 1152 bytes
 * of counters, about 0.05 % of one tensor). Pass a buffer of at least that size, 8-byte
 * aligned, owned by the caller and not used by any other call in flight. Its contents are
 * overwritten. With no workspace (or a smaller one) the call takes the row-streaming path
 * instead: same results up to fp32 rounding order, somewhat lower bandwidth. The tiled path
 * is an ordinary launch that needs no co-residency (workgroups claim tiles in order); if the
 * occupancy query fails, the call streams rows.
 *
 * Reference interface replaced (saeeddhqan/fpscan):
 *   csrc/main.cpp:7-11              PYBIND11_MODULE: "fullscan_forward" -> warpscan_fwd
 *   csrc/full_scan/full_scan.h:26-36 warpscan_fwd(Ax, Bx, out, reverse)
 *   csrc/full_scan/full_scan.cu:179-258 warpscan<T> / warpscan_forward (dtype dispatch,
 *                                    tile table, launch on the current stream)
 *   fpscan/ops.py:69-83             PScan.backward (7 ATen ops + a reverse scan), fused here
 */
#ifndef FPSCAN_HIP_H
#define FPSCAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FPSCAN_ABI_VERSION 1

/* Element type codes (the reference dispatches on the same three types,
 * full_scan.cu:245-256). */
#define FPSCAN_DTYPE_F32 0
#define FPSCAN_DTYPE_F16 1
#define FPSCAN_DTYPE_BF16 2

/* Operation codes for fpscan_workspace_bytes. */
#define FPSCAN_OP_FWD 0
#define FPSCAN_OP_BWD 1

/* Status codes. The reference raises RuntimeError through TORCH_CHECK for the first
 * three conditions (full_scan.cu:181-182, 232, 240-256); the binding maps every nonzero
 * status to RuntimeError with fpscan_strerror's text. */
#define FPSCAN_OK 0
#define FPSCAN_ERR_SEQLEN 1    /* seqlen not a power of two in [32, 65536] */
#define FPSCAN_ERR_DTYPE 2     /* dtype code not one of FPSCAN_DTYPE_* */
#define FPSCAN_ERR_SHAPE 3     /* negative batch/dim/stride, rows that overlap, or a tensor
                                  span of 2^48 bytes or more */
#define FPSCAN_ERR_ALIGN 4     /* pointer or stride not 16-byte aligned */
#define FPSCAN_ERR_NULL 5      /* null data pointer with a non-empty problem */
#define FPSCAN_ERR_WORKSPACE 6 /* workspace smaller than fpscan_workspace_bytes() */
#define FPSCAN_ERR_LAUNCH 7    /* hipGetLastError() reported a failure after the launch */
#define FPSCAN_ERR_DEVICE 8    /* the current device could not be queried */
#define FPSCAN_ERR_SCRATCH 9   /* tiled problem larger than fpscan_scan_fwd_noalloc's scratch */

/* Forward or reverse scan.
 * Replaces warpscan_fwd / warpscan_forward (csrc/full_scan/full_scan.h:26-36,
 * csrc/full_scan/full_scan.cu:238-258); `gates`/`tokens` are the reference's Ax/Bx and
 * `out` is written in full (the reference's caller allocates it, fpscan/ops.py:55-56).
 * `out` may alias `tokens` or `gates` exactly (in-place scan), never partly: the library does
 * not check pointer ranges (the torch binding refuses partial overlaps). */
int fpscan_scan_fwd(const void* gates, const void* tokens, void* out,
                    int64_t batch, int64_t dim, int64_t seqlen,
                    int64_t stride_b, int64_t stride_d,
                    int dtype, int reverse,
                    void* workspace, size_t workspace_bytes, void* stream);

/* fpscan_scan_fwd without a workspace argument and without any allocation: the tiled path's
 * status words and claim counters live in a static device array of the library (2 MiB + 1152
 * bytes per device, held until the process ends, found with hipGetSymbolAddress on the first
 * call on each device), so calls make no hipMalloc/hipFree and no allocating library call.
 * Same results and paths as fpscan_scan_fwd with a large enough workspace. A problem whose
 * tiled plan needs more than 262144 tiles (rows * seqlen / (8192 for 2-byte types, 4096 for
 * fp32) when it tiles) returns FPSCAN_ERR_SCRATCH. Every call on one device shares that
 * device's scratch and clears it at the start: calls that overlap on one device (other
 * streams, other host threads) race and must be serialised by the caller.
 * No counterpart in the reference (its kernel needs no scratch); for callers that cannot
 * allocate: tight serving loops and harnesses that forbid hipMalloc. HIP graph capture of
 * this library's kernels is untested: the one capture that was run (through torch's
 * torch.cuda.graph, streaming kernels) ended with a host segmentation fault during graph
 * instantiation, with no cause found, and the torch binding refuses capture since; no
 * capture through this entry point has been run. */
int fpscan_scan_fwd_noalloc(const void* gates, const void* tokens, void* out,
                            int64_t batch, int64_t dim, int64_t seqlen,
                            int64_t stride_b, int64_t stride_d,
                            int dtype, int reverse, void* stream);

/* Fused backward of the forward scan, given the saved forward output `out`.
 * Replaces the composition in PScan.backward (fpscan/ops.py:69-83): shifted-gate copy,
 * reverse scan (full_scan.cu:198-200), shifted-output copy and the product, in one pass
 * that reads gates, out and grad_out and writes grad_gates and grad_tokens. */
int fpscan_scan_bwd(const void* gates, const void* out, const void* grad_out,
                    void* grad_gates, void* grad_tokens,
                    int64_t batch, int64_t dim, int64_t seqlen,
                    int64_t stride_b, int64_t stride_d,
                    int dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Device workspace, in bytes, that the tiled path of fpscan_scan_fwd (op FPSCAN_OP_FWD) or
 * fpscan_scan_bwd (FPSCAN_OP_BWD) uses for this problem; 0 when the problem takes the
 * row-streaming path (which needs none). The two can differ: the backward tiles from a
 * smaller size on long rows.
 * No reference counterpart: the reference kernel keeps its carries in shared memory
 * (full_scan.cu:55-57). */
size_t fpscan_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int dtype, int op);

/* Channel-last scan: tensors (batch, seqlen, dim) with the dim axis contiguous, element
 * (b, t, d) at b*stride_b + t*stride_t + d, the recurrence running along seqlen:
 *   y[b,t,d] = gates[b,t,d] * y[b,t-1,d] + tokens[b,t,d]   (reverse: y[b,t+1,d]).
 * Same semantics as fpscan_scan_fwd on the transposed data (first gate ignored, zero initial
 * state, fp32 arithmetic), without the transposes. Any seqlen >= 1; dim, stride_t and
 * stride_b multiples of 16/itemsize elements; pointers 16-byte aligned; `out` may alias
 * `tokens` or `gates` exactly. With at least 512 strips of 64 16-byte vectors
 * (batch * dim / (64 * 16/itemsize)) and less than 512 MiB per tensor, one wave scans each
 * strip in one pass. Otherwise the time axis is tiled and needs fpscan_workspace_bytes_cl()
 * bytes of workspace: a single pass whose tiles (64 columns by 128 steps, 64 in fp32) look
 * back along time (3 N s bytes forward, results independent of timing). Where a tile does
 * not apply (seqlen within one tile, or a tile's rows beyond a 2 GiB buffer range), fewer
 * than 512 strips take segments (aggregates, carries, then the segments again: 5 N s bytes)
 * and more take the one pass. Without the workspace the call runs one pass per strip
 * (correct, slower), except that a batch slab of more than about 2 GiB needs the workspace
 * (FPSCAN_ERR_WORKSPACE otherwise). Calls sharing a workspace must not overlap.
 * No reference counterpart: the reference supports (batch, dim, seqlen) only and tells callers
 * of this layout to transpose in and out (README.md:94-99). */
int fpscan_scan_fwd_cl(const void* gates, const void* tokens, void* out,
                       int64_t batch, int64_t seqlen, int64_t dim,
                       int64_t stride_b, int64_t stride_t,
                       int dtype, int reverse,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Fused backward of fpscan_scan_fwd_cl (forward direction), given its output `out`:
 *   grad_tokens[b,t,d] = grad_out[b,t,d] + gates[b,t+1,d] * grad_tokens[b,t+1,d]  (gates[b,L,d] = 1)
 *   grad_gates[b,t,d]  = grad_tokens[b,t,d] * out[b,t-1,d]                      (out[b,-1,d] = 0)
 * Same layout rules as fpscan_scan_fwd_cl; outputs must not alias inputs. No reference
 * counterpart (the reference composes its backward from ATen ops, fpscan/ops.py:69-83). */
int fpscan_scan_bwd_cl(const void* gates, const void* out, const void* grad_out,
                       void* grad_gates, void* grad_tokens,
                       int64_t batch, int64_t seqlen, int64_t dim,
                       int64_t stride_b, int64_t stride_t,
                       int dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Workspace, in bytes, for the tiled or segmented channel-last path this problem takes (0: one
 * pass per strip); it depends on fpscan_set_tiling's setting. */
size_t fpscan_workspace_bytes_cl(int64_t batch, int64_t seqlen, int64_t dim, int64_t stride_t,
                                 int dtype, int op);

/* Scan with the gates produced inside the kernel: gates[b,d,t] = exp(-softplus(z[b,d,t]) *
 * rate[d]) (a Mamba-style decay, delta = softplus(z), A = -rate), so that the gates tensor is
 * never written or read: 3 N s bytes for the forward instead of 5 N s for "compute gates,
 * then scan". z and tokens as `gates`/`tokens` of fpscan_scan_fwd; rate: fp32, `dim` values,
 * 4-byte aligned. Always takes the row-streaming path (no workspace). No reference
 * counterpart (the reference scans materialised gates). */
int fpscan_scan_fwd_softplus(const void* z, const float* rate, const void* tokens, void* out,
                             int64_t batch, int64_t dim, int64_t seqlen,
                             int64_t stride_b, int64_t stride_d,
                             int dtype, int reverse, void* stream);

/* Fused backward of fpscan_scan_fwd_softplus (forward direction), given its output `out`:
 * grad_tokens as fpscan_scan_bwd; grad_z = grad_gates * gate * (-rate) * sigmoid(z); and, if
 * grad_rate_rows is not NULL, one fp32 partial sum of grad_gates * gate * (-softplus(z)) per
 * (b, d) row (batch * dim floats, index b * dim + d; summing over b gives d loss / d rate). */
int fpscan_scan_bwd_softplus(const void* z, const float* rate, const void* out,
                             const void* grad_out, void* grad_z, void* grad_tokens,
                             float* grad_rate_rows,
                             int64_t batch, int64_t dim, int64_t seqlen,
                             int64_t stride_b, int64_t stride_d,
                             int dtype, void* stream);

/* Contraction scan, in place into `tokens` (the reference's Bx):
 * replaces dimwise_forward / dimwise_fwd / dimwise_pscan (csrc/main.cpp:10,
 * csrc/dimwise/dimwise.h:27-42, csrc/dimwise/dimwise_scan_final.cu:387-576).
 * gates/tokens: (batch, dim, seqlen) contiguous; bh: (batch, dim, G) contiguous with
 * G = fpscan_dimwise_groups(seqlen); wq, wk: dim elements. All five share `dtype`.
 * seqlen a power of two in [64, 65536] (the reference rejects 32 and everything else too).
 * Per row, in chunks of W groups: zero-initial-state group scans (group 0 continues from the
 * previous chunk), then each group g >= 1 adds r[g-1], where r mixes the group ends v through
 * a first-maximum selection of (1+Wk)*Bh[h] * (1+Wq)*v[g] over earlier groups h. fp32
 * arithmetic with one rounding, except the selection's k, q and scores, which are rounded as
 * the reference rounds them in the tensors' type. Runs on `stream` (the reference uses the
 * legacy default stream). No backward (the reference has none). Takes the row kernel (one
 * workgroup per row); fpscan_dimwise_fwd_ws with a workspace can take the faster tiled path. */
int fpscan_dimwise_fwd(const void* gates, void* tokens, const void* bh, const void* wq,
                       const void* wk, int64_t batch, int64_t dim, int64_t seqlen, int dtype,
                       void* stream);

/* fpscan_dimwise_fwd with a workspace: problems of 384 MiB to 4 GiB per tensor with rows of
 * at least 64 KiB (seqlen * itemsize) then take a tiled path, whose 16 KiB tiles are
 * claimed in memory order and chained by a look-back over the chunks' carry maps (the carry
 * enters a chunk affinely: only group 0 depends on it, and the selection does not), with
 * bounded waits as the tiled scans'. It needs fpscan_dimwise_workspace_bytes() bytes, 8-byte
 * aligned, owned by the caller and not used by any call in flight; with no workspace or a
 * smaller one the call takes the row kernel. Same results up to fp32 rounding order, except
 * where the selection finds no score above the initial one (non-finite or |score| >= 1e10
 * inputs): the non-finite outputs may then differ in kind. fpscan_set_tiling applies (1: row
 * kernel only; 2: tiled for any seqlen of 8192 or more, where every chunk is 32 groups of 128,
 * below 4 GiB per tensor). The reference's dimwise_forward takes
 * no workspace: the torch binding allocates it from the caching allocator. */
int fpscan_dimwise_fwd_ws(const void* gates, void* tokens, const void* bh, const void* wq,
                          const void* wk, int64_t batch, int64_t dim, int64_t seqlen, int dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Workspace, in bytes, that fpscan_dimwise_fwd_ws uses for this problem (0: it takes the row
 * kernel, or the arguments are invalid). No reference counterpart. */
size_t fpscan_dimwise_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int dtype);

/* Number of Bh entries per row (G = W * C) that fpscan_dimwise_fwd expects for this seqlen,
 * 0 if seqlen is not supported. Only the first W (<= 32) are read: the reference indexes Bh
 * without the chunk (dimwise_scan_final.cu:133, :189). */
int fpscan_dimwise_groups(int64_t seqlen);

/* Static description of a status code (never NULL). The reference's equivalent is the
 * TORCH_CHECK message text (full_scan.h:7-9). */
const char* fpscan_strerror(int status);

/* FPSCAN_ABI_VERSION of the loaded library. */
int fpscan_abi_version(void);

/* Look-back waits (row, channel-last and dimwise tiled kernels) that gave up on the current device
 * since the library was loaded; 0 in a correct run. Waits for all work on the device first
 * (hipDeviceSynchronize), then copies the device counters. No reference counterpart: the
 * reference keeps every carry inside one block (full_scan.cu:77-175) and has no such wait. */
int fpscan_lookback_overruns(unsigned long long* count);

/* Test hook, process-wide: the tiled kernels never publish the map(s) of tile
 * `unpublished_tile` (a tile index in claim order; -1: none), and a look-back wait gives up
 * after `spin_limit` polls (0: the default, 65536 polls of about 1 us). Lets a test force a
 * wait to give up while every kernel still exits normally. No reference counterpart. */
int fpscan_set_lookback_test_hook(int64_t unpublished_tile, int spin_limit);

/* Launch-shape override for tuning sweeps (a tuning hook); process-wide, not synchronised
 * with calls in flight on other threads. waves_per_row in {0,1,2,4,8,16}, ring_depth in 0..4;
 * 0 restores the built-in choice. Every setting computes the same recurrence; only the
 * grouping of fp32 partial products (and so the last-bit rounding) changes. The ring
 * depth never changes results. No reference counterpart: the
 * reference fixes its tiles at compile time (full_scan.cu:207-233). */
int fpscan_set_launch_override(int waves_per_row, int ring_depth);

/* Path selection for tests and tuning (a test hook); process-wide, not synchronised with
 * calls in flight. 0: automatic (rows: tiled for problems of at least 512 MiB per tensor,
 * backward from 256 MiB with rows of 64 KiB or more, rows of exactly 16 sub-chunks from 1 GiB
 * except the 2-byte backward, which streams them; channel-last: tiled look-back when one pass
 * per strip lacks strips or from 512 MiB per tensor; dimwise: tiled for rows of 64 KiB or
 * more from 384 MiB per tensor), 1: no tiled look-back (rows streamed; channel-last one pass
 * or segments; dimwise's row kernel), 2: tiled whenever possible (rows with 16..1024
 * sub-chunks; any channel-last problem whose 130-row tile fits a 2 GiB buffer range; dimwise
 * seqlen 8192..65536 below 4 GiB per tensor). Tiled paths need the workspace. No reference
 * counterpart. */
int fpscan_set_tiling(int mode);

#ifdef __cplusplus
}
#endif

#endif /* FPSCAN_HIP_H */

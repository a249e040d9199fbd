/* Bandwidth probes of the fpscan library (libfpscan_hip.so): copy kernels with the access
 * patterns of the scan kernels and none of their arithmetic, so that the scans can be
 * measured against what their own memory-access order reaches on the device (bench.py
 * --workload ceiling). Measurement aids with no counterpart in the reference (its repository
 * has no bandwidth probe); the scans do not use them. */
#ifndef FPSCAN_PROBE_H
#define FPSCAN_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Access patterns */
#define FPSCAN_PROBE_TILES 0  /* 16 KiB tiles claimed in order from 8 counters by a persistent
                                 grid of 1024-thread workgroups, two tiles in flight each (the
                                 tiled scans' scheme) */
#define FPSCAN_PROBE_BLOCKS 1 /* one 64-thread workgroup per 2 KiB, dispatched in memory order
                                 (the row scan on rows of one sub-chunk) */
#define FPSCAN_PROBE_ROWS 2   /* one 1024-thread workgroup per row of row_bytes, 16 KiB rounds,
                                 four in flight (the row-streaming scan, 16 waves per row) */
#define FPSCAN_PROBE_BLOCKS_LOOKBACK 3 /* 256-thread blocks, one 16 KiB tile each, in memory
                                 order; after its loads a block publishes a word and waits
                                 (bounded) until every earlier tile of its row of row_bytes
                                 has published, as a single-pass scan in memory order would */
#define FPSCAN_PROBE_ROWS8 4  /* one 512-thread workgroup per row of row_bytes, 8 KiB rounds,
                                 two in flight (dimwise_forward's row kernel; the row scans'
                                 eight-wave rows) */
#define FPSCAN_PROBE_TILES8 5 /* as FPSCAN_PROBE_TILES with 8 KiB tiles and 512-thread
                                 workgroups, two per CU (a tile size the tiled kernels do not
                                 use, for comparison) */

#define FPSCAN_PROBE_OK 0
#define FPSCAN_PROBE_ERR_ARG 1    /* unknown pattern or read/write count, bad size, alignment,
                                     or a missing scratch buffer for the tile patterns */
#define FPSCAN_PROBE_ERR_LAUNCH 2 /* the launch failed */
#define FPSCAN_PROBE_ERR_DEVICE 3 /* the current device or the kernel's occupancy could not be
                                     queried */

/* Bytes of device scratch FPSCAN_PROBE_TILES and FPSCAN_PROBE_TILES8 need for their claim
 * counters (cleared by the call, on the stream, before the copy). */
size_t fpscan_probe_scratch_bytes(void);

/* Bytes of device scratch FPSCAN_PROBE_BLOCKS_LOOKBACK needs for tensors of tensor_bytes: two
 * counters (tiles that had to poll, waits that gave up) and one word per 16 KiB tile. Zero it
 * once before the first call; the words carry a per-call epoch, so later calls need no clear
 * and the counters accumulate. */
size_t fpscan_probe_lookback_scratch_bytes(int64_t tensor_bytes);

/* dst[o] = src[0] + (o + 1) * (src[1] + ... ) as 32-bit integer vectors, for nread inputs laid
 * out back to back at `src` (nread * tensor_bytes bytes) and nwrite outputs back to back at
 * `dst`; (nread, nwrite) is (2, 1) -- the forward scan's traffic -- or (3, 2) -- the fused
 * backward's. tensor_bytes: a multiple of 16 KiB, at most 4 GiB; row_bytes: for
 * FPSCAN_PROBE_ROWS, FPSCAN_PROBE_ROWS8 and FPSCAN_PROBE_BLOCKS_LOOKBACK a multiple of 16 KiB
 * that divides tensor_bytes (ignored otherwise). Pointers 16-byte aligned. Enqueued on
 * `stream` (a hipStream_t; NULL for the default stream). */
int fpscan_probe_copy(int pattern, int nread, int nwrite, const void* src, void* dst,
                      int64_t tensor_bytes, int64_t row_bytes, void* scratch,
                      size_t scratch_bytes, void* stream);

/* The channel-last tiled scan's pattern (fpscan_scan_fwd_cl / _bwd_cl on the tiled path):
 * tensors of `batch` x `seqlen` time rows of row_bytes (a (batch, seqlen, dim) tensor with
 * row_bytes = dim * itemsize), cut into chains of strip_bytes columns (128: 64 columns of a
 * 2-byte type; 256: 64 fp32 columns) over all time rows and tiles of 16 KiB of one chain,
 * claimed by a persistent grid from 8 counters, one per eighth of the chains, all of a
 * group's chains' first tiles first; two tiles in flight per workgroup. Same outputs as
 * fpscan_probe_copy. seqlen a multiple of 16 KiB / strip_bytes; row_bytes a multiple of
 * strip_bytes; at most 4 GiB per tensor; scratch as for FPSCAN_PROBE_TILES. */
int fpscan_probe_copy_cl(int nread, int nwrite, const void* src, void* dst, int64_t batch,
                         int64_t seqlen, int64_t row_bytes, int strip_bytes, void* scratch,
                         size_t scratch_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FPSCAN_PROBE_H */

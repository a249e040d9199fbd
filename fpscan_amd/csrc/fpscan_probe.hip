// Bandwidth probes: copy kernels that move the same bytes in the same order as this library's
// scan kernels, without the scan. Each output tensor is a sum of the input tensors (so every
// load is consumed) and every access is a 16-byte nontemporal one, as in the scan kernels.
// What one of them reaches on a device is the ceiling of that access pattern there; bench.py
// (--workload ceiling) times them beside the scans. No counterpart in the reference.
//
// Patterns (FPSCAN_PROBE_*, include/fpscan_probe.h):
//   TILES   16 KiB tiles of each tensor claimed in order from 8 counters, one per contiguous
//           eighth of the tiles, by a persistent grid of 1024-thread workgroups (the claim
//           scheme of the tiled scans, scan_common.h): two tiles in flight per workgroup and
//           the next claim issued before the current tile's stores.
//   BLOCKS  one 64-thread workgroup per 2 KiB of each tensor, dispatched in memory order
//           (the pattern of the row scan on rows of one sub-chunk, one wave per row).
//   ROWS    one 1024-thread workgroup per row of `row_bytes`, walked in 16 KiB rounds with four
//           rounds in flight (the pattern of the row-streaming scan with 16 waves per row).
//   ROWS8   one 512-thread workgroup per row, 8 KiB rounds, two in flight (the pattern of
//           dimwise_forward's row kernel and of the row scans with eight waves per row).
//   TILES8  as TILES with 8 KiB tiles and 512-thread workgroups, two per CU: the tile size
//           the tiled kernels do not use, for comparison with TILES.
//   BLOCKS_LOOKBACK  256-thread blocks of 16 KiB tiles in memory order, each waiting before its
//           stores until every earlier tile of its row has loaded its data: the wait a
//           single-pass scan in memory order needs.
//   channel-last tiles (fpscan_probe_copy_cl): (batch, seqlen, dim) tensors cut into chains of
//           64 columns over all time rows and tiles of 16 KiB of one chain (128 time rows of
//           128-byte strips, or 64 of 256-byte strips), claimed like TILES but per chain
//           group, all of a group's chains' first tiles, then their second ones, and so on;
//           lanes hold consecutive 16-byte pieces of a time row (the channel-last tiled scan).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "fpscan_probe.h"
#include "scan_common.h"

namespace {

constexpr int kTileBytes = 16 << 10;  // 1024 lanes x 16 bytes

template <int NR, int NW>
__device__ __forceinline__ void combine_store(const u32x4 (&v)[NR], const Rsrc (&out)[NW],
                                              uint32_t off) {
#pragma unroll
  for (int o = 0; o < NW; ++o) {
    u32x4 s = v[0];
#pragma unroll
    for (int i = 1; i < NR; ++i) s += v[i] * (unsigned)(o + 1);
    bst16(out[o], off, s);
  }
}

// Tile geometries of probe_tiles: the claim groups, where a tile lies in a tensor and this
// lane's byte offset in it.
// Row tiles: TB bytes contiguous (one 16-byte vector per lane), groups of contiguous eighths.
template <int TB>
struct RowTileGeo {
  int64_t ntiles;
  __device__ RowGroups groups() const { return RowGroups{ntiles, 0}; }
  __device__ uint32_t lane_off() const { return threadIdx.x * 16u; }
  __device__ Rsrc rsrc(const char* base, int64_t t) const {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + t * TB, (short)0, TB,
                                             kRsrcWord3);
  }
};

// Claim groups over chains (the channel-last scan's): group g holds chains
// [g chains / 8, (g + 1) chains / 8), tiles numbered segment-major inside a group.
struct ChainTileGroups {
  int64_t chains;
  int64_t nseg;
  __device__ int64_t chain_lo(int g) const {
    return (int64_t)(((uint64_t)g * (uint64_t)chains) / kClaimGroups);
  }
  __device__ int64_t first(int g) const { return chain_lo(g) * nseg; }
};

// Channel-last tiles: chain = (batch, strip of strip_bytes), tile = tile_rows time rows of
// one chain; lane l of wave w holds piece l % pieces of time row w * (64 / pieces) + l / pieces.
struct ClTileGeo {
  int64_t seqlen;
  int64_t row_bytes;  // one time row of one batch
  int64_t strips;     // chains per batch
  int strip_bytes;    // 128 or 256
  int tile_rows;      // 16 KiB / strip_bytes
  ChainTileGroups cg;
  __device__ ChainTileGroups groups() const { return cg; }
  __device__ uint32_t lane_off() const {
    const int pieces = strip_bytes >> 4;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    return (uint32_t)((w * (64 / pieces) + lane / pieces) * row_bytes + (lane % pieces) * 16);
  }
  __device__ Rsrc rsrc(const char* base, int64_t t) const {
    int g = 0;
#pragma unroll
    for (int i = 1; i < kClaimGroups; ++i) g += t >= cg.first(i) ? 1 : 0;
    const int64_t c_lo = cg.chain_lo(g);
    const uint32_t nch = (uint32_t)(cg.chain_lo(g + 1) - c_lo);
    const uint32_t k = (uint32_t)(t - c_lo * cg.nseg);
    // uniform integer divisions run on the vector unit: bring the results back to scalars
    const uint32_t seg = __builtin_amdgcn_readfirstlane(k / nch);
    const int64_t chain = c_lo + (int64_t)(k - seg * nch);
    const uint32_t b = __builtin_amdgcn_readfirstlane((uint32_t)chain / (uint32_t)strips);
    const int64_t strip = chain - (int64_t)b * strips;
    const int64_t start = ((int64_t)b * seqlen + (int64_t)seg * tile_rows) * row_bytes +
                          strip * strip_bytes;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base) + start, (short)0,
        (int)((int64_t)(tile_rows - 1) * row_bytes + strip_bytes), kRsrcWord3);
  }
};

template <int NR, int NW, class Geo, int THREADS>
__global__ void __launch_bounds__(THREADS)
probe_tiles(const char* __restrict__ src, char* __restrict__ dst, int64_t tensor_bytes,
            uint64_t* __restrict__ status, int64_t ntiles, const Geo geo) {
  const bool leader = threadIdx.x == 0;
  const uint32_t lane_off = geo.lane_off();
  const Rsrc st = __builtin_amdgcn_make_buffer_rsrc(
      status, (short)0, (int)(kStatusExtraWords * sizeof(uint64_t)), kRsrcWord3);
  // the status buffer holds no tile words here: the counters start at word kCounterStride
  Claims<decltype(geo.groups())> claims{(uint32_t)(kCounterStride * sizeof(uint64_t)),
                                        reinterpret_cast<const uint32_t*>(status + kCounterStride),
                                        geo.groups(), (int)(blockIdx.x % kClaimGroups)};
  const int64_t kBubble = ntiles, kDone = ntiles + 1;
  __shared__ int64_t next_tile;

  auto tile_rsrc = [&](const char* base, int64_t t) { return geo.rsrc(base, t); };
  auto load = [&](int64_t t, u32x4 (&v)[NR]) {
    const int64_t tt = t < ntiles ? t : 0;
    const uint32_t off = t < ntiles ? lane_off : kNoOffset;
#pragma unroll
    for (int i = 0; i < NR; ++i) v[i] = bld16(tile_rsrc(src + i * tensor_bytes, tt), off);
  };

  // the claim for the tile after the next one, made by the leader (and waited for) while the
  // other waves store the current tile
  // LDS-only barriers (scan_common.h): __syncthreads would also wait for every load in flight
  auto claim_after = [&](int64_t known) {
    lds_barrier();
    if (leader) next_tile = known < ntiles ? claims.next_now(st, kBubble, kDone) : kDone;
  };
  auto store = [&](int64_t t, const u32x4 (&v)[NR]) {
    Rsrc out[NW];
#pragma unroll
    for (int o = 0; o < NW; ++o) out[o] = tile_rsrc(dst + o * tensor_bytes, t);
    combine_store<NR, NW>(v, out, lane_off);
  };
  auto claimed = [&]() {
    lds_barrier();
    return (int64_t)__builtin_amdgcn_readfirstlane(next_tile);
  };

  if (leader) next_tile = claims.next_now(st, kBubble, kDone);
  int64_t t_a = claimed();
  claim_after(t_a);
  int64_t t_b = claimed();
  // two ring slots, a and b, each holding one tile's loads; while one slot's tile is stored,
  // the other's loads are in flight
  u32x4 a[NR], b[NR];
  load(t_a, a);
  load(t_b, b);
  for (;;) {
    if (t_a >= ntiles) break;
    claim_after(t_b);
    store(t_a, a);
    t_a = claimed();
    load(t_a, a);
    if (t_b >= ntiles) break;
    claim_after(t_a);
    store(t_b, b);
    t_b = claimed();
    load(t_b, b);
  }
}

template <int NR, int NW>
__global__ void __launch_bounds__(64)
probe_blocks(const char* __restrict__ src, char* __restrict__ dst, int64_t tensor_bytes) {
  constexpr int kBlockBytes = 2 << 10;  // two 1 KiB sub-chunks per wave
  const int64_t base = (int64_t)blockIdx.x * kBlockBytes;
  const uint32_t lane_off = threadIdx.x * 16u;
  u32x4 v[2][NR];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < NR; ++i)
      v[s][i] = bld16(row_rsrc(src + i * tensor_bytes, base, 1, kBlockBytes),
                      s * 1024u + lane_off);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    Rsrc out[NW];
#pragma unroll
    for (int o = 0; o < NW; ++o) out[o] = row_rsrc(dst + o * tensor_bytes, base, 1, kBlockBytes);
    combine_store<NR, NW>(v[s], out, s * 1024u + lane_off);
  }
}

// Memory-order blocks with the wait a single-pass scan in that order needs: 256-thread
// blocks, each one 16 KiB tile of every tensor (four 1 KiB sub-chunks per wave), dispatched in
// memory order. Once all four waves hold their data, wave 0 publishes one word for the tile
// and waits until every earlier tile of its row (a row = row_bytes of each tensor, at most 64
// tiles looked at) has published; then the block stores. Words carry the call's epoch, so the
// scratch needs no clear between calls. The wait is bounded (kSpinLimit polls); the number of
// tiles that had to poll and of waits that gave up are counted in the scratch's first words.
constexpr int kLookbackTileBytes = 16 << 10;

template <int NR, int NW>
__global__ void __launch_bounds__(256)
probe_blocks_lookback(const char* __restrict__ src, char* __restrict__ dst, int64_t tensor_bytes,
                      int row_tiles, uint32_t* __restrict__ words, uint32_t epoch) {
  constexpr int kSubs = 4;
  const int64_t tile = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t base = tile * kLookbackTileBytes + (int64_t)w * (kSubs << 10);
  const uint32_t lane_off = lane * 16u;
  u32x4 v[kSubs][NR];
#pragma unroll
  for (int s = 0; s < kSubs; ++s)
#pragma unroll
    for (int i = 0; i < NR; ++i)
      v[s][i] = bld16(row_rsrc(src + i * tensor_bytes, base, 1, kSubs << 10), s * 1024u + lane_off);
  // each wave waits for all of its loads, then the barrier: past it the whole tile has arrived
  // (a scan's reduce could start here)
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  uint32_t* status = words + 2;  // [0] tiles that polled, [1] waits that gave up
  if (w == 0) {
    if (lane == 0)
      __hip_atomic_store(status + tile, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int seg = (int)(tile % row_tiles);
    const bool mine = lane < seg;
    for (int it = 0;; ++it) {
      const uint32_t wd = mine ? __hip_atomic_load(status + tile - 1 - lane, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : epoch;
      if (__builtin_amdgcn_ballot_w64(wd != epoch) == 0) {
        if (it > 0 && lane == 0)
          __hip_atomic_fetch_add(words, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if (it >= kSpinLimit) {
        if (lane == 0)
          __hip_atomic_fetch_add(words + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  lds_barrier();
#pragma unroll
  for (int s = 0; s < kSubs; ++s) {
    Rsrc out[NW];
#pragma unroll
    for (int o = 0; o < NW; ++o) out[o] = row_rsrc(dst + o * tensor_bytes, base, 1, kSubs << 10);
    combine_store<NR, NW>(v[s], out, s * 1024u + lane_off);
  }
}

template <int NR, int NW, int W, int U>
__global__ void __launch_bounds__(64 * W)
probe_rows(const char* __restrict__ src, char* __restrict__ dst, int64_t tensor_bytes,
           int64_t row_bytes) {
  constexpr int kRoundBytes = W * 1024;  // one 16-byte vector per lane
  const int64_t base = (int64_t)blockIdx.x * row_bytes;
  const int nrounds = (int)(row_bytes / kRoundBytes);
  const uint32_t lane_off = threadIdx.x * 16u;
  Rsrc in[NR], out[NW];
#pragma unroll
  for (int i = 0; i < NR; ++i) in[i] = row_rsrc(src + i * tensor_bytes, base, 1, (int)row_bytes);
#pragma unroll
  for (int o = 0; o < NW; ++o) out[o] = row_rsrc(dst + o * tensor_bytes, base, 1, (int)row_bytes);
  auto off_of = [&](int r) { return r < nrounds ? (uint32_t)r * kRoundBytes + lane_off : kNoOffset; };
  u32x4 ring[U][NR];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < NR; ++i) ring[u][i] = bld16(in[i], off_of(u));
  for (int r0 = 0; r0 < nrounds; r0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + u;
      if (r < nrounds) combine_store<NR, NW>(ring[u], out, off_of(r));
#pragma unroll
      for (int i = 0; i < NR; ++i) ring[u][i] = bld16(in[i], off_of(r + U));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The persistent grid of probe_tiles over `geo`: one workgroup of THREADS per resident slot,
// after a clear of the claim counters on the same stream.
template <int NR, int NW, class Geo, int THREADS = 1024>
int launch_tiles(const char* s, char* d, int64_t tensor_bytes, int64_t ntiles, const Geo& geo,
                 void* scratch, hipStream_t stream) {
  uint64_t* status = static_cast<uint64_t*>(scratch);
  int64_t zero = 0;
  hipLaunchKernelGGL(clear_status, dim3(1), dim3(256), 0, stream, status, zero);
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(&probe_tiles<NR, NW, Geo, THREADS>), THREADS,
          0) != hipSuccess ||
      cus <= 0 || per_cu <= 0)
    return FPSCAN_PROBE_ERR_DEVICE;
  const int64_t grid = (int64_t)cus * per_cu < ntiles ? (int64_t)cus * per_cu : ntiles;
  hipLaunchKernelGGL((probe_tiles<NR, NW, Geo, THREADS>), dim3((unsigned)grid), dim3(THREADS), 0,
                     stream, s, d, tensor_bytes, status, ntiles, geo);
  return hipGetLastError() == hipSuccess ? FPSCAN_PROBE_OK : FPSCAN_PROBE_ERR_LAUNCH;
}

template <int NR, int NW>
int launch_probe(int pattern, const void* src, void* dst, int64_t tensor_bytes, int64_t row_bytes,
                 void* scratch, hipStream_t stream) {
  const char* s = static_cast<const char*>(src);
  char* d = static_cast<char*>(dst);
  if (pattern == FPSCAN_PROBE_BLOCKS) {
    const int64_t blocks = tensor_bytes / (2 << 10);
    hipLaunchKernelGGL((probe_blocks<NR, NW>), dim3((unsigned)blocks), dim3(64), 0, stream, s, d,
                       tensor_bytes);
  } else if (pattern == FPSCAN_PROBE_BLOCKS_LOOKBACK) {
    static std::atomic<uint32_t> epoch{0};
    uint32_t e = epoch.fetch_add(1, std::memory_order_relaxed) + 1;
    if (e == 0) e = epoch.fetch_add(1, std::memory_order_relaxed) + 1;  // never 0: cleared
    const int64_t tiles = tensor_bytes / kLookbackTileBytes;
    const int row_tiles = (int)(row_bytes / kLookbackTileBytes);
    hipLaunchKernelGGL((probe_blocks_lookback<NR, NW>), dim3((unsigned)tiles), dim3(256), 0,
                       stream, s, d, tensor_bytes, row_tiles, static_cast<uint32_t*>(scratch), e);
  } else if (pattern == FPSCAN_PROBE_ROWS) {
    hipLaunchKernelGGL((probe_rows<NR, NW, 16, 4>), dim3((unsigned)(tensor_bytes / row_bytes)),
                       dim3(1024), 0, stream, s, d, tensor_bytes, row_bytes);
  } else if (pattern == FPSCAN_PROBE_ROWS8) {
    hipLaunchKernelGGL((probe_rows<NR, NW, 8, 2>), dim3((unsigned)(tensor_bytes / row_bytes)),
                       dim3(512), 0, stream, s, d, tensor_bytes, row_bytes);
  } else if (pattern == FPSCAN_PROBE_TILES8) {
    const int64_t ntiles = tensor_bytes / (kTileBytes / 2);
    return launch_tiles<NR, NW, RowTileGeo<kTileBytes / 2>, 512>(
        s, d, tensor_bytes, ntiles, RowTileGeo<kTileBytes / 2>{ntiles}, scratch, stream);
  } else {
    const int64_t ntiles = tensor_bytes / kTileBytes;
    return launch_tiles<NR, NW>(s, d, tensor_bytes, ntiles, RowTileGeo<kTileBytes>{ntiles},
                                scratch, stream);
  }
  return hipGetLastError() == hipSuccess ? FPSCAN_PROBE_OK : FPSCAN_PROBE_ERR_LAUNCH;
}

}  // namespace

extern "C" {

size_t fpscan_probe_scratch_bytes(void) { return kStatusExtraWords * sizeof(uint64_t); }

size_t fpscan_probe_lookback_scratch_bytes(int64_t tensor_bytes) {
  return tensor_bytes > 0 ? (size_t)(2 + tensor_bytes / kLookbackTileBytes) * sizeof(uint32_t) : 0;
}

int fpscan_probe_copy(int pattern, int nread, int nwrite, const void* src, void* dst,
                      int64_t tensor_bytes, int64_t row_bytes, void* scratch,
                      size_t scratch_bytes, void* stream) {
  if (pattern != FPSCAN_PROBE_TILES && pattern != FPSCAN_PROBE_BLOCKS &&
      pattern != FPSCAN_PROBE_ROWS && pattern != FPSCAN_PROBE_BLOCKS_LOOKBACK &&
      pattern != FPSCAN_PROBE_ROWS8 && pattern != FPSCAN_PROBE_TILES8)
    return FPSCAN_PROBE_ERR_ARG;
  if (!((nread == 2 && nwrite == 1) || (nread == 3 && nwrite == 2))) return FPSCAN_PROBE_ERR_ARG;
  if (src == nullptr || dst == nullptr) return FPSCAN_PROBE_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0 || (reinterpret_cast<uintptr_t>(dst) & 15u) != 0)
    return FPSCAN_PROBE_ERR_ARG;
  // whole tiles; at most 4 GiB per tensor keeps every grid below 2^32 work-items
  if (tensor_bytes <= 0 || tensor_bytes % kTileBytes != 0 || tensor_bytes > (int64_t)1 << 32)
    return FPSCAN_PROBE_ERR_ARG;
  if ((pattern == FPSCAN_PROBE_ROWS || pattern == FPSCAN_PROBE_ROWS8) &&
      (row_bytes <= 0 || row_bytes % kTileBytes != 0 || tensor_bytes % row_bytes != 0 ||
       row_bytes > INT32_MAX))
    return FPSCAN_PROBE_ERR_ARG;
  if (pattern == FPSCAN_PROBE_BLOCKS_LOOKBACK &&
      (row_bytes <= 0 || row_bytes % kLookbackTileBytes != 0 || tensor_bytes % row_bytes != 0 ||
       row_bytes > INT32_MAX || scratch == nullptr ||
       (reinterpret_cast<uintptr_t>(scratch) & 3u) != 0 ||
       scratch_bytes < fpscan_probe_lookback_scratch_bytes(tensor_bytes)))
    return FPSCAN_PROBE_ERR_ARG;
  if ((pattern == FPSCAN_PROBE_TILES || pattern == FPSCAN_PROBE_TILES8) &&
      (scratch == nullptr || scratch_bytes < fpscan_probe_scratch_bytes() ||
       (reinterpret_cast<uintptr_t>(scratch) & 7u) != 0))
    return FPSCAN_PROBE_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return nread == 2 ? launch_probe<2, 1>(pattern, src, dst, tensor_bytes, row_bytes, scratch, s)
                    : launch_probe<3, 2>(pattern, src, dst, tensor_bytes, row_bytes, scratch, s);
}

int fpscan_probe_copy_cl(int nread, int nwrite, const void* src, void* dst, int64_t batch,
                         int64_t seqlen, int64_t row_bytes, int strip_bytes, void* scratch,
                         size_t scratch_bytes, void* stream) {
  if (!((nread == 2 && nwrite == 1) || (nread == 3 && nwrite == 2))) return FPSCAN_PROBE_ERR_ARG;
  if (src == nullptr || dst == nullptr || scratch == nullptr ||
      scratch_bytes < fpscan_probe_scratch_bytes())
    return FPSCAN_PROBE_ERR_ARG;
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(dst) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(scratch) & 7u) != 0)
    return FPSCAN_PROBE_ERR_ARG;
  if (strip_bytes != 128 && strip_bytes != 256) return FPSCAN_PROBE_ERR_ARG;
  const int tile_rows = kTileBytes / strip_bytes;
  if (batch <= 0 || seqlen <= 0 || seqlen % tile_rows != 0 || row_bytes <= 0 ||
      row_bytes % strip_bytes != 0)
    return FPSCAN_PROBE_ERR_ARG;
  // at most 4 GiB per tensor (tested factor by factor, so the product cannot overflow) and a
  // tile's range below 2 GiB (32-bit buffer offsets)
  constexpr int64_t kMaxTensor = (int64_t)1 << 32;
  if (row_bytes > kMaxTensor / seqlen || batch > kMaxTensor / (seqlen * row_bytes) ||
      (int64_t)tile_rows * row_bytes > INT32_MAX)
    return FPSCAN_PROBE_ERR_ARG;
  const int64_t tensor_bytes = batch * seqlen * row_bytes;
  const int64_t strips = row_bytes / strip_bytes;
  const int64_t nseg = seqlen / tile_rows;
  const int64_t ntiles = batch * strips * nseg;
  const ClTileGeo geo{seqlen, row_bytes, strips, strip_bytes, tile_rows,
                      ChainTileGroups{batch * strips, nseg}};
  const char* s = static_cast<const char*>(src);
  char* d = static_cast<char*>(dst);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return nread == 2 ? launch_tiles<2, 1>(s, d, tensor_bytes, ntiles, geo, scratch, st)
                    : launch_tiles<3, 2>(s, d, tensor_bytes, ntiles, geo, scratch, st);
}

}  // extern "C"

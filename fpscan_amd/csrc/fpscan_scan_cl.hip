// Channel-last scan for MI355X (gfx950): tensors laid out (batch, seqlen, dim) with dim
// contiguous, the recurrence running along seqlen,
//
//   y[b, t, d] = gates[b, t, d] * y[b, t-1, d] + tokens[b, t, d]   (reverse: t+1),
//
// and its fused backward. No reference counterpart: the reference scans (batch, dim, seqlen)
// rows only and tells users of this layout to transpose in and out around the call
// (README.md:94-99, which costs three extra copies); this path removes the copies. The C ABI
// is in include/fpscan_hip.h (fpscan_scan_fwd_cl, fpscan_scan_bwd_cl).
//
// Work decomposition
//   A "strip" is 64 lanes x one 16-byte vector per lane: 256 fp32 or 512 fp16/bf16
//   consecutive columns of one time step, one contiguous 1 KiB span per wave instruction.
//   Each lane carries the V independent recurrences of its vector down the time axis, so
//   there is no cross-lane scan at all: per step, y = fma(a, y, b) on V values. One wave owns
//   one strip of one batch over a segment of time steps, with a ring of U steps in flight.
//   When batch x strips alone cannot fill the device, the time axis is tiled instead: with
//   enough 64-column chains, one pass over tiles of 64 columns with a look-back along time
//   (scan_cl_tiles below, 3 N s bytes forward); otherwise segments in three launches (per-
//   segment per-column aggregates (A, B) into the workspace, a carry pass over the segments of
//   each column, then the segments again with their carry-in: 5 N s bytes forward).
// All arithmetic is fp32; half types are widened exactly on load and rounded to nearest even
// once on store.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "fpscan_hip.h"
#include "scan_common.h"


namespace fpscan_detail {
int tiling_mode();  // fpscan_set_tiling's setting (fpscan_scan.hip)
int64_t hook_skip_publish();  // fpscan_set_lookback_test_hook's settings (fpscan_scan.hip)
int hook_spin_limit();
}  // namespace fpscan_detail

namespace {

// Segment phases: one pass with zero initial state, aggregates only, or one pass from the
// carry-in left in the workspace by the carry pass.
constexpr int kSingle = 0;
constexpr int kAggregate = 1;
constexpr int kApply = 2;

// fwd/rev: in0 = gates, in1 = tokens, out0 = out.
// bwd:     in0 = gates, in1 = grad_out, in2 = saved forward output, out0 = grad_tokens,
//          out1 = grad_gates.
struct ClArgs {
  const void* in0;
  const void* in1;
  const void* in2;
  void* out0;
  void* out1;
  f32x2* ws;         // [segment][batch][dim] aggregates, then carry-in in .x
  int64_t batch;
  int64_t dim;
  int64_t stride_b;  // elements
  int64_t stride_t;  // elements
  int32_t seqlen;
  int32_t seg_len;   // time steps per segment
  int32_t nseg;
  int32_t strips;    // per batch: ceil(dim / (64 V))
  int64_t chains;    // tiled path: batch * strips64
  int64_t strips64;  // tiled path, per batch: ceil(dim / 64)
  // tiled path: a tile whose aggregates are never published (-1: none; a test hook that
  // forces waits to give up) and the polls before a wait gives up
  int64_t skip_publish;
  int32_t spin_limit;
};

// Look-back waits of the tiled channel-last kernel that gave up on this device since the
// library was loaded. Read by fpscan_lookback_overruns.
static __device__ unsigned long long g_cl_overruns;

// Loaded operands of one time step for one lane.
template <int kMode>
struct ClSlot {
  u32x4 v[kMode == kBwd ? 3 : 2];
};

template <int kMode>
struct ClRsrc {
  Rsrc in0, in1, in2, out0, out1;
};

// Resource for the rows [r0, r1) of one batch of one tensor.
__device__ __forceinline__ Rsrc cl_rsrc(const void* p, const ClArgs& a, int64_t b, int64_t r0,
                                        int64_t r1, int size) {
  const int64_t elem = b * a.stride_b + r0 * a.stride_t;
  const int bytes = (int)((r1 - r0) * a.stride_t * size);
  return __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(p)) + elem * size, (short)0, bytes, kRsrcWord3);
}

template <class E, int kMode, int kPhase, int U>
__global__ void __launch_bounds__(64) scan_cl(const ClArgs a) {
  constexpr int V = E::V;
  constexpr bool kReverse = kMode != kFwd;

  const int lane = threadIdx.x & 63;
  const int64_t task = blockIdx.x;  // one wave per block
  const int64_t ntasks = (int64_t)a.nseg * a.batch * a.strips;
  if (task >= ntasks) return;  // wave-uniform; no barrier below
  const int strip = (int)(task % a.strips);
  const int64_t b = (task / a.strips) % a.batch;
  const int seg = (int)(task / ((int64_t)a.strips * a.batch));

  const int L = a.seqlen;
  const int t0 = seg * a.seg_len;
  const int t1 = min(t0 + a.seg_len, L);
  const int n = t1 - t0;
  // rows this wave may touch: its segment plus one row on each side (the backward's shifted
  // operands); the resource base is row r0
  const int r0 = t0 > 0 ? t0 - 1 : 0;
  const int r1 = t1 < L ? t1 + 1 : L;
  const uint32_t row_bytes = (uint32_t)(a.stride_t * E::kSize);

  const int col = (strip * 64 + lane) * V;  // first column of this lane
  const bool active = col < a.dim;
  const uint32_t col_off = (uint32_t)col * E::kSize;

  ClRsrc<kMode> rr;
  rr.in0 = cl_rsrc(a.in0, a, b, r0, r1, E::kSize);
  rr.in1 = cl_rsrc(a.in1, a, b, r0, r1, E::kSize);
  if constexpr (kMode == kBwd) rr.in2 = cl_rsrc(a.in2, a, b, r0, r1, E::kSize);
  if constexpr (kPhase != kAggregate) {
    rr.out0 = cl_rsrc(a.out0, a, b, r0, r1, E::kSize);
    if constexpr (kMode == kBwd) rr.out1 = cl_rsrc(a.out1, a, b, r0, r1, E::kSize);
  }

  // time step of processing step k, and the byte offset of time t's row for this lane
  auto step_t = [&](int k) { return kReverse ? t1 - 1 - k : t0 + k; };
  auto row_off = [&](int t) { return (uint32_t)(t - r0) * row_bytes + col_off; };

  // Issues the loads of processing step k (kNoOffset past the segment end or for an inactive
  // lane, so that every lane issues the same instructions). Backward: gates at t+1 (past the
  // end reads 0 and is replaced by 1 where used), grad_out at t, saved output at t-1 (before
  // the start reads 0, which is y[-1]).
  auto load_step = [&](ClSlot<kMode>& s, int k) {
    const bool live = active && k < n;
    const int t = step_t(k);
    if constexpr (kMode == kBwd) {
      s.v[0] = bld16(rr.in0, live && t + 1 < L ? row_off(t + 1) : kNoOffset);
      s.v[1] = bld16(rr.in1, live ? row_off(t) : kNoOffset);
      s.v[2] = bld16(rr.in2, live && t >= 1 ? row_off(t - 1) : kNoOffset);
    } else {
      s.v[0] = bld16(rr.in0, live ? row_off(t) : kNoOffset);
      s.v[1] = bld16(rr.in1, live ? row_off(t) : kNoOffset);
    }
  };

  // state: the running value per column (single/apply) or the segment aggregate (aggregate)
  float y[V], A[V], B[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    y[e] = 0.0f;
    A[e] = 1.0f;
    B[e] = 0.0f;
  }
  const int64_t ws_base = ((int64_t)seg * a.batch + b) * a.dim + col;
  if constexpr (kPhase == kApply) {
    if (active) {
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = a.ws[ws_base + e].x;
    }
  }
  // the first element in processing order never uses its gate (full_scan.cu:96); the
  // backward's first element has the shifted gate gates[L] = 1 anyway
  const int first_t = kReverse ? L - 1 : 0;

  ClSlot<kMode> ring[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    load_step(ring[u], u);
    __builtin_amdgcn_sched_barrier(0);
  }
  const int nrounds = (n + U - 1) / U;
  for (int r = 0; r < nrounds; ++r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = r * U + u;
      const bool valid = k < n;  // wave-uniform
      const int t = step_t(k);
      float av[V], bv[V], yp[V];
      if constexpr (kMode == kBwd) {
        float g[V];
        E::unpack(ring[u].v[0], g);
        E::unpack(ring[u].v[1], bv);
        E::unpack(ring[u].v[2], yp);
        const bool past_end = t + 1 >= L;
#pragma unroll
        for (int e = 0; e < V; ++e) av[e] = past_end ? 1.0f : g[e];
      } else {
        E::unpack(ring[u].v[0], av);
        E::unpack(ring[u].v[1], bv);
        if (t == first_t) {
#pragma unroll
          for (int e = 0; e < V; ++e) av[e] = 1.0f;
        }
      }
      if constexpr (kPhase == kAggregate) {
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float ae = valid ? av[e] : 1.0f;
          const float be = valid ? bv[e] : 0.0f;
          B[e] = fmaf(ae, B[e], be);
          A[e] = ae * A[e];
        }
      } else {
        float o0[V], o1[V];
#pragma unroll
        for (int e = 0; e < V; ++e) {
          y[e] = fmaf(av[e], y[e], bv[e]);
          o0[e] = y[e];
          if constexpr (kMode == kBwd) o1[e] = y[e] * yp[e];
        }
        const uint32_t so = valid && active ? row_off(t) : kNoOffset;
        bst16(rr.out0, so, E::pack(o0));
        if constexpr (kMode == kBwd) bst16(rr.out1, so, E::pack(o1));
      }
      load_step(ring[u], k + U);
      // keep the ring order: the next slot's arithmetic must not move above this refill
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (kPhase == kAggregate) {
    if (active) {
#pragma unroll
      for (int e = 0; e < V; ++e) a.ws[ws_base + e] = f32x2{A[e], B[e]};
    }
  }
}

// Carry pass: for each column, the carry entering each segment in processing order, written
// over the segment's A. carry_in(first) = 0, carry_in(next) = A * carry_in + B.
__global__ void __launch_bounds__(256) cl_carry(f32x2* __restrict__ ws, int64_t columns,
                                                int nseg, int reverse) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= columns) return;
  float carry = 0.0f;
  for (int k = 0; k < nseg; ++k) {
    const int j = reverse ? nseg - 1 - k : k;
    f32x2 m = ws[(int64_t)j * columns + i];
    const float next = fmaf(m.x, carry, m.y);
    m.x = carry;
    ws[(int64_t)j * columns + i] = m;
    carry = next;
  }
}

// ---------------------------------------------------------------------------------------
// Tiled channel-last scan: one pass (3 N s bytes forward) with a decoupled look-back along
// the time axis, for problems with too few strips to fill the device one wave per strip.
//
// A chain is one batch's 64 consecutive columns over the whole time axis; a tile is
// 16 R consecutive time steps of one chain (R = V: 128 steps for 2-byte types, 64 for fp32),
// one workgroup of 16 waves. A lane of wave w holds the 16-byte vector c (V columns) of time
// step w R + r of the tile; every wave instruction reads R rows x 128 or 256 contiguous
// bytes, each row as 4 pieces of 16 R bytes read by consecutive lanes (the lane order is at
// the kernel). Per tile:
//   1. each lane turns its step into V affine maps (A, B) = (gate, token);
//   2. a DPP scan over the R steps of the wave (lanes 16 / R apart in a DPP row) gives each
//      lane the inclusive map of steps 0..r of its wave, and the last step the wave's total;
//   3. wave totals go through LDS; wave w scans the 16 wave totals of columns 4w..4w+3 with
//      one 16-lane DPP row each, which yields the prefix entering every wave and the tile's
//      aggregate map per column, published at once (one 64-bit word per column);
//   4. the carry into the tile, per column, from its predecessors (below); each lane then
//      has y = M(carry) for its V columns, with M its composed map, and stores;
//   5. wave 0 publishes the tile's last value per column (a 32-bit word), y_end = A c + B.
// The look-back below (its words, their composition, the polls and the claims) runs in wave
// 0 only, under a wave-uniform branch; the other waves skip it. Only the end-value store is
// issued by every wave, out of range outside wave 0, so that the compiler's count of
// outstanding memory operations is the same on both sides of the branch.
// Look-back: the predecessors of tile k are the earlier tiles of its chain, k-1, k-2, ...
// The carry into k is always composed the same way, so results do not depend on timing:
//     carry(k) = agg(k-1) o ... o agg(k-K) applied to y_end(k-K-1)
// (fewer maps and the zero state near the chain start; K = 3, 5 or 15, fixed by the shape,
// the type and the direction).
// Tiles are claimed in order (Claims over chain groups: within a group all chains' tile 0,
// then all chains' tile 1, ...), so a tile's predecessors were claimed before it. An
// aggregate is published by a reduce, which never waits; y_end(k-K-1) by a finish, which
// waits only for earlier tiles. So the workgroup holding the lowest unfinished tile of a
// group always progresses (the row kernel's argument, by induction over tile order). As in
// the row kernel, the words a finish needs are loaded one step ahead (here right after the
// tile's reduce, kClDefer = 1) and only missing ones are polled (bounded, device-coherent).
// The grid is every workgroup that fits on the device, so with few chains many tiles of one
// chain are in flight (16 or more per chain below 16 chains per 256 workgroups), and with
// K = 5 a finish would wait about once per step for a y_end(k-K-1) finished in the same step.
// Below kClWideMaxChains the look-back is therefore wide: K = 15, one word per wave, so that
// y_end(k-16) comes from the previous generation of the chain's tiles (see the kernel).
//
// Workspace: ntiles * 64 aggregate words (8 bytes; tile-major, one per column), ntiles * 64
// end values (4 bytes), then the overrun word and claim counters as in the row kernel.
// All-ones marks an unpublished word (NaNs are canonicalised, so data never has that form).
// ---------------------------------------------------------------------------------------
constexpr int kClTileWaves = 16;
constexpr int kClTileCols = 64;  // columns per chain and tile
constexpr int kClDefer = 1;      // steps between a tile's reduce and its finish
// Aggregates composed onto a predecessor's end value (the look-back depth K, a template
// parameter of the kernel): 5 where many tiles of a chain are in flight and a finish would
// otherwise wait for end(k-4) within the same step, 3 for forward and reverse scans with many
// chains (about 2 tiles of a chain in flight), where the two extra words cost more than the
// waits they save. Measured on MI355X, forward with 3 against 5 (us, one box): bf16 64
// chains 323 / 320, 96 chains 448 / 465, 128 chains 591 / 614; fp32 192 chains 1644 / 1592,
// 256 chains 271 / 277. The backward measured 0-2 % faster with 5 at every chain count up to
// 256. 7 spills registers in the half-type backward.
constexpr int kClAggsShallow = 3;
constexpr int kClAggsDeep = 5;
// Below this many chains the look-back is wide (kClAggsWide = 15 aggregates, one word per
// wave; see scan_cl_tiles): with 16 or more workgroups per chain, end(k-6) is finished in the
// same step as tile k, so a depth of 5 waits for it about once per step.
constexpr int kClAggsWide = kClTileWaves - 1;
constexpr int64_t kClWideMaxChains = 48;
constexpr int64_t kClShallowMinChainsHalf = 96;   // forward / reverse, 2-byte types
constexpr int64_t kClShallowMinChainsF32 = 256;  // forward / reverse, fp32
static_assert(kClTileWaves * 4 == kClTileCols, "wave w scans the totals of columns 4w..4w+3");

constexpr uint32_t kEndNotPublished = ~0u;

__device__ __forceinline__ uint32_t end_load(Rsrc r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kCacheCoherent);
}

__device__ __forceinline__ void end_store(Rsrc r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kCacheCoherent);
}

// Whether one of the first n predecessor aggregates is still unpublished.
template <int K>
__device__ __forceinline__ bool agg_missing(const uint64_t (&words)[K], int n) {
  bool missing = false;
#pragma unroll
  for (int j = 0; j < K; ++j) missing = missing || (j < n && words[j] == kNotPublished);
  return missing;
}

// Claim groups of chains: group g holds chains [g chains / 8, (g + 1) chains / 8), each of
// nseg tiles, claimed segment-major.
struct ChainGroups {
  int64_t chains;
  int64_t nseg;
  __device__ int64_t chain_lo(int g) const {
    return (int64_t)(((uint64_t)g * (uint64_t)chains) / kClaimGroups);
  }
  __device__ int64_t first(int g) const { return chain_lo(g) * nseg; }
};

// Time steps per tile: 16 waves of R = V steps (one 16-byte vector of V columns per lane).
template <class E>
constexpr int cl_tile_steps() {
  return kClTileWaves * E::V;
}

template <int kMode>
struct ClTile {
  u32x4 v[kMode == kBwd ? 3 : 2];  // this lane's operands (bwd: gates t+1, grad_out t, out t-1)
  int64_t base;    // element offset of the first row of the tile's buffer range, all tensors
  int32_t bytes;   // buffer range: the tile's rows plus one on each side
  uint32_t off;    // byte offset of this lane's vector in the range; kNoOffset: none
  bool first;      // this lane holds the chain's first step (processing order)
  int64_t tile;    // ntiles: no tile
  int seg;         // position of the tile along its chain (processing order)
  int nch;         // chains of the tile's claim group: the distance to its predecessor
};

__device__ __forceinline__ Rsrc cl_tile_rsrc(const void* p, int64_t base, int size, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(p)) + base * size, (short)0, bytes, kRsrcWord3);
}

// Locates tile `tile` of claim group `g` and issues its operand loads (lanes without an
// element load nothing).
template <class E, int kMode>
__device__ __forceinline__ void cl_tile_setup(const ClArgs& a, ClTile<kMode>& ts, int64_t tile,
                                              int g, int64_t ntiles, const ChainGroups& cg,
                                              int w, int c, int r) {
  constexpr int V = E::V;
  constexpr int T = cl_tile_steps<E>();
  constexpr bool kReverse = kMode != kFwd;
  const int L = a.seqlen;
  ts.tile = tile;
  const bool live = tile < ntiles;
  const int64_t c_lo = cg.chain_lo(g);
  const int nch = live ? (int)(cg.chain_lo(g + 1) - c_lo) : 1;
  const uint32_t k = live ? (uint32_t)(tile - c_lo * cg.nseg) : 0u;
  // integer division runs on the vector unit: move the (uniform) results back to scalars
  const int seg = __builtin_amdgcn_readfirstlane((int)(k / (uint32_t)nch));
  const int64_t chain = c_lo + (int64_t)(k - (uint32_t)seg * (uint32_t)nch);
  const int64_t b = __builtin_amdgcn_readfirstlane((uint32_t)chain / (uint32_t)a.strips64);
  const int strip = (int)(chain - b * a.strips64);
  ts.seg = seg;
  ts.nch = nch;
  // processing positions [p0, p1) of the tile; time rows [lo, hi)
  const int p0 = seg * T;
  const int p1 = min(p0 + T, L);
  const int lo = kReverse ? L - p1 : p0;
  const int hi = kReverse ? L - p0 : p1;
  const int r0 = lo > 0 ? lo - 1 : 0;
  const int r1 = hi < L ? hi + 1 : L;
  const uint32_t row_bytes = (uint32_t)(a.stride_t * E::kSize);
  ts.base = live ? b * a.stride_b + (int64_t)r0 * a.stride_t : 0;
  ts.bytes = live ? (int32_t)((uint32_t)(r1 - r0) * row_bytes) : 0;
  const int p = p0 + w * V + r;
  const int col = strip * kClTileCols + c * V;
  const bool mine = live && p < p1 && col < a.dim;
  const int t = kReverse ? L - 1 - p : p;
  ts.first = p == 0;
  ts.off = mine ? (uint32_t)(t - r0) * row_bytes + (uint32_t)col * E::kSize : kNoOffset;
  const Rsrc in0 = cl_tile_rsrc(a.in0, ts.base, E::kSize, ts.bytes);
  const Rsrc in1 = cl_tile_rsrc(a.in1, ts.base, E::kSize, ts.bytes);
  if constexpr (kMode == kBwd) {
    const Rsrc in2 = cl_tile_rsrc(a.in2, ts.base, E::kSize, ts.bytes);
    ts.v[0] = bld16(in0, mine && t + 1 < L ? ts.off + row_bytes : kNoOffset);
    ts.v[1] = bld16(in1, ts.off);
    ts.v[2] = bld16(in2, mine && t >= 1 ? ts.off - row_bytes : kNoOffset);
  } else {
    ts.v[0] = bld16(in0, ts.off);
    ts.v[1] = bld16(in1, ts.off);
  }
}

template <class E, int kMode, int D, int K, bool kStepLanes>
__global__ void __launch_bounds__(64 * kClTileWaves)
scan_cl_tiles(const ClArgs a, uint64_t* __restrict__ status, const int64_t ntiles) {
  constexpr int V = E::V;
  constexpr int R = V;  // time steps per wave
  constexpr int N = D + 2;
  constexpr int kPad = 2;             // LDS row padding (f32x2), keeps 16-byte alignment
  static_assert(N % D == 0, "the unrolled ring must map each step to a fixed deferral slot");
  static_assert(R * (kClTileCols / V) == 64, "a wave is R steps of 64 columns");
  // Wide look-back (K = 15, one predecessor word per wave): every wave loads one word per
  // column, and the carry is composed by a 16-lane DPP scan per column in the cross-wave
  // step. Otherwise wave 0 loads all K words and composes them serially.
  constexpr bool kWide = K == kClTileWaves - 1;
  static_assert(kWide || K <= 8, "narrow look-back depths are held in wave 0's registers");

  __shared__ f32x2 exch[kClTileWaves][kClTileCols + kPad];  // wave totals
  __shared__ f32x2 pref[kClTileWaves][kClTileCols + kPad];  // prefix entering each wave
  __shared__ f32x2 aggs[N][kClTileCols];                    // tile aggregates, by ring slot
  __shared__ float carry_in[kClTileCols];
  __shared__ uint64_t lbw[kWide ? kClTileWaves : 1][kClTileCols];  // wide: wave w's word
  __shared__ int64_t claimed;
  __shared__ int claimed_grp;
  __shared__ int64_t first_tiles[2];
  __shared__ int first_grps[2];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Lane (r, c) holds the 16-byte vector c (columns V c .. V c + V - 1) of step r of the
  // wave. By default P = 16 / R consecutive lanes hold consecutive vectors of one step, so
  // that each group of P lanes reads P * 16 contiguous bytes, and the R steps of a column
  // group sit P lanes apart inside one 16-lane DPP row, so that the scan over them is
  // full-row DPP steps. With kStepLanes, consecutive lanes hold consecutive steps (lane =
  // r + R c) and the scan runs over aligned R-lane segments: then every lane of a quad reads
  // another 128-byte line, which measured 2.5-3.5 % slower forward at 64 chains and more,
  // but 5 % faster for the 2-byte backward at 128 chains (and 5-10 % slower at 32 or fewer).
  constexpr int P = kStepLanes ? 1 : 16 / R;
  static_assert(kStepLanes || (P * R == 16 && P * 4 * V == kClTileCols),
                "a DPP row is P vectors of R steps");
  const int r = kStepLanes ? lane % R : (lane / P) % R;
  const int c = kStepLanes ? lane / R : lane % P + P * (lane / 16);
  const bool leader = threadIdx.x == 0;
  const int L = a.seqlen;
  // aggregate words, then end values (32-bit) from word nagg on, then the extra words
  const int64_t nagg = ntiles * kClTileCols;
  const int64_t nstatus = nagg + nagg / 2;
  const uint32_t ends_off = (uint32_t)(nagg * sizeof(uint64_t));
  const Rsrc st = __builtin_amdgcn_make_buffer_rsrc(
      status, (short)0, (int)((nstatus + kStatusExtraWords) * sizeof(uint64_t)), kRsrcWord3);
  const ChainGroups cg{a.chains, a.nseg};

  const int64_t kBubble = ntiles, kDone = ntiles + 1;
  Claims<ChainGroups> claims{(uint32_t)((nstatus + kCounterStride) * sizeof(uint64_t)),
                             reinterpret_cast<const uint32_t*>(status + nstatus + kCounterStride),
                             cg, (int)(blockIdx.x % kClaimGroups)};
  Claim pending[N];
#pragma unroll
  for (int i = 0; i < N; ++i) pending[i] = Claim{0, 0};
  bool claims_done = false;
  if (leader) {
    // a tile that next_now returns comes from the current group
    const int64_t t0 = claims.next_now(st, kBubble, kDone);
    first_grps[0] = claims.grp;
    const int64_t t1 = (t0 == kDone) ? kDone : claims.next_now(st, kBubble, kDone);
    first_grps[1] = claims.grp;
    first_tiles[0] = t0;
    first_tiles[1] = t1;
    claims_done = t1 == kDone;
  }
  __syncthreads();
  // The two steps before the loop issue what a steady-state step issues, in the same order
  // (the stores, here out of range; wave 0's predecessor words and claim; the refill), so
  // that the compiler's wait counts at the loop head are the steady-state ones. Otherwise the
  // path into the loop makes it wait there for loads just issued.
  uint64_t held_agg[kWide ? 1 : K] = {};  // wide: this wave's word (wave K: an end value)
  uint32_t held_end = 0;
  ClTile<kMode> ring[N];
#pragma unroll
  for (int i = 2; i < N; ++i) {  // filled at the end of the first steps
    ring[i].tile = ntiles;
    ring[i].seg = 0;
    ring[i].nch = 1;
    ring[i].base = 0;
    ring[i].bytes = 0;
    ring[i].off = kNoOffset;
    ring[i].first = false;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    status_store(st, kNoOffset, 0ull);
    end_store(st, kNoOffset, 0u);
    bst16(st, kNoOffset, u32x4{0u, 0u, 0u, 0u});
    if constexpr (kMode == kBwd) bst16(st, kNoOffset, u32x4{0u, 0u, 0u, 0u});
    if constexpr (kWide) {
      held_agg[0] = status_load(st, kNoOffset);
      held_end = end_load(st, kNoOffset);
      if (w == 0) pending[N - 2 + i] = claims.issue(st, leader && !claims_done);
    } else if (w == 0) {
#pragma unroll
      for (int j = 0; j < K; ++j) held_agg[j] = status_load(st, kNoOffset);
      held_end = end_load(st, kNoOffset);
      pending[N - 2 + i] = claims.issue(st, leader && !claims_done);
    }
    cl_tile_setup<E, kMode>(a, ring[i],
                            min(__builtin_amdgcn_readfirstlane(first_tiles[i]), ntiles),
                            __builtin_amdgcn_readfirstlane(first_grps[i]), ntiles, cg, w, c, r);
    __builtin_amdgcn_sched_barrier(0);
  }

  // per deferral slot: the map from the tile's carry to this lane's value, per column (the
  // prefix entering its wave, then its wave's steps up to its own)
  float held_A[D][V], held_B[D][V];
#pragma unroll
  for (int i = 0; i < D; ++i) {
#pragma unroll
    for (int e = 0; e < V; ++e) {
      held_A[i][e] = 1.0f;
      held_B[i][e] = 0.0f;
    }
  }
  bool all_claimed = false;

  for (;;) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      ClTile<kMode>& cur = ring[u];
      ClTile<kMode>& fin = ring[(u + 2) % N];
      const int hs = u % D;
      const bool cur_live = cur.tile < ntiles;
      const bool fin_live = fin.tile < ntiles;

      // (1) the current tile: this lane's maps (gate, token) per column, then an inclusive
      // scan over the R steps of the wave; the last step ends with the wave's total
      float pa[V], pb[V];
      {
        E::unpack(cur.v[0], pa);
        E::unpack(cur.v[1], pb);
        // the chain's first step keeps gate 1: forward and reverse never use its gate, and the
        // backward's shifted gate is gates[L] = 1. Lanes without an element loaded zeros, the
        // map (0, 0): such lanes are columns past dim or steps past the chain's end, and
        // columns never mix, so it reaches no stored value.
        if (cur.first) {
#pragma unroll
          for (int e = 0; e < V; ++e) pa[e] = 1.0f;
        }
        if constexpr (kStepLanes) {
          segment_scan_k<R>(pa, pb, r);
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e) {
            if constexpr (P <= 2) combine_from_row<2>(pa[e], pb[e]);
            if constexpr (P <= 4) combine_from_row<4>(pa[e], pb[e]);
            combine_from_row<8>(pa[e], pb[e]);
          }
        }
        if (r == R - 1) {
#pragma unroll
          for (int e = 0; e < V; ++e) exch[w][c * V + e] = f32x2{pa[e], pb[e]};
        }
        if constexpr (kWide) lbw[w][lane] = w == K ? (uint64_t)held_end : held_agg[0];
      }

      lds_barrier();

      // (2) the current tile's wave prefixes and aggregate (wave w: columns 4w..4w+3). The
      // aggregate is published before wave 0 waits for the finishing tile's predecessors, so
      // that no wait delays a publication: with many tiles of a chain in flight, a successor's
      // finish needs this word within the same step.
      {
        const int i = lane & 15;
        const int col = 4 * w + (lane >> 4);
        const f32x2 e = exch[i][col];
        float eA = e.x, eB = e.y;
        combine_from_row<1>(eA, eB);
        combine_from_row<2>(eA, eB);
        combine_from_row<4>(eA, eB);
        combine_from_row<8>(eA, eB);
        if (i < 15) pref[i + 1][col] = f32x2{eA, eB};
        if (i == 15) aggs[u][col] = f32x2{eA, eB};
        const bool publish = cur_live && i == 15 && cur.tile != a.skip_publish;
        status_store(st,
                     publish ? (uint32_t)((cur.tile * kClTileCols + col) * sizeof(uint64_t))
                             : kNoOffset,
                     pack_map(eA, eB));
      }

      uint32_t end_off = kNoOffset, end_word = 0;
      if constexpr (kWide) {
        // (2b) the finishing tile's carry per column (wave w: columns 4w..4w+3): lane i of a
        // 16-lane row takes the map of predecessor k-16+i (lane 0 the constant map of end
        // value k-16, or of the zero state near the chain start; lanes 1..15 the aggregates
        // of tiles k-15..k-1, or the identity before the chain start), and an inclusive DPP
        // scan leaves lane 15 with agg(k-1) o ... o agg(k-15) o end(k-16), whose B is the
        // carry. Missing words are polled by the lanes that need them (bounded, as below).
        const int i = lane & 15;
        const int col = 4 * w + (lane >> 4);
        const int wi = K - i;  // 0..14: tile k-1-wi's aggregate; K: end value of k-16
        const int na = min(fin.seg, K);
        const bool need = wi < K ? wi < na : fin.seg > K;
        uint64_t word = lbw[wi][col];
        auto missing = [&](uint64_t v) {
          return need && (wi < K ? v == kNotPublished : (uint32_t)v == kEndNotPublished);
        };
        if (__builtin_amdgcn_ballot_w64(missing(word)) != 0) {
          const bool overran = __hip_atomic_load(status + nstatus, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) != 0;
          for (int it = overran ? a.spin_limit : 0;; ++it) {
            __builtin_amdgcn_s_sleep(1);
            if (missing(word)) {
              if (wi < K)
                word = __hip_atomic_load(
                    status + (fin.tile - (int64_t)(wi + 1) * fin.nch) * kClTileCols + col,
                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              else
                word = __hip_atomic_load(reinterpret_cast<const uint32_t*>(status + nagg) +
                                             (fin.tile - (int64_t)(K + 1) * fin.nch) * kClTileCols +
                                             col,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (__builtin_amdgcn_ballot_w64(missing(word)) == 0) break;
            if (it >= a.spin_limit) {
              if (lane == 0) {
                __hip_atomic_fetch_add(status + nstatus, 1ull, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(&g_cl_overruns, 1ull, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
              }
              break;
            }
          }
          // only after an overrun: a word still missing becomes NaN, as in the narrow path
          if (missing(word)) word = wi < K ? kPoisonMap : (uint64_t)kPoisonValue;
        }
        float mA = 1.0f, mB = 0.0f;
        if (wi < K) {
          if (need) {
            mA = __uint_as_float((uint32_t)word);
            mB = __uint_as_float((uint32_t)(word >> 32));
          }
        } else {
          mA = 0.0f;
          mB = need ? __uint_as_float((uint32_t)word) : 0.0f;
        }
        combine_from_row<1>(mA, mB);
        combine_from_row<2>(mA, mB);
        combine_from_row<4>(mA, mB);
        combine_from_row<8>(mA, mB);
        // hand the carries on; the end values are read by tile k+K+1
        if (i == 15) carry_in[col] = mB;
        const f32x2 agg = aggs[(u + 2) % N][col];
        if (i == 15 && fin_live && fin.seg + K + 1 < a.nseg)
          end_off = ends_off + (uint32_t)((fin.tile * kClTileCols + col) * sizeof(uint32_t));
        end_word = canonical_bits(fmaf(agg.x, mB, agg.y));
      }

      // (3) wave 0 (narrow look-back): the finishing tile's carry per column from its
      // predecessors' words, and the tile's end values. The store is issued by every wave,
      // out of range outside wave 0: a store inside a branch would leave the compiler unsure
      // how many memory operations follow each load.
      if constexpr (!kWide) if (w == 0) {
        const int na = min(fin.seg, K);  // aggregates composed (uniform)
        if (__builtin_amdgcn_ballot_w64(agg_missing(held_agg, na) ||
                                        (fin.seg > K && held_end == kEndNotPublished)) != 0) {
          // a predecessor has not published yet: poll the missing words (bounded; once any
          // wait of this launch has overrun, which a correct launch never does, the others
          // give up at once, so that the launch still ends soon)
          const bool overran = __hip_atomic_load(status + nstatus, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) != 0;
          for (int it = overran ? a.spin_limit : 0;; ++it) {
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int j = 0; j < K; ++j) {
              if (j < na && held_agg[j] == kNotPublished)
                held_agg[j] = __hip_atomic_load(
                    status + (fin.tile - (int64_t)(j + 1) * fin.nch) * kClTileCols + lane,
                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (fin.seg > K && held_end == kEndNotPublished)
              held_end = __hip_atomic_load(
                  reinterpret_cast<const uint32_t*>(status + nagg) +
                      (fin.tile - (int64_t)(K + 1) * fin.nch) * kClTileCols + lane,
                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__builtin_amdgcn_ballot_w64(agg_missing(held_agg, na) ||
                                            (fin.seg > K && held_end == kEndNotPublished)) == 0)
              break;
            if (it >= a.spin_limit) {
              if (lane == 0) {
                __hip_atomic_fetch_add(status + nstatus, 1ull, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(&g_cl_overruns, 1ull, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
              }
              break;
            }
          }
          // only after an overrun: the words still missing become NaN, so that this tile's
          // outputs, its end values and every carry composed from them are NaN, not plausible
#pragma unroll
          for (int j = 0; j < K; ++j)
            held_agg[j] = held_agg[j] == kNotPublished ? kPoisonMap : held_agg[j];
          held_end = held_end == kEndNotPublished ? kPoisonValue : held_end;
        }
        // carry = agg(k-1) o ... o agg(k-na) applied to y_end(k-na-1), or to the zero state
        float carry = fin.seg > K ? __uint_as_float(held_end) : 0.0f;
#pragma unroll
        for (int j = K - 1; j >= 0; --j) {
          if (j < na) {
            const uint64_t word = held_agg[j];
            carry = fmaf(__uint_as_float((uint32_t)word), carry,
                         __uint_as_float((uint32_t)(word >> 32)));
          }
        }
        // hand the carries on; the end values are read by tile k+K+1
        carry_in[lane] = carry;
        const f32x2 agg = aggs[(u + 2) % N][lane];
        if (fin_live && fin.seg + K + 1 < a.nseg)
          end_off = ends_off + (uint32_t)((fin.tile * kClTileCols + lane) * sizeof(uint32_t));
        end_word = canonical_bits(fmaf(agg.x, carry, agg.y));
      }
      end_store(st, end_off, end_word);
      if (leader) {
        const int64_t t = claims_done ? kDone : claims.resolve(pending[(u + D) % N], kBubble, kDone);
        claims_done = t == kDone;
        claimed = t;
        claimed_grp = pending[(u + D) % N].grp;  // the group of a tile that resolve returns
      }
      lds_barrier();
      const int64_t claim = __builtin_amdgcn_readfirstlane(claimed);
      const int claim_grp = __builtin_amdgcn_readfirstlane(claimed_grp);
      all_claimed = claim == kDone;

      // (4) finish the oldest deferred tile
      {
        float y[V];
#pragma unroll
        for (int e = 0; e < V; ++e) y[e] = fmaf(held_A[hs][e], carry_in[c * V + e], held_B[hs][e]);
        const Rsrc out0 = cl_tile_rsrc(a.out0, fin.base, E::kSize, fin.bytes);
        bst16(out0, fin.off, E::pack(y));
        if constexpr (kMode == kBwd) {
          float ys[V], o1[V];
          E::unpack(fin.v[2], ys);
#pragma unroll
          for (int e = 0; e < V; ++e) o1[e] = y[e] * ys[e];
          const Rsrc out1 = cl_tile_rsrc(a.out1, fin.base, E::kSize, fin.bytes);
          bst16(out1, fin.off, E::pack(o1));
        }
      }

      // (5) the current tile's composed maps, held until its finish
      {
        float PA[V], PB[V];
#pragma unroll
        for (int e = 0; e < V; ++e) {
          PA[e] = 1.0f;
          PB[e] = 0.0f;
        }
        if (w > 0) {
#pragma unroll
          for (int e = 0; e < V; ++e) {
            const f32x2 q = pref[w][c * V + e];
            PA[e] = q.x;
            PB[e] = q.y;
          }
        }
#pragma unroll
        for (int e = 0; e < V; ++e) {
          held_B[hs][e] = fmaf(pa[e], PB[e], pb[e]);
          held_A[hs][e] = pa[e] * PA[e];
        }
      }

      // (6) wave 0: the predecessor words of the tile finished next step (the current one),
      // loaded before the refill below (vector loads return in issue order), and the claim
      // (the leader's lane)
      if constexpr (kWide) {
        // every wave: its one word (waves 0..K-1 an aggregate, wave K the end value)
        const ClTile<kMode>& nxt = ring[(u + 3) % N];
        const bool mine = nxt.tile < ntiles;
        const int64_t p = nxt.tile - (int64_t)(w + 1) * nxt.nch;
        held_agg[0] = status_load(
            st, mine && w < K && w < nxt.seg ? (uint32_t)((p * kClTileCols + lane) * sizeof(uint64_t))
                                             : kNoOffset);
        const int64_t q = nxt.tile - (int64_t)(K + 1) * nxt.nch;
        held_end = end_load(st, mine && w == K && nxt.seg > K
                                    ? ends_off + (uint32_t)((q * kClTileCols + lane) * sizeof(uint32_t))
                                    : kNoOffset);
        if (w == 0) pending[u] = claims.issue(st, leader && !claims_done);
      } else if (w == 0) {
        const ClTile<kMode>& nxt = ring[(u + 3) % N];
        const bool mine = nxt.tile < ntiles;
#pragma unroll
        for (int j = 0; j < K; ++j) {
          const int64_t p = nxt.tile - (int64_t)(j + 1) * nxt.nch;
          held_agg[j] = status_load(
              st, mine && j < nxt.seg ? (uint32_t)((p * kClTileCols + lane) * sizeof(uint64_t))
                                      : kNoOffset);
        }
        const int64_t q = nxt.tile - (int64_t)(K + 1) * nxt.nch;
        held_end = end_load(st, mine && nxt.seg > K
                                    ? ends_off + (uint32_t)((q * kClTileCols + lane) * sizeof(uint32_t))
                                    : kNoOffset);
        pending[u] = claims.issue(st, leader && !claims_done);
      }
      // (7) refill the finished slot with the tile claimed two steps ago
      cl_tile_setup<E, kMode>(a, fin, claim < ntiles ? claim : ntiles, claim_grp, ntiles, cg, w,
                              c, r);
      __builtin_amdgcn_sched_barrier(0);
    }
    bool busy = !all_claimed;
#pragma unroll
    for (int i = 0; i < N; ++i) busy = busy || ring[i].tile < ntiles;
    if (!busy) break;
  }
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------
// One wave (one strip task) per block: blocks of four waves put each four tasks on one CU, so
// that 512 tasks (the fewest that take the one pass) used only 128 of the 256 CUs. Measured on
// MI355X against four waves per block (p50 of one call, same buffers, outputs bit for bit
// equal): 512 tasks, fp32 (32, 512, 4096) forward / backward 161.0 / 272.5 -> 135.7 / 234.7 us,
// bf16 (64, 256, 4096) 78.0 / 135.8 -> 65.1 / 112.0; from 1024 tasks within +-2 %.
constexpr int kClWaves = 1;
// Below this many wave tasks in one pass the time axis is cut into segments: one wave per
// strip and batch would leave most of the 256 CUs idle. Measured on MI355X: with 512 tasks
// (fp32 16 x 4096 x 8192) one pass streams at 4.2 TB/s against 3.2 segmented, with 1024
// (config 5, 64 x 256 x 4096) at 5.6 against 3.2; with 16 tasks (8 x 65536 x 1024 bf16) one
// pass manages 0.24 TB/s and the segments 2.7.
constexpr int64_t kClMinTasks = 512;
constexpr int kClMinSegLen = 64;        // time steps per segment, at least
constexpr int kClTargetSegLen = 1024;   // time steps per segment, aimed at
constexpr int64_t kClTargetTasks = 1024;  // wave tasks, at least (as far as kClMinSegLen allows)

struct ClPlan {
  int nseg;
  int seg_len;
  size_t bytes;   // workspace: one (A, B) pair per segment per column
  bool required;  // one pass would not fit a segment's rows in one buffer range
};

int cl_vec(int size) { return 16 / size; }

// Segments of the time axis. A wave's buffer resource spans its segment's rows plus one on
// each side, which must stay below 2^31 bytes; otherwise one wave per strip and batch, cut
// into segments when that leaves too few waves: about kClTargetSegLen steps each, more if
// needed for kClTargetTasks waves, never below kClMinSegLen. Measured on MI355X at
// (8, 65536, 1024): 1024-step segments (1024 waves in bf16, 2048 in fp32) beat 128-step ones
// (8192 waves) by 30 % in bf16, and 4096-step ones by 15 %.
ClPlan plan_cl(int64_t batch, int64_t seqlen, int64_t dim, int64_t stride_t, int size) {
  ClPlan p{1, (int)seqlen, 0, false};
  const int64_t strips = (dim + 64 * cl_vec(size) - 1) / (64 * cl_vec(size));
  const int64_t tasks = batch * strips;
  if (tasks <= 0 || seqlen <= 0) return p;
  const int64_t max_len = (int64_t)INT32_MAX / (stride_t * size) - 2;  // >= 1 (validated)
  int64_t nseg = 1;
  if (tasks < kClMinTasks && seqlen >= 2 * kClMinSegLen) {
    nseg = (seqlen + kClTargetSegLen - 1) / kClTargetSegLen;
    const int64_t for_tasks = (kClTargetTasks + tasks - 1) / tasks;
    if (nseg < for_tasks) nseg = for_tasks;
    const int64_t most = seqlen / kClMinSegLen;
    if (nseg > most) nseg = most;
  }
  const int64_t fit = (seqlen + max_len - 1) / max_len;
  if (fit > 1) p.required = true;
  if (nseg < fit) nseg = fit;
  if (nseg < 2) return p;
  const int64_t seg_len = (seqlen + nseg - 1) / nseg;
  nseg = (seqlen + seg_len - 1) / seg_len;
  p.nseg = (int)nseg;
  p.seg_len = (int)seg_len;
  p.bytes = (size_t)nseg * (size_t)batch * (size_t)dim * sizeof(f32x2);
  return p;
}

template <class E, int kMode, int kPhase>
int launch_cl(const ClArgs& a, hipStream_t stream) {
  constexpr int U = kMode == kBwd ? 6 : 8;
  const int64_t ntasks = (int64_t)a.nseg * a.batch * a.strips;
  const int64_t blocks = (ntasks + kClWaves - 1) / kClWaves;
  if (blocks > INT32_MAX) return FPSCAN_ERR_SHAPE;
  ClArgs copy = a;
  void* params[] = {&copy};
  const hipError_t err =
      hipLaunchKernel(reinterpret_cast<const void*>(&scan_cl<E, kMode, kPhase, U>),
                      dim3((unsigned)blocks), dim3(64 * kClWaves), params, 0, stream);
  return err == hipSuccess ? FPSCAN_OK : FPSCAN_ERR_LAUNCH;
}

// Tiled path. It replaces the segments wherever one pass per strip lacks waves, whatever the
// number of chains, and the one pass from kClTiledMinBytes per tensor, with a persistent grid
// of every workgroup that fits on the device (at most one per tile). Measured on MI355X, bf16
// forward / backward, against the segments: (4, 65536, 1024) 64 chains 341 / 478 us against
// 484 / 689; (1, 65536, 1024) 16 chains 128 / 166 against 248 / 299; (1, 65536, 64) one chain
// 112 / 111 against 292 / 304. A cap of 2 workgroups per chain cost 40-150 % below 128
// chains.

struct ClTilePlan {
  bool use;
  int64_t chains;
  int64_t strips64;
  int64_t nseg;
  int64_t ntiles;
  size_t bytes;  // workspace: 64 aggregates and 64 end values per tile, the overrun word and
                 // claim counters
};

// 8-byte words of per-tile status: a 64-bit aggregate and a 32-bit end value per column.
int64_t cl_status_words(int64_t ntiles) { return ntiles * kClTileCols * 3 / 2; }

// From this size per tensor the tiled pass also replaces the one pass per strip. Measured on
// MI355X, one pass against tiled, fwd / bwd us: fp32 (16, 4096, 8192), 512 strips, 1466 / 2258
// against 1119 / 1970; fp32 (512, 256, 4096), 8192 strips, 1223 / 2069 against 1066 / 1799;
// bf16 (256, 1024, 8192) 2689 / 4490 against 2370 / 3580. Smaller problems with few tiles per
// chain keep the one pass: fp32 (64, 256, 4096) 143 / 249 against 150 / 246, bf16 (64, 256,
// 4096) 79 / 135 against 102 / 185.
constexpr int64_t kClTiledMinBytes = 512ll << 20;

ClTilePlan plan_cl_tiles(int64_t batch, int64_t seqlen, int64_t dim, int64_t stride_t, int size,
                         int tiling) {
  ClTilePlan t{false, 0, 0, 0, 0, 0};
  if (tiling == 1 || batch <= 0 || seqlen <= 0 || dim <= 0) return t;
  const int64_t steps = size == 4 ? cl_tile_steps<F32>() : cl_tile_steps<BF16>();
  t.strips64 = (dim + kClTileCols - 1) / kClTileCols;
  t.chains = batch * t.strips64;
  t.nseg = (seqlen + steps - 1) / steps;
  t.ntiles = t.chains * t.nseg;
  const int64_t words = cl_status_words(t.ntiles) + kStatusExtraWords;
  if (words * (int64_t)sizeof(uint64_t) > INT32_MAX) return t;
  if ((steps + 2) * stride_t * size > INT32_MAX) return t;
  if (tiling == 0) {
    const int64_t strips = (dim + 64 * cl_vec(size) - 1) / (64 * cl_vec(size));
    const bool large = batch * seqlen * dim * size >= kClTiledMinBytes;
    if ((batch * strips >= kClMinTasks && !large) || t.nseg < 2) return t;
  }
  t.use = true;
  t.bytes = (size_t)words * sizeof(uint64_t);
  return t;
}

// The 2-byte backward takes kStepLanes from this many chains (see scan_cl_tiles).
constexpr int64_t kClStepLanesMinChains = 96;

constexpr int kClMaxDevices = 64;
std::atomic<int> g_cl_resident[kClMaxDevices][36];  // 3 types x 3 modes x 4 kernel variants

// Workgroups of `kernel` resident at once on the current device (CUs x blocks per CU), cached
// per device and kernel; 0 if the device cannot be queried.
int cl_resident_blocks(const void* kernel, int slot, int threads) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kClMaxDevices) {
    const int cached = g_cl_resident[dev][slot].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
      cus <= 0 || per_cu <= 0)
    return 0;
  const int n = cus * per_cu;
  if (dev < kClMaxDevices) g_cl_resident[dev][slot].store(n, std::memory_order_relaxed);
  return n;
}

// Clears the status words and counters, then the persistent grid. -1 when the occupancy query
// fails (the caller then takes another path).
template <class E, int kMode>
int run_cl_tiled(ClArgs a, const ClTilePlan& plan, void* workspace, hipStream_t stream) {
  // variants: 0 shallow look-back, 1 deep, 2 deep with kStepLanes (2-byte backward only),
  // 3 wide (few chains)
  const void* kernel = nullptr;
  int variant = 1;
  if (plan.chains < kClWideMaxChains) {
    variant = 3;
    kernel = reinterpret_cast<const void*>(&scan_cl_tiles<E, kMode, kClDefer, kClAggsWide, false>);
  } else if constexpr (kMode != kBwd) {
    const bool shallow =
        plan.chains >= (E::kSize == 4 ? kClShallowMinChainsF32 : kClShallowMinChainsHalf);
    variant = shallow ? 0 : 1;
    kernel = shallow
                 ? reinterpret_cast<const void*>(&scan_cl_tiles<E, kMode, kClDefer, kClAggsShallow, false>)
                 : reinterpret_cast<const void*>(&scan_cl_tiles<E, kMode, kClDefer, kClAggsDeep, false>);
  } else if constexpr (E::kSize == 2) {
    const bool step_lanes = plan.chains >= kClStepLanesMinChains;
    variant = step_lanes ? 2 : 1;
    kernel = step_lanes
                 ? reinterpret_cast<const void*>(&scan_cl_tiles<E, kMode, kClDefer, kClAggsDeep, true>)
                 : reinterpret_cast<const void*>(&scan_cl_tiles<E, kMode, kClDefer, kClAggsDeep, false>);
  } else {
    kernel = reinterpret_cast<const void*>(&scan_cl_tiles<E, kMode, kClDefer, kClAggsDeep, false>);
  }
  const int threads = 64 * kClTileWaves;
  const int resident = cl_resident_blocks(kernel, (E::kSlot * 3 + kMode) * 4 + variant, threads);
  if (resident <= 0) return -1;
  uint64_t* status = static_cast<uint64_t*>(workspace);
  int64_t ntiles = plan.ntiles;
  int64_t nstatus = cl_status_words(ntiles);
  const int64_t nwords = nstatus + kStatusExtraWords;
  const int64_t clear_blocks = (nwords + 255) / 256 < 2048 ? (nwords + 255) / 256 : 2048;
  void* cargs[] = {&status, &nstatus};
  if (hipLaunchKernel(reinterpret_cast<const void*>(&clear_status), dim3((unsigned)clear_blocks),
                      dim3(256), cargs, 0, stream) != hipSuccess)
    return FPSCAN_ERR_LAUNCH;
  int64_t grid = resident;
  if (grid > ntiles) grid = ntiles;
  a.chains = plan.chains;
  a.strips64 = plan.strips64;
  a.nseg = (int32_t)plan.nseg;
  a.seg_len = cl_tile_steps<E>();
  a.ws = nullptr;
  a.skip_publish = fpscan_detail::hook_skip_publish();
  a.spin_limit = fpscan_detail::hook_spin_limit();
  void* kargs[] = {&a, &status, &ntiles};
  const hipError_t err =
      hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), kargs, 0, stream);
  return err == hipSuccess ? FPSCAN_OK : FPSCAN_ERR_LAUNCH;
}

template <class E, int kMode>
int run_cl(ClArgs a, void* workspace, size_t ws_bytes, hipStream_t stream) {
  const ClTilePlan tiles = plan_cl_tiles(a.batch, a.seqlen, a.dim, a.stride_t, E::kSize,
                                         fpscan_detail::tiling_mode());
  if (tiles.use && workspace != nullptr && ws_bytes >= tiles.bytes) {
    const int st = run_cl_tiled<E, kMode>(a, tiles, workspace, stream);
    if (st >= 0) return st;
  }
  const ClPlan plan = plan_cl(a.batch, a.seqlen, a.dim, a.stride_t, E::kSize);
  if (plan.nseg > 1 && workspace != nullptr && ws_bytes >= plan.bytes) {
    a.nseg = plan.nseg;
    a.seg_len = plan.seg_len;
    a.ws = static_cast<f32x2*>(workspace);
    int st = launch_cl<E, kMode, kAggregate>(a, stream);
    if (st != FPSCAN_OK) return st;
    const int64_t columns = a.batch * a.dim;
    int nseg = a.nseg;
    int reverse = kMode != kFwd ? 1 : 0;
    f32x2* ws = a.ws;
    int64_t cols = columns;
    void* cargs[] = {&ws, &cols, &nseg, &reverse};
    if (hipLaunchKernel(reinterpret_cast<const void*>(&cl_carry), dim3((unsigned)((columns + 255) / 256)),
                        dim3(256), cargs, 0, stream) != hipSuccess)
      return FPSCAN_ERR_LAUNCH;
    return launch_cl<E, kMode, kApply>(a, stream);
  }
  if (plan.required) return FPSCAN_ERR_WORKSPACE;
  a.nseg = 1;
  a.seg_len = a.seqlen;
  a.ws = nullptr;
  return launch_cl<E, kMode, kSingle>(a, stream);
}

template <int kMode>
int dispatch_cl(int dtype, const ClArgs& a, void* ws, size_t ws_bytes, hipStream_t stream) {
  switch (dtype) {
    case FPSCAN_DTYPE_F32: return run_cl<F32, kMode>(a, ws, ws_bytes, stream);
    case FPSCAN_DTYPE_F16: return run_cl<F16, kMode>(a, ws, ws_bytes, stream);
    case FPSCAN_DTYPE_BF16: return run_cl<BF16, kMode>(a, ws, ws_bytes, stream);
    default: return FPSCAN_ERR_DTYPE;
  }
}

int cl_itemsize(int dtype) {
  switch (dtype) {
    case FPSCAN_DTYPE_F32: return 4;
    case FPSCAN_DTYPE_F16: return 2;
    case FPSCAN_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool cl_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shapes, strides and alignment of a channel-last call. A buffer resource covers one
// segment's rows (plus one on each side), so three rows must fit in 2^31 bytes.
int validate_cl(int64_t batch, int64_t seqlen, int64_t dim, int64_t stride_b, int64_t stride_t,
                int dtype, const void* const* ptrs, int nptrs, ClArgs& a) {
  const int size = cl_itemsize(dtype);
  if (size == 0) return FPSCAN_ERR_DTYPE;
  if (batch < 0 || seqlen < 0 || dim < 0 || seqlen > INT32_MAX) return FPSCAN_ERR_SHAPE;
  if (batch == 0 || seqlen == 0 || dim == 0) return -1;  // nothing to do
  // stride_t is bounded first, so that (seqlen - 1) * stride_t cannot wrap around; the
  // element span (batch-1)*stride_b + (seqlen-1)*stride_t + dim is computed with checks
  if (stride_t < dim || stride_t > (INT32_MAX / 3) / size) return FPSCAN_ERR_SHAPE;
  const int64_t over_t = (seqlen - 1) * stride_t;
  int64_t over_b = 0, span = 0;
  if (stride_b < over_t + dim || __builtin_mul_overflow(batch - 1, stride_b, &over_b) ||
      __builtin_add_overflow(over_b, over_t + dim, &span) || span > ((int64_t)1 << 48) / size)
    return FPSCAN_ERR_SHAPE;
  const int64_t vec = 16 / size;
  if (dim % vec != 0 || stride_t % vec != 0 || stride_b % vec != 0) return FPSCAN_ERR_ALIGN;
  for (int i = 0; i < nptrs; ++i) {
    if (ptrs[i] == nullptr) return FPSCAN_ERR_NULL;
    if (!cl_aligned16(ptrs[i])) return FPSCAN_ERR_ALIGN;
  }
  a.batch = batch;
  a.dim = dim;
  a.stride_b = stride_b;
  a.stride_t = stride_t;
  a.seqlen = (int32_t)seqlen;
  a.seg_len = (int32_t)seqlen;
  a.nseg = 1;
  a.strips = (int32_t)((dim + 64 * vec - 1) / (64 * vec));
  a.ws = nullptr;
  return FPSCAN_OK;
}

}  // namespace

namespace fpscan_detail {
// The channel-last counter of given-up waits on the current device (a synchronous copy).
int cl_overruns(unsigned long long* count) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_cl_overruns)) != hipSuccess || p == nullptr)
    return FPSCAN_ERR_DEVICE;
  if (hipMemcpy(count, p, sizeof(*count), hipMemcpyDeviceToHost) != hipSuccess)
    return FPSCAN_ERR_DEVICE;
  return FPSCAN_OK;
}
}  // namespace fpscan_detail

extern "C" {

int fpscan_scan_fwd_cl(const void* gates, const void* tokens, void* out, int64_t batch,
                       int64_t seqlen, int64_t dim, int64_t stride_b, int64_t stride_t,
                       int dtype, int reverse, void* workspace, size_t workspace_bytes,
                       void* stream) {
  ClArgs a{};
  const void* ptrs[] = {gates, tokens, out};
  const int st = validate_cl(batch, seqlen, dim, stride_b, stride_t, dtype, ptrs, 3, a);
  if (st < 0) return FPSCAN_OK;
  if (st != FPSCAN_OK) return st;
  a.in0 = gates;
  a.in1 = tokens;
  a.in2 = nullptr;
  a.out0 = out;
  a.out1 = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return reverse ? dispatch_cl<kRev>(dtype, a, workspace, workspace_bytes, s)
                 : dispatch_cl<kFwd>(dtype, a, workspace, workspace_bytes, s);
}

int fpscan_scan_bwd_cl(const void* gates, const void* out, const void* grad_out,
                       void* grad_gates, void* grad_tokens, int64_t batch, int64_t seqlen,
                       int64_t dim, int64_t stride_b, int64_t stride_t, int dtype,
                       void* workspace, size_t workspace_bytes, void* stream) {
  ClArgs a{};
  const void* ptrs[] = {gates, out, grad_out, grad_gates, grad_tokens};
  const int st = validate_cl(batch, seqlen, dim, stride_b, stride_t, dtype, ptrs, 5, a);
  if (st < 0) return FPSCAN_OK;
  if (st != FPSCAN_OK) return st;
  a.in0 = gates;
  a.in1 = grad_out;
  a.in2 = out;
  a.out0 = grad_tokens;
  a.out1 = grad_gates;
  return dispatch_cl<kBwd>(dtype, a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

size_t fpscan_workspace_bytes_cl(int64_t batch, int64_t seqlen, int64_t dim, int64_t stride_t,
                                 int dtype, int op) {
  const int size = cl_itemsize(dtype);
  if (size == 0 || batch <= 0 || seqlen <= 0 || dim <= 0 || seqlen > INT32_MAX) return 0;
  if (stride_t < dim || stride_t * size > (INT32_MAX / 3)) return 0;
  if (op != FPSCAN_OP_FWD && op != FPSCAN_OP_BWD) return 0;
  int64_t steps = 0, elems = 0;
  if (__builtin_mul_overflow(batch, seqlen, &steps) ||
      __builtin_mul_overflow(steps, stride_t, &elems) || elems > ((int64_t)1 << 48) / size)
    return 0;  // no call of this size passes validation
  const ClTilePlan tiles =
      plan_cl_tiles(batch, seqlen, dim, stride_t, size, fpscan_detail::tiling_mode());
  if (tiles.use) return tiles.bytes;
  return plan_cl(batch, seqlen, dim, stride_t, size).bytes;
}

}  // extern "C"

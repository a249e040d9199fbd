// Contraction scan ("dimwise") for MI355X (gfx950): the second function of the reference's
// extension module, dimwise_forward(Ax, Bx, Bh, Wq, Wk) (csrc/main.cpp:10,
// csrc/dimwise/dimwise.h:27-42), computed in place into Bx.
//
// Semantics (csrc/dimwise/dimwise_scan_final.cu:12-382, launcher :387-576), per row (b, d) of
// (batch, dim, seqlen) tensors, in chunks of W groups of P elements (table in dw_geom):
//   local[g][j]  zero-initial-state scan y = a*y + x inside group g; in chunks after the first,
//                group 0 starts from the previous chunk's carry (y = a*carry + x at its first
//                element); the row's very first gate is ignored
//   v[g]         local[g][P-1]
//   k[g]         (1 + Wk[d]) * Bh[b, d, g]   (g < W; the chunk index is not used, :133, :189)
//   q[g]         (1 + Wq[d]) * v[g]
//   r[0] = v[0]; for 1 <= g <= W-2: m = first h < g with the strictly largest k[h]*q[g] over
//                an initial -1e10, r[g] = (k[m]*q[g]) * v[m] + v[g]
//   out[g][j]    local[g][j] + (g > 0 ? r[g-1] : 0); carry = out[W-1][P-1]
// The reference computes everything in the tensors' own type. Here the scans, v, r and the
// outputs are fp32 with one rounding at the store (more accurate), while the selection
// reproduces the reference's arithmetic on k, q and the scores in the tensors' type
// (fp16/bf16 rounding after each operation, fp32 fused multiply-adds as nvcc contracts them),
// so that the same m is chosen whenever the group sums round to the same value. Where the
// reference leaves m undefined (no score above the initial value, :83, :200), m = 0 here.
//
// Work decomposition: one workgroup per row; its waves are the sub-chunks (64 lanes x one
// 16-byte vector per lane) of one chunk; a group is GL consecutive lanes, scanned with a
// segmented DPP scan. v and r go through LDS; wave 0 selects (lane g for group g, W <= 32)
// and keeps the chunk carry in a register, so a chunk costs two barriers. The next chunk's
// operands are in flight while a chunk is computed.
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

struct DwArgs {
  const void* ax;
  void* bx;
  const void* bh;
  const void* wq;
  const void* wk;
  int64_t rows;
  int64_t dim;
  int32_t seqlen;
  int32_t W;  // groups per chunk
  int32_t C;  // chunks per row
};

// The tensors' own rounding, applied where the reference's selection arithmetic rounds.
template <class E>
__device__ __forceinline__ float round_t(float x) {
  if constexpr (E::kSlot == F16::kSlot) {
    return static_cast<float>(static_cast<_Float16>(x));
  } else if constexpr (E::kSlot == BF16::kSlot) {
    return static_cast<float>(static_cast<__bf16>(x));
  } else {
    return x;
  }
}

// w * x + x as the reference computes it in its type: one fused multiply-add in fp32,
// multiply then add (each rounded) in fp16/bf16.
template <class E>
__device__ __forceinline__ float scale1p(float w, float x) {
  if constexpr (E::kSize == 4) {
    return fmaf(w, x, x);
  } else {
    return round_t<E>(round_t<E>(w * x) + x);
  }
}

template <class E>
__device__ __forceinline__ float load1(const void* p, int64_t i) {
  if constexpr (E::kSize == 4) {
    return static_cast<const float*>(p)[i];
  } else {
    return E::widen16(static_cast<const unsigned short*>(p)[i]);
  }
}

template <class E, int GL, int NW>
__global__ void __launch_bounds__(64 * NW) dimwise_rows(const DwArgs a) {
  constexpr int V = E::V;
  constexpr int P = GL * V;   // elements per group
  constexpr int kSub = 64 * V;

  __shared__ float v_lds[32];
  __shared__ float r_lds[32];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = a.W;
  const int chunk = W * P;                               // elements per chunk
  const int per_wave = chunk < kSub ? chunk : kSub;      // elements per wave per chunk
  const int groups_per_wave = per_wave / P;
  const bool active = lane * V < per_wave;
  const int sl = lane % GL;
  const int g = w * groups_per_wave + lane / GL;         // this lane's group in the chunk
  const int L = a.seqlen;
  const int G = W * a.C;                                 // Bh row length

  // the initial score, as the reference's `tens score = -1e10` (fp16: -inf)
  const float kInit = round_t<E>(-1e10f);

  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const int64_t d = row % a.dim;
    const Rsrc ax = row_rsrc(a.ax, row * L, E::kSize, L * E::kSize);
    const Rsrc bx = row_rsrc(a.bx, row * L, E::kSize, L * E::kSize);
    const uint32_t lane_off = (uint32_t)((w * kSub + lane * V) * E::kSize);
    auto chunk_off = [&](int c) {
      return (c < a.C && active) ? (uint32_t)(c * chunk * E::kSize) + lane_off : kNoOffset;
    };

    // wave 0, lane h < W: k[h] in the tensors' arithmetic; every lane: Wq[d]
    float k = 0.0f, wq = 0.0f;
    if (w == 0) {
      wq = load1<E>(a.wq, d);
      if (lane < W) k = scale1p<E>(load1<E>(a.wk, d), load1<E>(a.bh, row * G + lane));
    }

    u32x4 ring[2][2];
    ring[0][0] = bld16(ax, chunk_off(0));
    ring[0][1] = bld16(bx, chunk_off(0));
    __builtin_amdgcn_sched_barrier(0);
    ring[1][0] = bld16(ax, chunk_off(1));
    ring[1][1] = bld16(bx, chunk_off(1));
    __builtin_amdgcn_sched_barrier(0);

    float carry = 0.0f;  // wave 0: the previous chunk's last output
    for (int c0 = 0; c0 < a.C; c0 += 2) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = c0 + u;
        if (c >= a.C) break;  // uniform; only after the last chunk
        float av[V], bv[V];
        E::unpack(ring[u][0], av);
        E::unpack(ring[u][1], bv);
        // refill this slot with the chunk two ahead now, so its loads overlap this chunk's
        // scans, selection and barriers
        ring[u][0] = bld16(ax, chunk_off(c + 2));
        ring[u][1] = bld16(bx, chunk_off(c + 2));
        if (c == 0 && w == 0 && lane == 0) av[0] = 1.0f;  // the row's first gate is ignored

        // local scans: lane aggregate, segmented scan over the group's lanes, then the
        // elements again from the value entering the lane
        float A = av[0], B = bv[0];
#pragma unroll
        for (int i = 1; i < V; ++i) {
          B = fmaf(av[i], B, bv[i]);
          A = av[i] * A;
        }
        segment_scan<GL>(A, B, sl);
        const float c_in = (w == 0 && g == 0) ? carry : 0.0f;
        float y = dpp<kWaveShr1>(c_in, fmaf(A, c_in, B));
        y = (sl == 0) ? c_in : y;
        float ys[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          y = fmaf(av[i], y, bv[i]);
          ys[i] = y;
        }
        if (active && sl == GL - 1) v_lds[g] = y;
        lds_barrier();

        if (w == 0) {
          // lane g selects for group g
          const float vg = lane < W ? v_lds[lane] : 0.0f;
          const float q = scale1p<E>(wq, round_t<E>(vg));
          float best = kInit;
          int m = 0;
          for (int h = 0; h < W - 1; ++h) {
            const float s = round_t<E>(readlane(k, h) * q);
            if (h < lane && s > best) {
              best = s;
              m = h;
            }
          }
          const float r = lane == 0 ? vg : fmaf(best, v_lds[m], vg);
          if (lane < W) r_lds[lane] = r;
          carry = readlane(vg, W - 1) + readlane(r, W - 2);
        }
        lds_barrier();

        float o[V];
        const float add = g > 0 ? r_lds[g > 0 ? g - 1 : 0] : 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = ys[i] + add;
        bst16(bx, chunk_off(c), E::pack(o));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Long rows, tiled (seqlen 8192..65536, where every chunk is W = 32 groups of P = 128).
//
// Between chunks only the carry passes, and it enters a chunk affinely. With zero-initial
// group scans, group 0 ends at v0(c) = a0 c + b0 (a0 its gate product, b0 its zero-carry end)
// and every other group end v[g] is independent of c; so are the scores of groups g >= 1 (q
// uses v[g]) and with them the selected m. Hence r[g](c) = best v0(c) + v[g] when m = 0 and a
// constant otherwise, and the chunk's outgoing carry v[W-1] + r[W-2](c) is an affine map of c.
// A persistent grid claims 16 KiB tiles (two chunks of a 2-byte type, one of fp32) in memory
// order (Claims, as the tiled row scan) and chains the tiles of a row by a decoupled
// look-back over these maps: a tile reduces its chunks, selects, publishes the composed map,
// and is finished D steps later from the carry its look-back found. A step has two barriers:
// after the reduce, the selection waves test the candidate groups (each wave a share of
// them) while one other wave runs the look-back of the tile finished in this step and makes
// the claims; after the second barrier wave 1 combines the selection and publishes the map
// while the other waves finish the deferred tile, whose terms were made D steps earlier.
// Measured on MI355X (B8 D1024 L65536 bf16, each against the kernel of its time in one
// timing): the combine and publish before that barrier, with a third one between selection
// and combine, 5 % slower; 8 KiB tiles (one chunk, two workgroups per CU) 6 % slower -- their
// copy pattern alone is 8 % slower than that of 16 KiB tiles (FPSCAN_PROBE_TILES8).
//
// Workspace: as the tiled row scan's ([0, ntiles) tile status, [ntiles] wait overruns, claim
// counters after it).
// ---------------------------------------------------------------------------------------
constexpr int kDwW = 32;          // groups per chunk on tiled rows
constexpr int kDwChunk = 4096;    // elements per chunk on tiled rows (W * P, P = 128)
constexpr int kDwTileWaves = 16;  // 16 KiB tiles
constexpr int kDwDefer = 2;       // steps between a tile's reduce and its finish
constexpr int kDwSelWave = 1;     // the wave that combines the selection and publishes

// Tile geometry by element type: chunks per 16 KiB tile (two of a 2-byte type, one of fp32),
// and the selection's split: kSelWaves waves test kSelSpan candidates h each, four per lane
// (2-byte types: lane = chunk * 32 + group; fp32: lane = half * 32 + group, each half taking
// four of the wave's eight candidates).
template <class E>
struct DwGeo {
  static constexpr int kChunks = kDwTileWaves * 64 * E::V / kDwChunk;
  static constexpr int kSelWaves = 4 * kChunks;
  static constexpr int kSelSpan = kDwW / kSelWaves;
  static_assert(kChunks == 1 || kChunks == 2, "one or two chunks per tile");
};

// Look-back waits of the tiled dimwise kernel that gave up on this device since the library
// was loaded. Read by fpscan_lookback_overruns.
static __device__ unsigned long long g_dw_overruns;

struct DwTileArgs {
  const void* ax;
  void* bx;
  const void* bh;
  const void* wq;
  const void* wk;
  int64_t dim;
  int32_t seqlen;
  int32_t G;           // Bh row length
  int64_t skip_publish;  // test hook: a tile whose map is never published (-1: none)
  int32_t spin_limit;    // polls before a look-back wait gives up
};

// One ring slot: the tile, this lane's operands and the row's selection parameters (lane
// j < kSelSpan of selection wave w: Bh[row][kSelSpan w + j]; lane 32: Wq[d]; lanes 33..63:
// Wk[d]; as loaded bits). The row and the segment are derived from the tile where they are
// used: kept per slot (with per-row buffer resources) they are 44 more scalar registers,
// which the compiler then spills to VGPR lanes and reloads with a VALU instruction each.
struct DwSlot {
  u32x4 ax, bx;
  uint32_t par;
  int64_t tile;
};

// The tiled path addresses Ax and Bx through one buffer resource per tensor (the launcher
// takes it only for tensors below 4 GiB), tile t at byte t * tile bytes: the rows are
// contiguous, so a tile's offset needs no per-row arithmetic. An offset of all ones is
// outside every such range: loads from it return 0 and stores to it are dropped.
constexpr uint32_t kDwNoOffset = 0xfffffff0u;

template <class E>
__device__ __forceinline__ float widen_par(uint32_t bits) {
  if constexpr (E::kSize == 4) {
    return __uint_as_float(bits);
  } else {
    return E::widen16((unsigned short)bits);
  }
}

template <int TW>
__device__ __forceinline__ uint32_t dw_offset(int64_t tile, int w, uint32_t lane_off) {
  return (uint32_t)tile * (uint32_t)(TW * 1024) + (uint32_t)w * 1024u + lane_off;
}

template <class E, int TW>
__device__ __forceinline__ void dw_setup(const DwTileArgs& a, Rsrc tax, Rsrc tbx, DwSlot& s,
                                         int64_t tile, int64_t ntiles, int tpr_log2, int w,
                                         int lane) {
  s.tile = tile;
  const bool live = tile < ntiles;
  const int64_t row = live ? (tile >> tpr_log2) : 0;
  const uint32_t off = live ? dw_offset<TW>(tile, w, (uint32_t)lane * 16u) : kDwNoOffset;
  s.ax = bld16(tax, off);
  s.bx = bld16(tbx, off);
  // every wave loads the parameters (a branch here would make the compiler wait for the
  // operand loads at the join); all lanes read valid addresses of row `row`
  const int64_t d = row < ((int64_t)1 << 32) ? (int64_t)((uint32_t)row % (uint32_t)a.dim)
                                              : row % a.dim;
  // lanes j < 32: k's operand of candidate h = kSelSpan w + j % kSelSpan (a selection wave
  // uses lanes j < kSelSpan; the other waves read valid entries they never use)
  constexpr int kSelWaves = DwGeo<E>::kSelWaves, kSelSpan = DwGeo<E>::kSelSpan;
  const int h = (w < kSelWaves ? kSelSpan * w : 0) + lane % kSelSpan;
  const char* p = lane < kDwW ? static_cast<const char*>(a.bh) + (row * a.G + h) * E::kSize
                  : lane == kDwW ? static_cast<const char*>(a.wq) + d * E::kSize
                                 : static_cast<const char*>(a.wk) + d * E::kSize;
  if constexpr (E::kSize == 4) {
    s.par = *reinterpret_cast<const uint32_t*>(p);
  } else {
    s.par = *reinterpret_cast<const unsigned short*>(p);
  }
}

template <class E, int TW, int D>
__global__ void __launch_bounds__(64 * TW) __attribute__((amdgpu_waves_per_eu(4)))
dimwise_tiles(const DwTileArgs a, uint64_t* __restrict__ status, const int tpr_log2,
              const int64_t ntiles) {
  constexpr int V = E::V;
  constexpr int GL = 128 / V;  // lanes per group
  constexpr int kGroupsPerWave = 64 / GL;
  constexpr int N = D + 2;
  static_assert(N == 4, "the drain below is written out for a ring of four slots");
  constexpr int kChunks = DwGeo<E>::kChunks;
  static_assert(TW * 64 * V == kChunks * kDwChunk, "whole chunks per tile");
  constexpr int kWavesPerChunk = TW / kChunks;
  constexpr int kTileGroups = kChunks * kDwW;  // (chunk, group) pairs of a tile
  constexpr int kSelWaves = DwGeo<E>::kSelWaves;
  constexpr int kSelSpan = DwGeo<E>::kSelSpan;
  static_assert(kSelWaves * kSelSpan == kDwW && kSelWaves < TW, "every candidate tested");
  // the first wave after the selection waves runs the look-back and makes the claims, at
  // the same time as the selection
  constexpr int kLookWave = kSelWaves;

  __shared__ float v_lds[2][kTileGroups];  // zero-carry group ends, by step parity
  __shared__ f32x2 part_lds[kSelWaves][kTileGroups];   // partial selections: (best, m as bits)
  __shared__ f32x2 sel_lds[N][kTileGroups];  // per ring slot: r[g](c) = via0 ? x v0(c) + y : y
  __shared__ uint64_t via0_lds[N];           // per ring slot: groups whose r goes through v0
  __shared__ f32x2 g0_lds[N][kChunks];       // per ring slot and chunk: group 0's (a0, b0)
  __shared__ f32x2 map_lds[N];               // per ring slot: chunk 0's carry map
  __shared__ float tile_carry;
  __shared__ int64_t claimed;
  __shared__ int64_t first_tiles[2];

  const int lane0 = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const Rsrc st = __builtin_amdgcn_make_buffer_rsrc(
      status, (short)0, (int)((ntiles + kStatusExtraWords) * sizeof(uint64_t)), kRsrcWord3);
  const int tensor_bytes = (int)((uint32_t)ntiles * (uint32_t)(TW * 1024));  // below 4 GiB
  const Rsrc tax = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.ax), (short)0,
                                                     tensor_bytes, kRsrcWord3);
  const Rsrc tbx = __builtin_amdgcn_make_buffer_rsrc(a.bx, (short)0, tensor_bytes, kRsrcWord3);
  // the initial score, as the reference's `tens score = -1e10` (fp16: -inf)
  const float kInit = round_t<E>(-1e10f);

  const int64_t kBubble = ntiles, kDone = ntiles + 1;
  Claims<RowGroupsLazy> claims{(uint32_t)((ntiles + kCounterStride) * sizeof(uint64_t)),
                             reinterpret_cast<const uint32_t*>(status + ntiles + kCounterStride),
                             RowGroupsLazy{ntiles >> tpr_log2, tpr_log2},
                             (int)(blockIdx.x % kClaimGroups)};
  Claim pending[N];
#pragma unroll
  for (int i = 0; i < N; ++i) pending[i] = Claim{0, 0};
  bool claims_done = false;
  if (threadIdx.x == 64 * kLookWave) {
    const int64_t t0 = claims.next_now(st, kBubble, kDone);
    const int64_t t1 = (t0 == kDone) ? kDone : claims.next_now(st, kBubble, kDone);
    first_tiles[0] = t0;
    first_tiles[1] = t1;
    claims_done = t1 == kDone;
  }
  __syncthreads();
  // the two steps before the loop issue what a steady-state step issues, in the same order,
  // so that the compiler's wait counts at the loop head are the steady-state ones
  uint64_t held_word = 0;
  DwSlot ring[N];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    held_word = status_load(st, kNoOffset);
    pending[N - 2 + i] = claims.issue(st, threadIdx.x == 64 * kLookWave && !claims_done);
    dw_setup<E, TW>(a, tax, tbx, ring[i],
                    min(__builtin_amdgcn_readfirstlane(first_tiles[i]), ntiles), ntiles, tpr_log2,
                    w, lane0);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 2; i < N; ++i) ring[i].tile = ntiles;  // filled at the end of the first steps
  const int64_t seg_mask = ((int64_t)1 << tpr_log2) - 1;

  // what a deferred tile's finish needs from its reduce: the lane's inclusive map inside its
  // group
  float held_A[D], held_B[D];
  bool have[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    held_A[i] = 1.0f;
    held_B[i] = 0.0f;
    have[i] = false;
  }
  bool all_claimed = false;

  auto step = [&](const int u) __attribute__((always_inline)) {
    // the lane's position, derived each step from an opaque copy of its index: the per-lane
    // masks (lane 0, group ends, ...) then live within one step, where recomputing one costs
    // a compare, instead of across the loop in scalar registers that the compiler spills
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const bool leader = w == kLookWave && lane == 0;
    const int ch = w / kWavesPerChunk;                               // this lane's chunk
    const int g = (w % kWavesPerChunk) * kGroupsPerWave + lane / GL;  // its group in it
    const int sl = lane % GL;
    const uint32_t lane_off = (uint32_t)lane * 16u;
    DwSlot& cur = ring[u];
    const int fs = (u + 2) % N;
    DwSlot& fin = ring[fs];  // reduced D steps ago
    const int hs = u % D;
    const bool cur_live = cur.tile < ntiles;

    // (1) reduce the current tile: zero-initial scans of the lane's elements and of its group
    float A, B;
    {
      float av[V], bv[V];
      E::unpack(cur.ax, av);
      E::unpack(cur.bx, bv);
      if ((cur.tile & seg_mask) == 0 && w == 0 && lane == 0) av[0] = 1.0f;  // first gate
      A = av[0];
      B = bv[0];
#pragma unroll
      for (int i = 1; i < V; ++i) {
        B = fmaf(av[i], B, bv[i]);
        A = av[i] * A;
      }
    }
    segment_scan<GL>(A, B, sl);
    if (sl == GL - 1) {
      v_lds[u % 2][ch * kDwW + g] = B;
      if (g == 0) g0_lds[u][ch] = f32x2{A, B};
    }
    lds_barrier();

    // (2) selection waves w < kSelWaves: the first maximum of each group's scores over the
    // candidates h = kSelSpan w .. kSelSpan (w + 1) - 1 with h < g, from the initial score.
    // Four candidates per lane: with two chunks, lane = chunk * 32 + group; with one, lanes
    // 32..63 take the second four of the group's eight and the halves are combined.
    if (w < kSelWaves) {
      const int sg = lane % kDwW;
      const int upper = lane / kDwW;  // the lane's chunk (two chunks) or half (one chunk)
      const int pair = kChunks == 2 ? lane : sg;
      const int h0 = kSelSpan * w + (kChunks == 1 ? 4 * upper : 0);
      const float wk = widen_par<E>((uint32_t)__builtin_amdgcn_readlane((int)cur.par, kDwW + 1));
      const float wq = widen_par<E>((uint32_t)__builtin_amdgcn_readlane((int)cur.par, kDwW));
      const float k = scale1p<E>(wk, widen_par<E>(cur.par));  // lanes j < kSelSpan: k[h]
      const float q = scale1p<E>(wq, round_t<E>(v_lds[u % 2][pair]));
      float best = kInit;
      int mi = 0;
      int t = sg - h0;  // candidate i passes h < g iff i < t
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float kk =
            (kChunks == 1 && upper) ? readlane(k, 4 + i) : readlane(k, i);
        const float sc = round_t<E>(kk * q);
        // tied to this candidate's score, so that the compare stays here instead of all of
        // them being hoisted ahead of the loop with their masks held in scalar registers
        asm volatile("" : "+v"(t) : "v"(sc));
        if (i < t && sc > best) {
          best = sc;
          mi = i;
        }
      }
      int m = h0 + mi;
      if constexpr (kChunks == 1) {
        // the upper half's candidates come later: they win only if strictly larger
        const int src = ((lane + kDwW) & 63) << 2;
        const float bu = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(best)));
        const int mu = __builtin_amdgcn_ds_bpermute(src, m);
        if (bu > best) {
          best = bu;
          m = mu;
        }
      }
      if (lane < kTileGroups) part_lds[w][pair] = f32x2{best, __int_as_float(m)};
    }

    // (3) the look-back wave, meanwhile: the finishing tile's carry from its predecessor
    // words (loaded right after the previous step's finish), and the claim resolved
    if (w == kLookWave) {
      uint64_t word = held_word;
      if (__builtin_amdgcn_ballot_w64(word == kNotPublished) != 0) {
        // a predecessor was not published yet: poll (bounded), with an atomic load that the
        // compiler re-issues every iteration
        const int64_t p = fin.tile - 64 + lane;
        const bool in_row = p >= fin.tile - (fin.tile & seg_mask);
        for (int it = 0;; ++it) {
          __builtin_amdgcn_s_sleep(1);
          word = in_row ? __hip_atomic_load(status + p, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT)
                        : 0ull;
          if (__builtin_amdgcn_ballot_w64(word == kNotPublished) == 0) break;
          if (it >= a.spin_limit) {
            // only after an overrun: count it where the caller can see it, and make the
            // tile's outputs NaN (a NaN map poisons the composed carry) instead of plausible
            if (lane == 0) {
              __hip_atomic_fetch_add(status + ntiles, 1ull, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_fetch_add(&g_dw_overruns, 1ull, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
            }
            word = word == kNotPublished ? kPoisonMap : word;
            break;
          }
        }
      }
      float cA = __uint_as_float((uint32_t)word);
      float cB = __uint_as_float((uint32_t)(word >> 32));
      wave_scan(cA, cB);
      if (lane == 63) tile_carry = cB;
    }
    if (leader) {
      const int64_t t = claims_done ? kDone : claims.resolve(pending[(u + D) % N], kBubble, kDone);
      claims_done = t == kDone;
      claimed = t;
    }
    lds_barrier();
    const int64_t claim = __builtin_amdgcn_readfirstlane(claimed);
    all_claimed = claim == kDone;
    const int64_t refill = claim < ntiles ? claim : ntiles;

    // (4) wave 1: a group's selection is the first of the partial maxima that exceeds the
    // ones before it (ties keep the earlier h, as one pass over h does); then the terms r[g]
    // for the tile's finish and its carry map, published at once. Off the other waves'
    // path: they go on to finish the deferred tile, whose terms were made D steps ago.
    if (w == kDwSelWave) {
      const int pair = lane % kTileGroups;
      const int sg = pair % kDwW, sc = pair / kDwW;
      f32x2 pm = part_lds[0][pair];
      float best = pm.x;
      int m = __float_as_int(pm.y);
#pragma unroll
      for (int i = 1; i < kSelWaves; ++i) {
        pm = part_lds[i][pair];
        if (pm.x > best) {
          best = pm.x;
          m = __float_as_int(pm.y);
        }
      }
      const float vg = v_lds[u % 2][pair];
      // r[0] = v0(c); r[g] = best v0(c) + v[g] when m = 0; else the constant best v[m] + v[g]
      const bool via0 = sg == 0 || m == 0;
      const float x = sg == 0 ? 1.0f : best;
      const float y = sg == 0 ? 0.0f : (m == 0 ? vg : fmaf(best, v_lds[u % 2][sc * kDwW + m], vg));
      if (lane < kTileGroups) sel_lds[u][pair] = f32x2{x, y};
      const uint64_t via0_mask = __builtin_amdgcn_ballot_w64(via0);
      if (lane == 0) via0_lds[u] = via0_mask;
      // each chunk's carry map v[W-1] + r[W-2](c) = A c + B, composed over the tile's chunks
      float tA = 1.0f, tB = 0.0f;
#pragma unroll
      for (int cc = 0; cc < kChunks; ++cc) {
        const int l = cc * kDwW + kDwW - 2;
        const float x30 = readlane(x, l), y30 = readlane(y, l), v31 = readlane(vg, l + 1);
        const f32x2 g0 = g0_lds[u][cc];
        const bool f30 = ((via0_mask >> l) & 1) != 0;
        const float mA = f30 ? x30 * g0.x : 0.0f;
        const float mB = v31 + (f30 ? fmaf(x30, g0.y, y30) : y30);
        if (cc == 0) {
          if (lane == 0) map_lds[u] = f32x2{mA, mB};
          tA = mA;
          tB = mB;
        } else {
          tB = fmaf(mA, tB, mB);
          tA = mA * tA;
        }
      }
      const bool publisher = cur_live && lane == 0 && cur.tile != a.skip_publish;
      status_store(st, publisher ? (uint32_t)(cur.tile * sizeof(uint64_t)) : kNoOffset,
                   pack_map(tA, tB));
    }

    // (5) finish the oldest deferred tile (nothing is stored while the ring fills)
    {
      const float c_tile = tile_carry;
      float c_chunk = c_tile;  // the carry into this lane's chunk
      if constexpr (kChunks == 2) {
        const f32x2 m0 = map_lds[fs];
        c_chunk = ch == 0 ? c_tile : fmaf(m0.x, c_tile, m0.y);
      }
      const f32x2 g0 = g0_lds[fs][ch];
      const float v0c = fmaf(g0.x, c_chunk, g0.y);
      const int gi = ch * kDwW + (g > 0 ? g - 1 : 0);
      const f32x2 r = sel_lds[fs][gi];
      const bool r_via0 = ((via0_lds[fs] >> gi) & 1) != 0;
      const float add = g == 0 ? 0.0f : (r_via0 ? fmaf(r.x, v0c, r.y) : r.y);
      const float c_in = g == 0 ? c_chunk : 0.0f;
      float y = dpp<kWaveShr1>(c_in, fmaf(held_A[hs], c_in, held_B[hs]));
      y = (sl == 0) ? c_in : y;
      float av[V], bv[V], o[V];
      E::unpack(fin.ax, av);
      E::unpack(fin.bx, bv);
      const int fseg = (int)(fin.tile & seg_mask);
      if (fseg == 0 && w == 0 && lane == 0) av[0] = 1.0f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        y = fmaf(av[i], y, bv[i]);
        o[i] = y + add;
      }
      bst16(tbx, have[hs] ? dw_offset<TW>(fin.tile, w, lane_off) : kDwNoOffset, E::pack(o));
    }
    held_A[hs] = A;
    held_B[hs] = B;
    have[hs] = cur_live;

    // (6) the look-back wave: load the predecessor words of the tile finished in the next
    // step, before the refill (vector loads complete in issue order); lanes before the row
    // start and all other waves read 0, the constant map 0 (the zero initial state)
    {
      const DwSlot& nxt = ring[(u + 3) % N];
      const bool nxt_live = nxt.tile < ntiles;
      const int64_t q = nxt.tile - 64 + lane;
      const int64_t nseg = nxt.tile & seg_mask;
      const bool mine = w == kLookWave && nxt_live && nseg > 0 && q >= nxt.tile - nseg;
      held_word = status_load(st, mine ? (uint32_t)(q * sizeof(uint64_t)) : kNoOffset);
    }
    pending[u] = claims.issue(st, leader && !claims_done);
    // (7) refill the finished slot with the tile claimed two steps ago
    dw_setup<E, TW>(a, tax, tbx, fin, refill, ntiles, tpr_log2, w, lane);
    __builtin_amdgcn_sched_barrier(0);
  };

  auto busy = [&]() __attribute__((always_inline)) {
    bool b = false;
#pragma unroll
    for (int i = 0; i < D; ++i) b = b || have[i];
#pragma unroll
    for (int i = 0; i < N; ++i) b = b || ring[i].tile < ntiles;
    return b;
  };
  // Steady state, then the drain, as in the tiled row scan: only the claim stream ends the
  // loop (a workgroup moving between used-up groups may hold tiles in claims still in flight),
  // and the drain runs the steps written out until nothing is left to finish.
  for (;;) {
#pragma unroll
    for (int u = 0; u < N; ++u) step(u);
    if (all_claimed) break;
  }
  for (;;) {
    if (!busy()) return;
    step(0);
    if (!busy()) return;
    step(1);
    if (!busy()) return;
    step(2);
    if (!busy()) return;
    step(3);
  }
}

// (W, P, C) by seqlen, as the reference's launcher picks kernels (:408-572); W = 0: rejected
// (seqlen 32 included, :573-575).
struct DwGeom {
  int W, P, C;
};

DwGeom dw_geom(int64_t L) {
  switch (L) {
    case 64: return {2, 32, 1};
    case 128: return {4, 32, 1};
    case 256: return {8, 32, 1};
    case 512: return {16, 32, 1};
    case 1024: return {16, 64, 1};
    case 2048: return {32, 64, 1};
    case 4096: return {32, 128, 1};
    case 8192:
    case 16384:
    case 32768:
    case 65536: return {32, 128, (int)(L / 4096)};
    default: return {0, 0, 0};
  }
}

template <class E, int GL, int NW>
int launch_dw(const DwArgs& a, hipStream_t stream) {
  const int64_t cap = 1 << 20;  // rows per launch wave; the kernel loops over the rest
  const unsigned blocks = (unsigned)(a.rows < cap ? a.rows : cap);
  DwArgs copy = a;
  void* params[] = {&copy};
  const hipError_t err = hipLaunchKernel(
      reinterpret_cast<const void*>(&dimwise_rows<E, GL, NW>), dim3(blocks), dim3(64 * NW),
      params, 0, stream);
  return err == hipSuccess ? FPSCAN_OK : FPSCAN_ERR_LAUNCH;
}

// Lanes per group GL = P / V and waves per row NW = max(1, W * P / (64 V)).
template <class E>
int run_dw(const DwArgs& a, int P, hipStream_t stream) {
  constexpr int V = E::V;
  const int GL = P / V;
  const int NW = (a.W * P) / (64 * V) > 1 ? (a.W * P) / (64 * V) : 1;
  if constexpr (V == 4) {
    if (GL == 8 && NW == 1) return launch_dw<E, 8, 1>(a, stream);
    if (GL == 8 && NW == 2) return launch_dw<E, 8, 2>(a, stream);
    if (GL == 16 && NW == 4) return launch_dw<E, 16, 4>(a, stream);
    if (GL == 16 && NW == 8) return launch_dw<E, 16, 8>(a, stream);
    if (GL == 32 && NW == 16) return launch_dw<E, 32, 16>(a, stream);
  } else {
    if (GL == 4 && NW == 1) return launch_dw<E, 4, 1>(a, stream);
    if (GL == 8 && NW == 2) return launch_dw<E, 8, 2>(a, stream);
    if (GL == 8 && NW == 4) return launch_dw<E, 8, 4>(a, stream);
    if (GL == 16 && NW == 8) return launch_dw<E, 16, 8>(a, stream);
  }
  return FPSCAN_ERR_SEQLEN;
}

// Tiled path, taken automatically for rows of at least 64 KiB from 384 MiB per tensor.
// Measured on MI355X with `bench.py --workload dw --shape B,D,L --tiling 1|2` (bf16, p50 ms,
// row kernel / tiled): 128 KiB rows (8, 1024, 65536) 0.623 / 0.560, (2, 1024, 65536) 0.159 /
// 0.163 (256 MiB: within 3 % either way over two runs; 384 MiB measured the tiles 8 % ahead),
// (1, 1024, 65536) 0.076 / 0.092; 64 KiB rows (8, 1024, 32768) 0.304 / 0.299; 32 KiB rows
// (16, 1024, 16384) 0.279 / 0.298, (32, 1024, 16384) 0.565 / 0.559; 16 KiB rows (64, 1024,
// 8192) 0.528 / 0.558. Short rows stream well in the row kernel, and at small sizes the tiled
// launch's fixed cost (status clear, start-up claims, filling and draining the ring) is a
// large share.
constexpr int64_t kDwTiledMinBytes = 384ll << 20;
constexpr int64_t kDwTiledMinRowBytes = 64ll << 10;

struct DwTilePlan {
  bool use;
  int tpr_log2;    // tiles per row, log2
  int64_t ntiles;  // rows * tiles per row
  size_t bytes;    // workspace: one status word per tile + overrun and claim counters
};

DwTilePlan plan_dw_tiles(int64_t rows, int64_t seqlen, int size) {
  DwTilePlan t{false, 0, 0, 0};
  const int tiling = fpscan_detail::tiling_mode();
  if (tiling == 1 || seqlen < 2 * kDwChunk) return t;
  const int64_t bytes = rows * seqlen * size;  // below 2^48: no wrap
  if (bytes >= ((int64_t)1 << 32)) return t;  // one buffer range per tensor
  if (tiling == 0 && (bytes < kDwTiledMinBytes || seqlen * size < kDwTiledMinRowBytes)) return t;
  const int64_t tpr = seqlen * size / (kDwTileWaves * 1024);
  while (((int64_t)1 << t.tpr_log2) < tpr) ++t.tpr_log2;
  t.ntiles = rows << t.tpr_log2;
  if ((t.ntiles + kStatusExtraWords) * (int64_t)sizeof(uint64_t) > INT32_MAX) return t;
  t.use = true;
  t.bytes = (size_t)(t.ntiles + kStatusExtraWords) * sizeof(uint64_t);
  return t;
}

constexpr int kDwMaxDevices = 64;
std::atomic<int> g_dw_resident[kDwMaxDevices][3];  // per device and element type

// Workgroups of the tiled kernel that fit on the current device at once; 0 if the device
// cannot be queried. Cached per device and element type.
int dw_resident_blocks(const void* kernel, int slot, int threads) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kDwMaxDevices) {
    const int cached = g_dw_resident[dev][slot].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
      cus <= 0 || per_cu <= 0)
    return 0;
  const int n = cus * per_cu;
  if (dev < kDwMaxDevices) g_dw_resident[dev][slot].store(n, std::memory_order_relaxed);
  return n;
}

// Clear the status words and counters, then the persistent grid (one workgroup per resident
// slot). Returns -1 when the occupancy query fails, so that the caller takes the row kernel.
template <class E>
int run_dw_tiled(const DwArgs& a, const DwTilePlan& plan, void* workspace, hipStream_t stream) {
  constexpr int TW = kDwTileWaves;
  const void* kernel = reinterpret_cast<const void*>(&dimwise_tiles<E, TW, kDwDefer>);
  const int resident = dw_resident_blocks(kernel, E::kSlot, 64 * TW);
  if (resident <= 0) return -1;
  uint64_t* status = static_cast<uint64_t*>(workspace);
  int64_t ntiles = plan.ntiles;
  const int64_t nwords = ntiles + kStatusExtraWords;
  const int64_t clear_blocks = (nwords + 255) / 256 < 1024 ? (nwords + 255) / 256 : 1024;
  void* cargs[] = {&status, &ntiles};
  if (hipLaunchKernel(reinterpret_cast<const void*>(&clear_status), dim3((unsigned)clear_blocks),
                      dim3(256), cargs, 0, stream) != hipSuccess)
    return FPSCAN_ERR_LAUNCH;
  DwTileArgs t{a.ax, a.bx, a.bh, a.wq, a.wk, a.dim, a.seqlen, a.W * a.C,
               fpscan_detail::hook_skip_publish(), fpscan_detail::hook_spin_limit()};
  int tpr_log2 = plan.tpr_log2;
  const int64_t grid = ntiles < resident ? ntiles : resident;
  void* kargs[] = {&t, &status, &tpr_log2, &ntiles};
  const hipError_t err =
      hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(64 * TW), kargs, 0, stream);
  return err == hipSuccess ? FPSCAN_OK : FPSCAN_ERR_LAUNCH;
}

// Shape validation: FPSCAN_OK with `rows` set, or the error.
int dw_check_shape(int64_t batch, int64_t dim, int64_t seqlen, int dtype, int64_t* rows_out) {
  if (dtype != FPSCAN_DTYPE_F32 && dtype != FPSCAN_DTYPE_F16 && dtype != FPSCAN_DTYPE_BF16)
    return FPSCAN_ERR_DTYPE;
  if (dw_geom(seqlen).W == 0) return FPSCAN_ERR_SEQLEN;
  if (batch < 0 || dim < 0) return FPSCAN_ERR_SHAPE;
  // rows and elements checked for wrap-around; the tensors' bytes must stay below 2^48
  // (256 TiB, far above any device memory)
  int64_t rows = 0, elems = 0;
  if (__builtin_mul_overflow(batch, dim, &rows) || __builtin_mul_overflow(rows, seqlen, &elems) ||
      elems > ((int64_t)1 << 48) / 4)
    return FPSCAN_ERR_SHAPE;
  *rows_out = rows;
  return FPSCAN_OK;
}

// Pointer validation of a non-empty call.
int dw_check_ptrs(const void* gates, const void* tokens, const void* bh, const void* wq,
                  const void* wk, int dtype) {
  const void* ptrs[] = {gates, tokens, bh, wq, wk};
  for (const void* p : ptrs)
    if (p == nullptr) return FPSCAN_ERR_NULL;
  if ((reinterpret_cast<uintptr_t>(gates) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(tokens) & 15u) != 0)
    return FPSCAN_ERR_ALIGN;
  const int size = dtype == FPSCAN_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(bh) & (size - 1)) != 0 ||
      (reinterpret_cast<uintptr_t>(wq) & (size - 1)) != 0 ||
      (reinterpret_cast<uintptr_t>(wk) & (size - 1)) != 0)
    return FPSCAN_ERR_ALIGN;
  return FPSCAN_OK;
}

}  // namespace

namespace fpscan_detail {
// The tiled dimwise kernel's counter of given-up waits on the current device (a synchronous
// copy).
int dw_overruns(unsigned long long* count) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_dw_overruns)) != hipSuccess || p == nullptr)
    return FPSCAN_ERR_DEVICE;
  if (hipMemcpy(count, p, sizeof(*count), hipMemcpyDeviceToHost) != hipSuccess)
    return FPSCAN_ERR_DEVICE;
  return FPSCAN_OK;
}
}  // namespace fpscan_detail

extern "C" {

int fpscan_dimwise_groups(int64_t seqlen) {
  const DwGeom geo = dw_geom(seqlen);
  return geo.W * geo.C;
}

size_t fpscan_dimwise_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int dtype) {
  int64_t rows = 0;
  if (dw_check_shape(batch, dim, seqlen, dtype, &rows) != FPSCAN_OK || rows == 0) return 0;
  const DwTilePlan plan = plan_dw_tiles(rows, seqlen, dtype == FPSCAN_DTYPE_F32 ? 4 : 2);
  return plan.use ? plan.bytes : 0;
}

int fpscan_dimwise_fwd_ws(const void* gates, void* tokens, const void* bh, const void* wq,
                          const void* wk, int64_t batch, int64_t dim, int64_t seqlen, int dtype,
                          void* workspace, size_t workspace_bytes, void* stream) {
  int64_t rows = 0;
  int st = dw_check_shape(batch, dim, seqlen, dtype, &rows);
  if (st != FPSCAN_OK || rows == 0) return st;
  st = dw_check_ptrs(gates, tokens, bh, wq, wk, dtype);
  if (st != FPSCAN_OK) return st;
  if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return FPSCAN_ERR_ALIGN;
  const DwGeom geo = dw_geom(seqlen);
  DwArgs a{gates, tokens, bh, wq, wk, rows, dim, (int32_t)seqlen, geo.W, geo.C};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const DwTilePlan plan = plan_dw_tiles(rows, seqlen, dtype == FPSCAN_DTYPE_F32 ? 4 : 2);
  if (plan.use && workspace != nullptr && workspace_bytes >= plan.bytes) {
    int r = -1;
    switch (dtype) {
      case FPSCAN_DTYPE_F32: r = run_dw_tiled<F32>(a, plan, workspace, s); break;
      case FPSCAN_DTYPE_F16: r = run_dw_tiled<F16>(a, plan, workspace, s); break;
      default: r = run_dw_tiled<BF16>(a, plan, workspace, s); break;
    }
    if (r >= 0) return r;  // -1: the occupancy query failed; the row kernel runs instead
  }
  switch (dtype) {
    case FPSCAN_DTYPE_F32: return run_dw<F32>(a, geo.P, s);
    case FPSCAN_DTYPE_F16: return run_dw<F16>(a, geo.P, s);
    default: return run_dw<BF16>(a, geo.P, s);
  }
}

int fpscan_dimwise_fwd(const void* gates, void* tokens, const void* bh, const void* wq,
                       const void* wk, int64_t batch, int64_t dim, int64_t seqlen, int dtype,
                       void* stream) {
  return fpscan_dimwise_fwd_ws(gates, tokens, bh, wq, wk, batch, dim, seqlen, dtype, nullptr, 0,
                               stream);
}

}  // extern "C"

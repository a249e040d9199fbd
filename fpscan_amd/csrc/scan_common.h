// Pieces shared by the scan kernels of this library (row-major and channel-last): element
// types, buffer-resource loads and stores, mode codes. Internal header: each kernel source
// includes it, and everything in it has internal linkage.
#ifndef FPSCAN_SCAN_COMMON_H
#define FPSCAN_SCAN_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------
// Element types: V elements per 16-byte vector, exact widening, round-to-nearest-even
// narrowing (the reference's to_float/from_float, csrc/full_scan/conversion.h:7-13).
// ---------------------------------------------------------------------------------------
struct F32 {
  static constexpr int V = 4;
  static constexpr int kSize = 4;
  static constexpr int kSlot = 0;  // index of this type in per-type tables
  __device__ static __forceinline__ void unpack(const u32x4 v, float (&f)[V]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  }
  __device__ static __forceinline__ u32x4 pack(const float (&f)[V]) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __float_as_uint(f[i]);
    return v;
  }
};

struct F16 {
  static constexpr int V = 8;
  static constexpr int kSize = 2;
  static constexpr int kSlot = 1;  // index of this type in per-type tables
  __device__ static __forceinline__ void unpack(const u32x4 v, float (&f)[V]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // copy the element out first: a bit_cast of the vector-element lvalue v[i] reads
      // element 0 for every i with this compiler
      const unsigned int word = v[i];
      const f16x2 h = __builtin_bit_cast(f16x2, word);
      f[2 * i] = static_cast<float>(h.x);
      f[2 * i + 1] = static_cast<float>(h.y);
    }
  }
  __device__ static __forceinline__ u32x4 pack(const float (&f)[V]) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16x2 h;
      h.x = static_cast<_Float16>(f[2 * i]);  // v_cvt_f16_f32: round to nearest even
      h.y = static_cast<_Float16>(f[2 * i + 1]);
      v[i] = __builtin_bit_cast(unsigned int, h);
    }
    return v;
  }
  __device__ static __forceinline__ float widen16(unsigned short bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
  }
};

struct BF16 {
  static constexpr int V = 8;
  static constexpr int kSize = 2;
  static constexpr int kSlot = 2;  // index of this type in per-type tables
  __device__ static __forceinline__ void unpack(const u32x4 v, float (&f)[V]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(v[i] << 16);
      f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  }
  __device__ static __forceinline__ u32x4 pack(const float (&f)[V]) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x2 x;
      x.x = f[2 * i];
      x.y = f[2 * i + 1];
      // v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN
      v[i] = __builtin_bit_cast(unsigned int, __builtin_convertvector(x, bf16x2));
    }
    return v;
  }
  __device__ static __forceinline__ float widen16(unsigned short bits) {
    return __uint_as_float((unsigned int)bits << 16);
  }
};

// Modes: 0 forward, 1 reverse, 2 fused backward (a reverse scan).
constexpr int kFwd = 0;
constexpr int kRev = 1;
constexpr int kBwd = 2;

// Buffer resources: one per tensor per row, base = the row's first element, range = the
// row's bytes. Loads and stores then carry only a 32-bit in-row byte offset in a VGPR, and
// the hardware range check turns any offset outside the row into a zero read / dropped
// write instead of a fault.
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format
constexpr int kCacheNT = 2;             // cache-policy bit: nontemporal (streamed once)

typedef __amdgpu_buffer_rsrc_t Rsrc;

__device__ __forceinline__ Rsrc row_rsrc(const void* p, int64_t row_base, int size, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(p)) + row_base * size, (short)0, bytes, kRsrcWord3);
}

// Every element is read once: the 16-byte operand loads are nontemporal, like the stores.
__device__ __forceinline__ u32x4 bld16(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCacheNT));
}

__device__ __forceinline__ void bst16(Rsrc r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCacheNT);
}

// Byte offset that no row range contains: loads from it return 0 without touching memory.
constexpr uint32_t kNoOffset = 0x80000000u;

// ---------------------------------------------------------------------------------------
// Wave64 lane movement (DPP). Lanes whose source is outside the row / wave, or whose row is
// masked off, keep `old`.
// ---------------------------------------------------------------------------------------
constexpr int kRowShr1 = 0x111;
constexpr int kRowShr2 = 0x112;
constexpr int kRowShr4 = 0x114;
constexpr int kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142;
constexpr int kRowBcast31 = 0x143;
constexpr int kWaveShl1 = 0x130;
constexpr int kWaveShr1 = 0x138;

template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float dpp(float old, float src) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, src),
                                         kCtrl, kRowMask, 0xf, false));
}

// Workgroup barrier that orders LDS only. __syncthreads() is a workgroup-scope fence on all
// memory, which on gfx9 waits for every outstanding global load -- it would drain the operand
// ring at each barrier. The barriers here guard LDS exchanges only: operands are read-only
// and every output element is written by the lane that read its inputs.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Lane movement in which lanes without a source read 0 (bound_ctrl), for values whose such
// lanes are selected away afterwards: unlike dpp() it needs no `old` value moved into place
// first, so it is one instruction instead of two.
template <int kCtrl>
__device__ __forceinline__ float dpp_any(float src) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, src), kCtrl, 0xf, 0xf, true));
}

// Scan steps combine a lane's affine map (A, B) with an earlier lane's map (pA, pB), which is
// applied first: (A, B) := (pA·A, pB·A + B). The identity is (1, 0).
//
// combine_from_masked: the earlier lane is kCtrl's DPP source; lanes with !ok combine with
// the identity (segments narrower than a DPP row).
template <int kCtrl>
__device__ __forceinline__ void combine_from_masked(float& A, float& B, bool ok) {
  float pA = dpp_any<kCtrl>(A);
  float pB = dpp_any<kCtrl>(B);
  pA = ok ? pA : 1.0f;
  pB = ok ? pB : 0.0f;
  B = fmaf(pB, A, B);
  A = pA * A;
}

// (A, B) := (lane - 4's map) o (A, B) in DPP banks 1 and 3 (lanes 4-7 and 12-15 of each
// row); lanes of banks 0 and 2 keep their map. This is the last step of a scan over aligned
// 8-lane segments, whose lanes 4..7 are exactly those banks, so the bank mask does what a
// per-lane select would: each half is one instruction with the lane movement folded in
// (B first, from the old A). s_nop 1 gives the two wait states a DPP read of a VGPR written
// by the previous VALU instruction needs.
__device__ __forceinline__ void combine_shr4_upper_banks(float& A, float& B) {
  asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shr:4 row_mask:0xf bank_mask:0xa"
      : "+v"(B)
      : "v"(A));
  asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xa" : "+v"(A));
}

// combine_from_row: the earlier lane is kShift lanes down in the same DPP row
// (row_shr:kShift); the first kShift lanes of each row keep their map. The lane movement is
// folded into the arithmetic: B += B[lane - kShift] * A as one DPP multiply-add whose missing
// sources read 0 (bound_ctrl), then A *= A[lane - kShift] as one bank-masked DPP multiply
// (shifts 4 and 8: the lanes without a source are whole banks) or as a DPP select of 1 for
// the first kShift lanes of each row plus a multiply (shifts 1 and 2). 2-3 VALU instructions
// instead of 6 (an identity moved into place, two lane moves, multiply-add, multiply).
// s_nop 1: a DPP read of a VGPR just written needs two wait states.
template <int kShift>
__device__ __forceinline__ void combine_from_row(float& A, float& B) {
  static_assert(kShift == 1 || kShift == 2 || kShift == 4 || kShift == 8, "row shifts");
  if constexpr (kShift == 1)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shr:1 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(B) : "v"(A));
  else if constexpr (kShift == 2)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shr:2 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(B) : "v"(A));
  else if constexpr (kShift == 4)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shr:4 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(B) : "v"(A));
  else
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_shr:8 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(B) : "v"(A));
  if constexpr (kShift == 4) {
    asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xe" : "+v"(A));
  } else if constexpr (kShift == 8) {
    asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xc" : "+v"(A));
  } else {
    float pA;
    if constexpr (kShift == 1)
      asm("s_mov_b32 vcc_lo, 0x00010001\n\ts_mov_b32 vcc_hi, 0x00010001\n\ts_nop 1\n\t"
          "v_cndmask_b32_dpp %0, %1, %2, vcc row_shr:1 row_mask:0xf bank_mask:0xf bound_ctrl:1"
          : "=&v"(pA) : "v"(A), "v"(1.0f) : "vcc");
    else
      asm("s_mov_b32 vcc_lo, 0x00030003\n\ts_mov_b32 vcc_hi, 0x00030003\n\ts_nop 1\n\t"
          "v_cndmask_b32_dpp %0, %1, %2, vcc row_shr:2 row_mask:0xf bank_mask:0xf bound_ctrl:1"
          : "=&v"(pA) : "v"(A), "v"(1.0f) : "vcc");
    A = pA * A;
  }
}

// The two cross-row steps of a wave scan, folded the same way: rows outside the row mask are
// not written, which keeps their map. Row 1 takes lane 15's map and row 3 lane 47's
// (row_bcast:15, rows 1 and 3); rows 2 and 3 take lane 31's (row_bcast:31, rows 2 and 3).
__device__ __forceinline__ void combine_from_bcast15(float& A, float& B) {
  asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_bcast:15 row_mask:0xa bank_mask:0xf"
      : "+v"(B) : "v"(A));
  asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf" : "+v"(A));
}
__device__ __forceinline__ void combine_from_bcast31(float& A, float& B) {
  asm("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 row_bcast:31 row_mask:0xc bank_mask:0xf"
      : "+v"(B) : "v"(A));
  asm("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf" : "+v"(A));
}

// Inclusive scan over all 64 lanes.
__device__ __forceinline__ void wave_scan(float& A, float& B) {
  combine_from_row<1>(A, B);
  combine_from_row<2>(A, B);
  combine_from_row<4>(A, B);
  combine_from_row<8>(A, B);
  combine_from_bcast15(A, B);  // lane 15 -> row 1, lane 47 -> row 3
  combine_from_bcast31(A, B);  // lane 31 -> rows 2 and 3
}

// One step of a scan over aligned segments of 8 lanes: lanes whose position in the segment is
// below kShift keep their map, the others combine with the map kShift lanes down.
// Each select takes the lane movement as its operand (VOP2 v_cndmask with DPP, VCC = the
// lanes that keep theirs, a compile-time pattern; bound_ctrl makes row-start lanes read 0,
// and those lanes select the identity anyway), so a step is 4 VALU instructions instead of
// 6. s_nop 1 gives the two wait states a DPP read of a just-written VGPR needs. (For segments
// of 4 lanes, fp32 in the channel-last tiles, the set-up measured no faster than the plain
// masked combine, so those keep it.)
#define FPSCAN_SEGMENT_STEP(MASK, SHIFT)                                                   \
  "s_mov_b32 vcc_lo, " MASK "\n\t"                                                       \
  "s_mov_b32 vcc_hi, " MASK "\n\t"                                                       \
  "s_nop 1\n\t"                                                                          \
  "v_cndmask_b32_dpp %0, %2, %4, vcc row_shr:" SHIFT                                    \
  " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"                                          \
  "v_cndmask_b32_dpp %1, %3, %5, vcc row_shr:" SHIFT " row_mask:0xf bank_mask:0xf bound_ctrl:1"
template <int kShift>
__device__ __forceinline__ void combine_segment_step(float& A, float& B) {
  static_assert(kShift == 1 || kShift == 2, "masked DPP steps");
  float pA, pB;
  if constexpr (kShift == 1)
    asm(FPSCAN_SEGMENT_STEP("0x01010101", "1")
        : "=&v"(pA), "=&v"(pB) : "v"(A), "v"(B), "v"(1.0f), "v"(0.0f) : "vcc");
  else
    asm(FPSCAN_SEGMENT_STEP("0x03030303", "2")
        : "=&v"(pA), "=&v"(pB) : "v"(A), "v"(B), "v"(1.0f), "v"(0.0f) : "vcc");
  B = fmaf(pB, A, B);
  A = pA * A;
}
#define FPSCAN_SEGMENT_STEP2(MASK, SHIFT)                                                  \
  "s_mov_b32 vcc_lo, " MASK "\n\t"                                                       \
  "s_mov_b32 vcc_hi, " MASK "\n\t"                                                       \
  "s_nop 1\n\t"                                                                          \
  "v_cndmask_b32_dpp %0, %4, %8, vcc row_shr:" SHIFT                                    \
  " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"                                          \
  "v_cndmask_b32_dpp %1, %5, %9, vcc row_shr:" SHIFT                                    \
  " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"                                          \
  "v_cndmask_b32_dpp %2, %6, %8, vcc row_shr:" SHIFT                                    \
  " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"                                          \
  "v_cndmask_b32_dpp %3, %7, %9, vcc row_shr:" SHIFT " row_mask:0xf bank_mask:0xf bound_ctrl:1"
// combine_segment_step on two maps per lane at once: one VCC set-up for both.
template <int kShift>
__device__ __forceinline__ void combine_segment_step2(float& A0, float& B0, float& A1,
                                                      float& B1) {
  static_assert(kShift == 1 || kShift == 2, "masked DPP steps");
  float pA0, pB0, pA1, pB1;
  if constexpr (kShift == 1)
    asm(FPSCAN_SEGMENT_STEP2("0x01010101", "1")
        : "=&v"(pA0), "=&v"(pB0), "=&v"(pA1), "=&v"(pB1)
        : "v"(A0), "v"(B0), "v"(A1), "v"(B1), "v"(1.0f), "v"(0.0f) : "vcc");
  else
    asm(FPSCAN_SEGMENT_STEP2("0x03030303", "2")
        : "=&v"(pA0), "=&v"(pB0), "=&v"(pA1), "=&v"(pB1)
        : "v"(A0), "v"(B0), "v"(A1), "v"(B1), "v"(1.0f), "v"(0.0f) : "vcc");
  B0 = fmaf(pB0, A0, B0);
  A0 = pA0 * A0;
  B1 = fmaf(pB1, A1, B1);
  A1 = pA1 * A1;
}
#undef FPSCAN_SEGMENT_STEP
#undef FPSCAN_SEGMENT_STEP2

// Inclusive scan inside aligned segments of G lanes (G in {2, 4, 8, 16, 32}); sl = lane % G.
template <int G>
__device__ __forceinline__ void segment_scan(float& A, float& B, int sl) {
  if constexpr (G >= 16) {
    combine_from_row<1>(A, B);
    combine_from_row<2>(A, B);
    combine_from_row<4>(A, B);
    combine_from_row<8>(A, B);
    if constexpr (G == 32) combine_from_bcast15(A, B);
  } else if constexpr (G == 8) {
    combine_segment_step<1>(A, B);
    combine_segment_step<2>(A, B);
    combine_shr4_upper_banks(A, B);
  } else {
    combine_from_masked<kRowShr1>(A, B, sl >= 1);
    if constexpr (G == 4) combine_from_masked<kRowShr2>(A, B, sl >= 2);
  }
}

// segment_scan of K maps per lane (K even) over aligned segments of G lanes, sl = lane % G;
// segments of 8 take the maps two at a time.
template <int G, int K>
__device__ __forceinline__ void segment_scan_k(float (&A)[K], float (&B)[K], int sl) {
  static_assert(K % 2 == 0, "pairs of maps");
#pragma unroll
  for (int e = 0; e < K; e += 2) {
    if constexpr (G == 8) {
      combine_segment_step2<1>(A[e], B[e], A[e + 1], B[e + 1]);
      combine_segment_step2<2>(A[e], B[e], A[e + 1], B[e + 1]);
      combine_shr4_upper_banks(A[e], B[e]);
      combine_shr4_upper_banks(A[e + 1], B[e + 1]);
    } else {
      segment_scan<G>(A[e], B[e], sl);
      segment_scan<G>(A[e + 1], B[e + 1], sl);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Tile status words and tile claims of the persistent (look-back) kernels.
//
// A status word is 64 bits: an affine map (A, B) with B in the high half and A in the low
// half, or all-ones while nothing is published (NaNs are canonicalised, so all-ones never
// occurs as data). Workspace layout (8-byte words), `nstatus` status words first:
// [0, nstatus) status, [nstatus] wait overruns, [nstatus + kCounterStride * (1 + g)] claim
// counter of group g.
// ---------------------------------------------------------------------------------------
constexpr uint64_t kNotPublished = ~0ull;
// The map (NaN, NaN): stands in for a predecessor whose wait gave up, so that everything
// composed from it is NaN.
constexpr uint64_t kPoisonMap = 0x7fc000007fc00000ull;
constexpr uint32_t kPoisonValue = 0x7fc00000u;
constexpr int kSpinLimit = 1 << 16;  // default polls of ~1 us each (a device-coherent load)

__device__ __forceinline__ uint32_t canonical_bits(float v) {
  return v != v ? 0x7fc00000u : __float_as_uint(v);
}

__device__ __forceinline__ uint64_t pack_map(float A, float B) {
  return ((uint64_t)canonical_bits(B) << 32) | canonical_bits(A);
}

constexpr int kClaimGroups = 8;
constexpr int kCounterStride = 16;  // words: each counter on its own 128-byte line
constexpr int kStatusExtraWords = kCounterStride * (1 + kClaimGroups);

__global__ void __launch_bounds__(256) clear_status(uint64_t* __restrict__ status, int64_t ntiles) {
  const int64_t n = ntiles + kStatusExtraWords;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    status[i] = (i < ntiles) ? kNotPublished : 0ull;
}

// Claim groups over rows: group g holds rows [g rows / 8, (g + 1) rows / 8), each of
// 2^tpr_log2 tiles (the probes' tiles).
struct RowGroups {
  int64_t rows;
  int tpr_log2;
  __device__ int64_t first(int g) const { return ((int64_t)g * rows / kClaimGroups) << tpr_log2; }
};

// RowGroups with each group's first tile computed where it is used: the index is made opaque,
// so the compiler does not precompute all nine bounds ahead of a kernel's loop and hold them
// (18 scalar registers) across it. For kernels short of scalar registers (the tiled dimwise
// kernel: its spills to VGPR lanes cost it; the tiled row scan measured the same either way).
// g is uniform (one lane claims).
struct RowGroupsLazy {
  int64_t rows;
  int tpr_log2;
  __device__ int64_t first(int g) const {
    g = __builtin_amdgcn_readfirstlane(g);
    asm volatile("" : "+s"(g));
    return ((int64_t)g * rows / kClaimGroups) << tpr_log2;
  }
};

// Tile claims, made by one lane per workgroup. One counter at one address serialises at the
// memory side (measured: about 70 claims per microsecond, fewer than a bf16 forward scan
// finishes tiles), so the tiles are split into kClaimGroups contiguous ranges with a counter
// each (whole rows, or whole chains of the channel-last scan, per group: `Groups`). A
// workgroup starts in the group its kernel picks (most: blockIdx % kClaimGroups, its XCD
// under round-robin dispatch) and, when that one is used up, moves to the group with the most
// tiles left. A row never spans two groups and tiles of a group are claimed in order, so a
// tile's predecessors are always claimed before it. Claims are issued two steps before their
// tile is needed (an atomic at the memory side takes a few microseconds under full streaming
// load), so each claim is kept with the group it was made in. In the main loop every lane of
// every wave issues the claim as a buffer atomic that is out of range except in the leader's
// lane: a claim inside a branch, or any use of its result before it is resolved, makes the
// compiler wait for it together with every load issued before it. Counters are the low 32
// bits of their words.
struct Claim {
  uint32_t raw;
  int grp;
};

template <class Groups>
struct Claims {
  uint32_t counters_off;  // byte offset of group 0's counter in the status buffer
  const uint32_t* counters;
  Groups groups;          // first tile of each group: groups.first(g), g in [0, kClaimGroups]
  int grp;

  __device__ int64_t group_first(int g) const { return groups.first(g); }
  __device__ uint32_t counter_off() const {
    return counters_off + (uint32_t)(grp * kCounterStride * sizeof(uint64_t));
  }
  // Straight-line claim: `mine` selects the one lane that really claims.
  __device__ Claim issue(Rsrc st, bool mine) const {
    return Claim{(uint32_t)__builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(
                     1, st, mine ? counter_off() : kNoOffset, 0, 0),
                 grp};
  }
  // The group with the most unclaimed tiles, or -1 when every tile is claimed. All counters
  // are read at once (one round trip).
  __device__ int pick_group() const {
    uint32_t c[kClaimGroups];
#pragma unroll
    for (int g = 0; g < kClaimGroups; ++g)
      c[g] = __hip_atomic_load(counters + 2 * kCounterStride * g, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    int best = -1;
    int64_t best_left = 0;
#pragma unroll
    for (int g = 0; g < kClaimGroups; ++g) {
      const int64_t left = group_first(g + 1) - group_first(g) - (int64_t)c[g];
      if (left > best_left) {
        best_left = left;
        best = g;
      }
    }
    return best;
  }
  // The tile a claim stands for: a tile index, `bubble` when its group was used up (claims
  // then go to the group with the most tiles left), or `done` once every tile is claimed.
  __device__ int64_t resolve(Claim c, int64_t bubble, int64_t done) {
    const int64_t lo = group_first(c.grp);
    if (lo + (int64_t)c.raw < group_first(c.grp + 1)) return lo + (int64_t)c.raw;
    if (c.grp != grp) return bubble;  // made before the move to the current group
    const int g = pick_group();
    if (g < 0) return done;
    grp = g;
    return bubble;
  }
  // Claims until a tile or `done` comes back (start-up, leader only: waits for each atomic).
  __device__ int64_t next_now(Rsrc st, int64_t bubble, int64_t done) {
    int64_t t = bubble;
    while (t == bubble) t = resolve(issue(st, true), bubble, done);
    return t;
  }
};

// Status words go through a buffer resource too: every lane and wave issues the same
// instructions, and the ones that must not touch memory use kNoOffset (reads return 0, writes
// are dropped). Straight-line code keeps the compiler's wait counts partial, which is what
// keeps the operand ring in flight. The cache policy is the device-coherent one (sc1), the
// same instruction an agent-scope relaxed atomic load/store of 64 bits compiles to here.
constexpr int kCacheCoherent = 16;

__device__ __forceinline__ uint64_t status_load(Rsrc r, uint32_t off) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCacheCoherent));
  return ((uint64_t)v.y << 32) | v.x;
}

__device__ __forceinline__ void status_store(Rsrc r, uint32_t off, uint64_t word) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  u32x2 v;
  v.x = (uint32_t)word;
  v.y = (uint32_t)(word >> 32);
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kCacheCoherent);
}

}  // namespace

#endif  // FPSCAN_SCAN_COMMON_H

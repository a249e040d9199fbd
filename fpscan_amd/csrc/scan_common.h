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

// (A, B) := (earlier) o (A, B): the earlier lane's map is applied first.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ void combine_from(float& A, float& B) {
  const float pA = dpp<kCtrl, kRowMask>(1.0f, A);
  const float pB = dpp<kCtrl, kRowMask>(0.0f, B);
  B = fmaf(pB, A, B);
  A = pA * A;
}

// Same, but lanes with !ok combine with the identity (segments narrower than a DPP row).
template <int kCtrl>
__device__ __forceinline__ void combine_from_masked(float& A, float& B, bool ok) {
  float pA = dpp<kCtrl>(1.0f, A);
  float pB = dpp<kCtrl>(0.0f, B);
  pA = ok ? pA : 1.0f;
  pB = ok ? pB : 0.0f;
  B = fmaf(pB, A, B);
  A = pA * A;
}

// Inclusive scan over all 64 lanes.
__device__ __forceinline__ void wave_scan(float& A, float& B) {
  combine_from<kRowShr1>(A, B);
  combine_from<kRowShr2>(A, B);
  combine_from<kRowShr4>(A, B);
  combine_from<kRowShr8>(A, B);
  combine_from<kRowBcast15, 0xa>(A, B);  // lane 15 -> row 1, lane 47 -> row 3
  combine_from<kRowBcast31, 0xc>(A, B);  // lane 31 -> rows 2 and 3
}

// Inclusive scan inside aligned segments of G lanes (G in {4, 8, 16, 32}); sl = lane % G.
template <int G>
__device__ __forceinline__ void segment_scan(float& A, float& B, int sl) {
  if constexpr (G >= 16) {
    combine_from<kRowShr1>(A, B);
    combine_from<kRowShr2>(A, B);
    combine_from<kRowShr4>(A, B);
    combine_from<kRowShr8>(A, B);
    if constexpr (G == 32) combine_from<kRowBcast15, 0xa>(A, B);
  } else {
    combine_from_masked<kRowShr1>(A, B, sl >= 1);
    combine_from_masked<kRowShr2>(A, B, sl >= 2);
    if constexpr (G == 8) combine_from_masked<kRowShr4>(A, B, sl >= 4);
  }
}

}  // namespace

#endif  // FPSCAN_SCAN_COMMON_H

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

#include "fpscan_hip.h"
#include "scan_common.h"

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

}  // namespace

extern "C" {

int fpscan_dimwise_groups(int64_t seqlen) {
  const DwGeom geo = dw_geom(seqlen);
  return geo.W * geo.C;
}

int fpscan_dimwise_fwd(const void* gates, void* tokens, const void* bh, const void* wq,
                       const void* wk, int64_t batch, int64_t dim, int64_t seqlen, int dtype,
                       void* stream) {
  if (dtype != FPSCAN_DTYPE_F32 && dtype != FPSCAN_DTYPE_F16 && dtype != FPSCAN_DTYPE_BF16)
    return FPSCAN_ERR_DTYPE;
  const DwGeom geo = dw_geom(seqlen);
  if (geo.W == 0) return FPSCAN_ERR_SEQLEN;
  if (batch < 0 || dim < 0) return FPSCAN_ERR_SHAPE;
  if (batch == 0 || dim == 0) return FPSCAN_OK;
  // rows and elements checked for wrap-around; the tensors' bytes must stay below 2^48
  // (256 TiB, far above any device memory)
  int64_t rows = 0, elems = 0;
  if (__builtin_mul_overflow(batch, dim, &rows) || __builtin_mul_overflow(rows, seqlen, &elems) ||
      elems > ((int64_t)1 << 48) / 4)
    return FPSCAN_ERR_SHAPE;
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
  DwArgs a{gates, tokens, bh, wq, wk, rows, dim, (int32_t)seqlen, geo.W, geo.C};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FPSCAN_DTYPE_F32: return run_dw<F32>(a, geo.P, s);
    case FPSCAN_DTYPE_F16: return run_dw<F16>(a, geo.P, s);
    default: return run_dw<BF16>(a, geo.P, s);
  }
}

}  // extern "C"

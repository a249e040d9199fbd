// First-order linear-recurrence scan for MI355X (gfx950, wave64), behind the C ABI in
// include/fpscan_hip.h.
//
//   y[t] = gates[t] * y[t-1] + tokens[t]          (forward; reverse runs t = L-1 .. 0)
//
// Reference kernel replaced: csrc/full_scan/full_scan.cu:50-177 (blocked 3-level scan,
// 32-lane warps, 3 barriers per chunk, carry through shared memory) and its launcher
// full_scan.cu:179-258. The backward composition of fpscan/ops.py:69-83 is fused into one
// kernel here.
//
// Work decomposition
//   A "sub-chunk" is 64 lanes x one 16-byte vector per lane per tensor: 256 fp32 or 512
//   fp16/bf16 consecutive elements of one row. Every global load/store instruction of a
//   wave therefore covers one contiguous 1 KiB span.
//   Long rows (seqlen >= one sub-chunk): W waves (1..16) own a row and walk its sub-chunks
//   in rounds of W; wave w takes sub-chunk r*W+w of round r. A ring of U sub-chunks per wave
//   is kept in flight (loads for round r+U are issued as round r is retired). The carry
//   between rounds is a wave-uniform fp32 value; with W > 1 the W sub-chunk aggregates of a
//   round are exchanged through 2 x W x 8 bytes of LDS and one barrier.
//   Short rows (seqlen < one sub-chunk): each wave holds 64/G whole rows of G lanes and runs
//   a segmented wave scan; no carry.
//
// Per sub-chunk, per lane (V elements, processing order):
//   phase 1  lane aggregate (A, B) = composition of the lane's V affine maps y -> a*y + b;
//   scan     inclusive wave scan of the lane aggregates with DPP row_shr 1/2/4/8 and
//            row_bcast 15/31; identity (1, 0) enters through DPP's `old` operand;
//   carry    value entering the lane = wave_shr:1 of (B + A * c_in), lane 0 takes c_in;
//   phase 2  the lane's V elements re-run serially from that value: y = fma(a, y, b).
// All arithmetic is fp32; half types are widened exactly on load and rounded to nearest
// even once on store.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "fpscan_hip.h"
#include "scan_common.h"

namespace {

// ---------------------------------------------------------------------------------------
// Launch arguments. Modes: 0 forward, 1 reverse, 2 fused backward (a reverse scan).
// fwd/rev: in0 = gates, in1 = tokens, out0 = out.
// bwd:     in0 = gates, in1 = grad_out, in2 = saved forward output, out0 = grad_tokens,
//          out1 = grad_gates.
// ---------------------------------------------------------------------------------------
struct Args {
  const void* in0;
  const void* in1;
  const void* in2;
  void* out0;
  void* out1;
  int64_t rows;
  int64_t dim;
  int64_t stride_b;
  int64_t stride_d;
  int32_t seqlen;
  int32_t contiguous;
  // fused softplus gates only: per-channel rate (dim floats) and, for the backward, one
  // partial sum of d loss / d rate per row (rows floats, may be null)
  const float* rate;
  float* grad_rate_rows;
  // tiled path: polls before a look-back wait gives up, and a tile whose map is never
  // published (-1: none; a test hook that forces a wait to give up)
  int64_t skip_publish;
  int32_t spin_limit;
};

// Look-back waits that gave up on this device since the library was loaded (the tiled row
// kernel's; the channel-last kernels keep their own). Read by fpscan_lookback_overruns.
static __device__ unsigned long long g_row_overruns;


__device__ __forceinline__ int64_t row_offset(const Args& a, int64_t row) {
  if (a.contiguous) return row * a.seqlen;
  const int64_t b = row / a.dim;
  const int64_t d = row - b * a.dim;
  return b * a.stride_b + d * a.stride_d;
}

__device__ __forceinline__ u32x4 ld16(const void* base, int64_t elem, int size) {
  return *reinterpret_cast<const u32x4*>(static_cast<const char*>(base) + elem * size);
}

__device__ __forceinline__ void st16(void* base, int64_t elem, int size, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<char*>(base) + elem * size));
}


// One element, as loaded: its bits (a 16-bit type zero-extended); widen_bits makes the fp32
// value. The two are apart so that a kernel can keep the conversion next to its use.
template <class E>
__device__ __forceinline__ uint32_t bld1_bits(Rsrc r, uint32_t off) {
  if constexpr (E::kSize == 4) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
}

template <class E>
__device__ __forceinline__ float widen_bits(uint32_t bits) {
  if constexpr (E::kSize == 4) {
    return __uint_as_float(bits);
  } else {
    return E::widen16((unsigned short)bits);
  }
}

// Loaded operands of one sub-chunk for one lane, plus the two wave-uniform boundary values
// the backward needs (as loaded, see bld1_bits): the gate just past the sub-chunk and the
// output just before it.
template <int kMode>
struct Slot {
  u32x4 v[kMode == kBwd ? 3 : 2];
  uint32_t gate_after;
  uint32_t out_before;
};

template <int kMode>
struct RowRsrc {
  Rsrc in0, in1, in2, out0, out1;
};


// Issues the loads of one sub-chunk. `sub_bytes` is the wave-uniform byte offset of the
// sub-chunk inside the row, or kNoOffset for a ring slot past the end of the row (the loads
// are still issued so that the wait counts stay static). Boundary values read outside the
// row come back as 0 and are replaced by the identity where they are used.
template <class E, int kMode>
__device__ __forceinline__ void load_slot(const RowRsrc<kMode>& rr, Slot<kMode>& s,
                                          uint32_t sub_bytes, uint32_t lane_off) {
  constexpr int kSubBytes = 64 * 16;
  const uint32_t off = sub_bytes + lane_off;
  s.v[0] = bld16(rr.in0, off);
  s.v[1] = bld16(rr.in1, off);
  if constexpr (kMode == kBwd) {
    s.v[2] = bld16(rr.in2, off);
    s.gate_after = bld1_bits<E>(rr.in0, sub_bytes + kSubBytes);
    s.out_before = bld1_bits<E>(rr.in2, sub_bytes - E::kSize);
  }
}

// ---------------------------------------------------------------------------------------
// Gate producers. GatePlain: the gates tensor holds the gates. GateSoftplus: it holds z, and
// the gate is exp(-softplus(z) * rate[d]) -- a Mamba-style decay (delta = softplus(z),
// A = -rate) -- computed on load, so the gates never exist in memory.
// ---------------------------------------------------------------------------------------
struct GatePlain {
  static constexpr bool kFused = false;
  template <int V>
  struct Aux {};
  __device__ static __forceinline__ float gate(float g, float) { return g; }
};

struct GateSoftplus {
  static constexpr bool kFused = true;
  // per element, memory order, for the backward: from eval, rate * sigmoid(z) and softplus(z)
  // (d gate / d z and d gate / d rate are -gate times them); make_maps then multiplies both by
  // -gate * y[t-1]
  template <int V>
  struct Aux {
    float dz[V];
    float dr[V];
  };
  // softplus(z) = max(z, 0) + ln(1 + t), t = exp(-|z|) in (0, 1]; exp and log through the
  // hardware's base-2 instructions, so ln(w) = ln2 * log2(w) and the gate is
  // exp2(-rate * log2(e) * softplus(z)). sigmoid(z) = 1/w (z >= 0) or t/w, w = fl(1 + t).
  //
  // Rounding w = fl(1 + t) drops the low bits of t: ln(w) alone is off by up to 6e-8 absolute,
  // which for z below about -7 (softplus t-sized) is 1e-4 relative at z = -10 and all of it
  // below z = -16.6 (w = 1). Both the gate (whose exponent is softplus * rate, so the error
  // grows with the rate) and d gate / d rate = -gate * softplus need softplus to relative
  // accuracy there. The dropped part is recovered exactly (Fast2Sum: e = t - (w - 1), both
  // subtractions exact for t in [0, 1]) and ln(1 + t) = ln(w) + ln(1 + e/w) = ln(w) + e up to
  // e * t / w < 2^-24 t, below fp32 resolution: the log1p correction for three VALU
  // instructions and no further transcendental one (4 in all, 3 where only the gate is used).
  __device__ static __forceinline__ void eval(float z, float rate, float& gate, float& dz,
                                              float& dr) {
    constexpr float kLog2e = 1.4426950408889634f;
    constexpr float kLn2 = 0.6931471805599453f;
    const float t = __builtin_amdgcn_exp2f(-fabsf(z) * kLog2e);
    const float w = 1.0f + t;
    const float rw = __builtin_amdgcn_rcpf(w);
    float zpos;
    // max(z, 0) in one instruction (fmaxf adds a canonicalising one); a NaN z still gives a
    // NaN softplus, through t
    asm("v_max_f32 %0, 0, %1" : "=v"(zpos) : "v"(z));
    const float sum_err = t - (w - 1.0f);  // exact: the part of t that w = fl(1 + t) dropped
    const float sp = fmaf(__builtin_amdgcn_logf(w), kLn2, zpos + sum_err);
    gate = __builtin_amdgcn_exp2f(-(sp * (rate * kLog2e)));
    const float sig = (z >= 0.0f) ? rw : t * rw;
    dz = rate * sig;  // d gate / d z = -gate * dz
    dr = sp;          // d gate / d rate = -gate * dr
  }
  __device__ static __forceinline__ float gate(float z, float rate) {
    float g, dz, dr;
    eval(z, rate, g, dz, dr);
    return g;
  }
};

// Builds the per-lane affine maps (alpha, beta) in processing order from a loaded slot.
// For the backward also returns y[t-1] per element (processing order) in ysh.
// `gate_next`/`out_prev` are the neighbour values for the lanes at the edges of the span
// (uniform boundary values for long rows, the identity for short-row segments);
// `span_first_lane`/`span_last_lane` say whether this lane is the first/last lane of its
// span in processing order.
template <class E, int kMode, class Gp = GatePlain>
__device__ __forceinline__ void make_maps(const Slot<kMode>& s, float (&al)[E::V], float (&be)[E::V],
                                          float (&ysh)[E::V], float gate_next, float out_prev,
                                          bool span_first_lane, bool span_last_lane,
                                          float rate = 0.0f,
                                          typename Gp::template Aux<E::V>* aux = nullptr) {
  constexpr int V = E::V;
  float g[V], x[V];
  E::unpack(s.v[0], g);
  E::unpack(s.v[1], x);
  if constexpr (Gp::kFused) {
    // z -> gates (memory order); `gate_next` arrives already converted
#pragma unroll
    for (int e = 0; e < V; ++e) Gp::eval(g[e], rate, g[e], aux->dz[e], aux->dr[e]);
  }
  if constexpr (kMode == kBwd) {
    float y[V];
    E::unpack(s.v[2], y);
    // gates[t+1]: inside the vector, then from the lane holding the next vector in memory
    // (scan lane - 1, wave_shr:1); the span's first lane (memory-last vector) takes gate_next.
    float gs_last = dpp<kWaveShr1>(gate_next, g[0]);
    gs_last = span_first_lane ? gate_next : gs_last;
    // y[t-1]: inside the vector, then from the lane holding the previous vector in memory
    // (scan lane + 1, wave_shl:1); the span's last lane (memory-first vector) takes out_prev.
    float ys_first = dpp<kWaveShl1>(out_prev, y[V - 1]);
    ys_first = span_last_lane ? out_prev : ys_first;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int e = V - 1 - k;  // memory index, processed last-to-first
      al[k] = (e == V - 1) ? gs_last : g[e + 1];
      be[k] = x[e];
      ysh[k] = (e == 0) ? ys_first : y[e - 1];
    }
    if constexpr (Gp::kFused) {
      // d loss / d z = grad_tokens * (y[t-1] * d gate / d z), and likewise for the rate: the
      // products with -gate * y[t-1] are formed here, so that neither the gate nor y[t-1] is
      // held across the scan
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float c = -g[e] * ysh[V - 1 - e];
        aux->dz[e] *= c;
        aux->dr[e] *= c;
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int e = (kMode == kRev) ? V - 1 - k : k;
      al[k] = g[e];
      be[k] = x[e];
      ysh[k] = 0.0f;
    }
  }
}

template <class E>
__device__ __forceinline__ void lane_aggregate(const float (&al)[E::V], const float (&be)[E::V],
                                               float& A, float& B) {
  A = al[0];
  B = be[0];
#pragma unroll
  for (int k = 1; k < E::V; ++k) {
    B = fmaf(al[k], B, be[k]);
    A = A * al[k];
  }
}

// Re-runs the lane's elements from the value entering the lane; returns the packed output
// vector(s) in memory order (o1 only for the backward: grad_gates).
template <class E, int kMode, class Gp = GatePlain>
__device__ __forceinline__ void finish_lane(const float (&al)[E::V], const float (&be)[E::V],
                                            const float (&ysh)[E::V], float y, u32x4& o0,
                                            u32x4& o1,
                                            const typename Gp::template Aux<E::V>* aux = nullptr,
                                            float* rate_sum = nullptr) {
  constexpr int V = E::V;
  float res[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    y = fmaf(al[k], y, be[k]);
    res[k] = y;
  }
  float om[V];
#pragma unroll
  for (int e = 0; e < V; ++e) om[e] = (kMode == kFwd) ? res[e] : res[V - 1 - e];
  o0 = E::pack(om);
  if constexpr (kMode == kBwd) {
    float gg[V];
    if constexpr (Gp::kFused) {
      // d loss / d z (written) and d loss / d rate (summed per row); aux holds the gate
      // derivatives already multiplied by y[t-1]
#pragma unroll
      for (int e = 0; e < V; ++e) {
        *rate_sum = fmaf(om[e], aux->dr[e], *rate_sum);
        gg[e] = om[e] * aux->dz[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) gg[e] = om[e] * ysh[V - 1 - e];
    }
    o1 = E::pack(gg);
  }
}

// Sums of one value over the wave (result in every lane) and over aligned segments of G
// lanes (inclusive: the segment's last lane holds its total).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kRowShr1>(0.0f, v);
  v += dpp<kRowShr2>(0.0f, v);
  v += dpp<kRowShr4>(0.0f, v);
  v += dpp<kRowShr8>(0.0f, v);
  v += dpp<kRowBcast15, 0xa>(0.0f, v);
  v += dpp<kRowBcast31, 0xc>(0.0f, v);
  return readlane(v, 63);
}

template <int G>
__device__ __forceinline__ float segment_sum(float v, int sl) {
  if constexpr (G >= 16) {
    v += dpp<kRowShr1>(0.0f, v);
    v += dpp<kRowShr2>(0.0f, v);
    v += dpp<kRowShr4>(0.0f, v);
    v += dpp<kRowShr8>(0.0f, v);
    if constexpr (G == 32) v += dpp<kRowBcast15, 0xa>(0.0f, v);
  } else {
    float s = dpp<kRowShr1>(0.0f, v);
    v += sl >= 1 ? s : 0.0f;
    s = dpp<kRowShr2>(0.0f, v);
    v += sl >= 2 ? s : 0.0f;
    if constexpr (G == 8) {
      s = dpp<kRowShr4>(0.0f, v);
      v += sl >= 4 ? s : 0.0f;
    }
  }
  return v;
}

// ---------------------------------------------------------------------------------------
// Long rows: W waves per row, U sub-chunks in flight per wave.
// ---------------------------------------------------------------------------------------
// R: rows per block when W == 1 (one wave per row), 1 otherwise.
template <class E, int kMode, int W, int U, class Gp = GatePlain, int R = (W == 1 ? 4 : 1)>
__global__ void __launch_bounds__(W == 1 ? 64 * R : 64 * W) scan_long_rows(const Args a) {
  constexpr int V = E::V;
  constexpr int kSub = 64 * V;
  constexpr bool kReverse = kMode != kFwd;
  constexpr int kRowsPerBlock = (W == 1) ? R : 1;
  static_assert(W == 1 || R == 1, "several rows per block only with one wave per row");

  __shared__ f32x2 exch[2][W];
  __shared__ float rate_part[W];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = (W == 1) ? 0 : wave;
  const int vec = kReverse ? 63 - lane : lane;  // memory vector of this lane in a sub-chunk
  const uint32_t lane_off = (uint32_t)vec * 16u;
  const int nsub = a.seqlen / kSub;
  const int nrounds = nsub / W;
  const int row_bytes = a.seqlen * E::kSize;
  const int64_t ngroups = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;

  for (int64_t grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {
    const int64_t row = grp * kRowsPerBlock + ((W == 1) ? wave : 0);
    if (W == 1 && row >= a.rows) break;  // wave-uniform; no barriers when W == 1
    const int64_t base = row_offset(a, row);
    RowRsrc<kMode> rr;
    rr.in0 = row_rsrc(a.in0, base, E::kSize, row_bytes);
    rr.in1 = row_rsrc(a.in1, base, E::kSize, row_bytes);
    rr.out0 = row_rsrc(a.out0, base, E::kSize, row_bytes);
    if constexpr (kMode == kBwd) {
      rr.in2 = row_rsrc(a.in2, base, E::kSize, row_bytes);
      rr.out1 = row_rsrc(a.out1, base, E::kSize, row_bytes);
    }
    float rate = 0.0f, rate_sum = 0.0f;
    if constexpr (Gp::kFused) rate = a.rate[row % a.dim];

    // byte offset inside the row of the sub-chunk this wave handles in round r
    auto sub_bytes = [&](int r) -> uint32_t {
      const int j = r * W + w;
      return (uint32_t)((kReverse ? (nsub - 1 - j) : j) * kSub * E::kSize);
    };

    Slot<kMode> ring[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      load_slot<E, kMode>(rr, ring[u], sub_bytes(u), lane_off);
      __builtin_amdgcn_sched_barrier(0);  // slot u's loads before slot u+1's (wait counts)
    }

    float carry = 0.0f;
    for (int r0 = 0; r0 < nrounds; r0 += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u;
        const uint32_t sb = sub_bytes(r);
        float gate_next = 1.0f, out_prev = 0.0f;
        if constexpr (kMode == kBwd) {
          // identity at the row edges: gates[L] = 1, y[-1] = 0
          gate_next = (sb + kSub * E::kSize < (uint32_t)row_bytes)
                          ? Gp::gate(widen_bits<E>(ring[u].gate_after), rate)
                          : 1.0f;
          out_prev = (sb > 0) ? widen_bits<E>(ring[u].out_before) : 0.0f;
        }
        float al[V], be[V], ysh[V];
        typename Gp::template Aux<V> aux;
        make_maps<E, kMode, Gp>(ring[u], al, be, ysh, gate_next, out_prev, lane == 0, lane == 63,
                                rate, &aux);
        if constexpr (Gp::kFused && kMode == kBwd) {
          // the gate derivatives are formed here, before the scan: left to the compiler, it
          // sinks them to their use after the barrier and keeps their five inputs per element
          // live across the scan instead of the two results
#pragma unroll
          for (int e = 0; e < V; ++e) asm volatile("" : "+v"(aux.dz[e]), "+v"(aux.dr[e]));
        }
        if (kMode != kBwd && r == 0 && w == 0 && lane == 0) {
          // the first element of the row in processing order never uses its gate
          // (gates[0] forward, gates[L-1] reverse), as in full_scan.cu:96
          al[0] = 1.0f;
        }
        float A, B;
        lane_aggregate<E>(al, be, A, B);
        wave_scan(A, B);
        float c_in = carry;
        if constexpr (W == 1) {
          carry = fmaf(readlane(A, 63), carry, readlane(B, 63));
        } else {
          // the W sub-chunk aggregates of this round, scanned across lanes 0..W-1 (one DPP row)
          if (lane == 63) exch[r & 1][w] = f32x2{A, B};
          lds_barrier();
          float eA = 1.0f, eB = 0.0f;
          if (lane < W) {
            const f32x2 t = exch[r & 1][lane];
            eA = t.x;
            eB = t.y;
          }
          combine_from_row<1>(eA, eB);
          if constexpr (W > 2) combine_from_row<2>(eA, eB);
          if constexpr (W > 4) combine_from_row<4>(eA, eB);
          if constexpr (W > 8) combine_from_row<8>(eA, eB);
          if (w > 0) c_in = fmaf(readlane(eA, w - 1), carry, readlane(eB, w - 1));
          carry = fmaf(readlane(eA, W - 1), carry, readlane(eB, W - 1));
        }
        const float y_lane_end = fmaf(A, c_in, B);
        const float y_enter = dpp<kWaveShr1>(c_in, y_lane_end);
        u32x4 o0, o1;
        finish_lane<E, kMode, Gp>(al, be, ysh, y_enter, o0, o1, &aux, &rate_sum);
        bst16(rr.out0, sb + lane_off, o0);
        if constexpr (kMode == kBwd) bst16(rr.out1, sb + lane_off, o1);
        const uint32_t next = (r + U < nrounds) ? sub_bytes(r + U) : kNoOffset;
        load_slot<E, kMode>(rr, ring[u], next, lane_off);
        // keep the ring order: without this the scheduler hoists the next slot's arithmetic
        // above this slot's refill, which turns every wait into a wait for all loads
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (Gp::kFused && kMode == kBwd) {
      // d loss / d rate of this row: lanes, then waves in order (deterministic)
      const float s = wave_sum(rate_sum);
      if constexpr (W == 1) {
        if (a.grad_rate_rows != nullptr && lane == 0) a.grad_rate_rows[row] = s;
      } else {
        if (lane == 0) rate_part[w] = s;
        lds_barrier();
        if (w == 0 && lane == 0 && a.grad_rate_rows != nullptr) {
          float tot = 0.0f;
          for (int i = 0; i < W; ++i) tot += rate_part[i];
          a.grad_rate_rows[row] = tot;
        }
        lds_barrier();  // rate_part is rewritten by the next row
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Long rows, tiled: a persistent grid walks tiles in memory order.
//
// A tile is TW consecutive sub-chunks of one row (TW KiB of each tensor), handled by one
// workgroup of TW waves. Workgroups claim tiles in increasing order from counters (one atomic
// per tile; see Claims), so the tiles in flight at any moment form a few contiguous windows
// of each tensor -- the access pattern of a plain streaming kernel. Tiles of one row are
// chained by a decoupled look-back:
//   1. each tile reduces its own data to one affine map (A, B) and publishes it at once as
//      one 64-bit word in `status` (B in the high half, A in the low half; all-ones = not yet
//      published; NaNs are canonicalised so all-ones never occurs as data);
//   2. the carry into the tile is the composition of the words of all preceding tiles of the
//      row (a row has at most 64 tiles, so one wave scan over 64 lanes covers them; tiles
//      before the row start enter as the constant map 0, i.e. the zero initial state);
//   3. the tile applies that carry and stores.
// The look-back is deferred by one tile to keep its coherent-load latency off the critical
// path: after reducing and publishing tile k, wave 0 loads tile k's predecessor words (before
// issuing the next operand loads, since vector loads complete in issue order); the workgroup
// then reduces tile k+1 and only after that uses the words to finish tile k. A ring of three
// tiles per workgroup (k finishing, k+1 reducing, k+2 in flight) holds the operands.
// Forward progress needs no co-residency: publishing never waits, a tile is claimed only by a
// workgroup that is already running, and a tile's predecessors were claimed before it. So,
// within each claim group, the workgroup owning the lowest unpublished tile is running and
// only ever waits on lower tiles, which are published; it makes progress. Each wait is also
// bounded; a wait that exceeds the bound (which a correct launch never reaches) counts itself
// in the overrun word after the status array and in a per-device counter that the host can
// read, replaces the missing maps by NaN maps, so that the tile's outputs are NaN rather than
// plausible, and proceeds, so the kernel always terminates.
//
// Workspace layout (8-byte words): [0, ntiles) tile status, [ntiles] wait overruns,
// [ntiles + kCounterStride * (1 + g)] claim counter of group g.
// ---------------------------------------------------------------------------------------

// Per-slot state of the tile ring: the tile, its row resources, its segment in the row and
// the operands of this wave's sub-chunk.
template <int kMode>
struct TileSlot {
  Slot<kMode> data;
  RowRsrc<kMode> rr;
  int64_t tile;
  int seg;
};

template <class E, int kMode, int TW>
__device__ __forceinline__ void tile_setup(const Args& a, TileSlot<kMode>& ts, int64_t tile,
                                           int64_t ntiles, int tpr_log2, int w, uint32_t lane_off) {
  constexpr int kSub = 64 * E::V;
  constexpr bool kReverse = kMode != kFwd;
  ts.tile = tile;
  const bool live = tile < ntiles;
  const int64_t row = live ? (tile >> tpr_log2) : 0;
  ts.seg = live ? (int)(tile & ((1 << tpr_log2) - 1)) : 0;
  const int64_t base = row_offset(a, row);
  const int row_bytes = a.seqlen * E::kSize;
  ts.rr.in0 = row_rsrc(a.in0, base, E::kSize, row_bytes);
  ts.rr.in1 = row_rsrc(a.in1, base, E::kSize, row_bytes);
  ts.rr.out0 = row_rsrc(a.out0, base, E::kSize, row_bytes);
  if constexpr (kMode == kBwd) {
    ts.rr.in2 = row_rsrc(a.in2, base, E::kSize, row_bytes);
    ts.rr.out1 = row_rsrc(a.out1, base, E::kSize, row_bytes);
  }
  const int nsub = a.seqlen / kSub;
  const int j = ts.seg * TW + w;
  const uint32_t sb = live ? (uint32_t)((kReverse ? nsub - 1 - j : j) * kSub * E::kSize) : kNoOffset;
  load_slot<E, kMode>(ts.rr, ts.data, sb, lane_off);
}

// The affine maps of this wave's sub-chunk of a tile, in processing order (see make_maps);
// returns the sub-chunk's byte offset in its row.
template <class E, int kMode, int TW>
__device__ __forceinline__ uint32_t tile_maps(const TileSlot<kMode>& ts, int nsub, int row_bytes,
                                              int w, int lane, float (&al)[E::V],
                                              float (&be)[E::V], float (&ysh)[E::V]) {
  constexpr int kSub = 64 * E::V;
  constexpr bool kReverse = kMode != kFwd;
  const int j = ts.seg * TW + w;
  const uint32_t sb = (uint32_t)((kReverse ? nsub - 1 - j : j) * kSub * E::kSize);
  float gate_next = 1.0f, out_prev = 0.0f;
  if constexpr (kMode == kBwd) {
    // converted here, where the step waits for the slot's loads anyway: the empty asm keeps
    // the compiler from converting right after the load, which would wait for it there
    uint32_t ga = ts.data.gate_after, ob = ts.data.out_before;
    asm volatile("" : "+v"(ga), "+v"(ob));
    gate_next = (sb + kSub * E::kSize < (uint32_t)row_bytes) ? widen_bits<E>(ga) : 1.0f;
    out_prev = (sb > 0) ? widen_bits<E>(ob) : 0.0f;
  }
  make_maps<E, kMode>(ts.data, al, be, ysh, gate_next, out_prev, lane == 0, lane == 63);
  if (kMode != kBwd && j == 0 && lane == 0) al[0] = 1.0f;  // full_scan.cu:96
  return sb;
}

template <class E, int kMode, int TW, int D>
__global__ void __launch_bounds__(64 * TW)
scan_tiles(const Args a, uint64_t* __restrict__ status, const int tpr_log2, const int64_t ntiles) {
  constexpr int V = E::V;
  constexpr int kSub = 64 * V;
  constexpr bool kReverse = kMode != kFwd;
  // ring slots: the tile being reduced, D reduced tiles waiting for their carry (the oldest is
  // finished this step) and one tile in flight
  constexpr int N = D + 2;
  static_assert(N % D == 0, "the unrolled ring must map each step to a fixed deferral slot");

  __shared__ f32x2 exch[TW];
  __shared__ float tile_carry;
  __shared__ int64_t claimed;
  __shared__ int64_t first_tiles[2];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool leader = threadIdx.x == 0;
  const int vec = kReverse ? 63 - lane : lane;
  const uint32_t lane_off = (uint32_t)vec * 16u;
  const int nsub = a.seqlen / kSub;
  const int row_bytes = a.seqlen * E::kSize;
  const Rsrc st = __builtin_amdgcn_make_buffer_rsrc(
      status, (short)0, (int)((ntiles + kStatusExtraWords) * sizeof(uint64_t)), kRsrcWord3);

  // Claim results: a tile index, kBubble (no tile this step, more to come) or kDone.
  const int64_t kBubble = ntiles, kDone = ntiles + 1;
  // First claim group. Forward and reverse: blockIdx % 8, so that under round-robin dispatch
  // each XCD works through one group and a tile's predecessors were published on its own XCD.
  // Backward: blockIdx / 8 % 8, every group served by workgroups of all eight XCDs, so that
  // the groups advance at the XCDs' mean speed and end together instead of waiting for the
  // slowest XCD's group. A/B on MI355X (same buffers, alternated, median of 7, tiled calls at
  // D1024 L65536): backward B8 bf16 888.8 -> 881.1 us, fp32 1768.5 -> 1715.1, B4 431.9 ->
  // 425.8 / 918.1 -> 858.1, B2 bf16 234.1 -> 216.9, B1 fp32 238.3 -> 223.6. The forward
  // loses with it (B8 fp32 1012.4 -> 1057.6); timestamps per step phase put that loss in the
  // waits for operand data, not in the look-back, which polls as rarely either way.
  const int first_group = kMode == kBwd ? (int)((blockIdx.x / kClaimGroups) % kClaimGroups)
                                        : (int)(blockIdx.x % kClaimGroups);
  Claims<RowGroups> claims{(uint32_t)((ntiles + kCounterStride) * sizeof(uint64_t)),
                           reinterpret_cast<const uint32_t*>(status + ntiles + kCounterStride),
                           RowGroups{ntiles >> tpr_log2, tpr_log2}, first_group};
  // leader: claims in flight. Step u of the unrolled ring issues into pending[u] and resolves
  // pending[(u + D) % N], issued two steps earlier; no copies, which would wait for the atomic.
  Claim pending[N];
#pragma unroll
  for (int i = 0; i < N; ++i) pending[i] = Claim{0, 0};
  bool claims_done = false;
  if (leader) {
    const int64_t t0 = claims.next_now(st, kBubble, kDone);
    const int64_t t1 = (t0 == kDone) ? kDone : claims.next_now(st, kBubble, kDone);
    first_tiles[0] = t0;
    first_tiles[1] = t1;
    claims_done = t1 == kDone;
  }
  __syncthreads();
  // The two steps before the loop issue what a steady-state step issues, in the same order
  // (the predecessor word, here out of range; the claim two steps ahead; the refill), so that
  // the compiler's wait counts at the loop head are the steady-state ones. Otherwise the path
  // into the loop makes it wait there for the word and the claim just issued.
  uint64_t held_word = 0;
  TileSlot<kMode> ring[N];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    held_word = status_load(st, kNoOffset);
    pending[N - 2 + i] = claims.issue(st, leader && !claims_done);
    tile_setup<E, kMode, TW>(a, ring[i],
                             min(__builtin_amdgcn_readfirstlane(first_tiles[i]), ntiles), ntiles,
                             tpr_log2, w, lane_off);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 2; i < N; ++i) {  // filled at the end of the first steps
    ring[i].tile = ntiles;
    ring[i].seg = 0;
    ring[i].rr = ring[0].rr;
  }

  // what a deferred tile's finish needs from its reduce: the lane's inclusive map and the
  // wave's exclusive prefix inside the tile; and (wave 0) the predecessor words of the tile
  // finished next, loaded one step ahead
  float held_A[D], held_B[D], held_pA[D], held_pB[D];
  bool have[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    held_A[i] = 1.0f;
    held_B[i] = 0.0f;
    held_pA[i] = 1.0f;
    held_pB[i] = 0.0f;
    have[i] = false;
  }
  bool all_claimed = false;  // uniform: the leader has no more tiles to hand out

  // One step of the ring: u (a constant once the loops below are unrolled) picks the slots.
  auto step = [&](const int u) __attribute__((always_inline)) {
    TileSlot<kMode>& cur = ring[u];
    TileSlot<kMode>& fin = ring[(u + 2) % N];  // reduced D steps ago
    const int hs = u % D;  // deferral slot of `fin` (and of `cur` after this step)
    const bool cur_live = cur.tile < ntiles;  // uniform across the workgroup

    // (1) reduce the current tile (a dead tile reduces zeros and publishes nothing)
    float al[V], be[V], ysh[V];
    tile_maps<E, kMode, TW>(cur, nsub, row_bytes, w, lane, al, be, ysh);
    float A, B;
    lane_aggregate<E>(al, be, A, B);
    wave_scan(A, B);
    if (lane == 63) exch[w] = f32x2{A, B};
    lds_barrier();
    float eA = 1.0f, eB = 0.0f;
    if (lane < TW) {
      const f32x2 e = exch[lane];
      eA = e.x;
      eB = e.y;
    }
    combine_from_row<1>(eA, eB);
    if constexpr (TW > 2) combine_from_row<2>(eA, eB);
    if constexpr (TW > 4) combine_from_row<4>(eA, eB);
    if constexpr (TW > 8) combine_from_row<8>(eA, eB);
    const float cur_pA = (w > 0) ? readlane(eA, w - 1) : 1.0f;
    const float cur_pB = (w > 0) ? readlane(eB, w - 1) : 0.0f;
    const bool publisher = cur_live && w == 0 && lane == 0 && cur.tile != a.skip_publish;
    status_store(st, publisher ? (uint32_t)(cur.tile * sizeof(uint64_t)) : kNoOffset,
                 pack_map(readlane(eA, TW - 1), readlane(eB, TW - 1)));

    // (2) the finishing tile's carry from its predecessor words (loaded by wave 0 right
    // after its reduce; other waves hold zeros and compute a carry nobody uses)
    uint64_t word = held_word;
    if (__builtin_amdgcn_ballot_w64(word == kNotPublished) != 0) {
      // a predecessor was not published yet: poll (bounded). The poll is an atomic load,
      // which the compiler must re-issue every iteration (a plain buffer load would be
      // hoisted out of the loop).
      const int64_t p = fin.tile - 64 + lane;
      const bool in_row = p >= fin.tile - fin.seg;
      for (int it = 0;; ++it) {
        __builtin_amdgcn_s_sleep(1);
        word = in_row ? __hip_atomic_load(status + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : 0ull;
        if (__builtin_amdgcn_ballot_w64(word == kNotPublished) == 0) break;
        if (it >= a.spin_limit) {
          // only after an overrun: count it where the caller can see it, and make the
          // tile's outputs NaN (a NaN map poisons the composed carry) instead of plausible
          if (lane == 0) {
            __hip_atomic_fetch_add(status + ntiles, 1ull, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(&g_row_overruns, 1ull, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          }
          word = word == kNotPublished ? kPoisonMap : word;
          break;
        }
      }
    }
    float mA = __uint_as_float((uint32_t)word);
    float mB = __uint_as_float((uint32_t)(word >> 32));
    wave_scan(mA, mB);
    if (w == 0 && lane == 63) tile_carry = mB;
    if (leader) {
      const int64_t t = claims_done ? kDone : claims.resolve(pending[(u + D) % N], kBubble, kDone);
      claims_done = t == kDone;
      claimed = t;
    }
    lds_barrier();
    const int64_t claim = __builtin_amdgcn_readfirstlane(claimed);
    all_claimed = claim == kDone;
    const int64_t refill = claim < ntiles ? claim : ntiles;

    // (3) finish the oldest deferred tile (nothing is stored while the ring fills)
    {
      const float c_tile = tile_carry;
      const float c_in = fmaf(held_pA[hs], c_tile, held_pB[hs]);
      float pal[V], pbe[V], pys[V];
      const uint32_t sb = tile_maps<E, kMode, TW>(fin, nsub, row_bytes, w, lane, pal, pbe, pys);
      const float y_lane_end = fmaf(held_A[hs], c_in, held_B[hs]);
      const float y_enter = dpp<kWaveShr1>(c_in, y_lane_end);
      u32x4 o0, o1;
      finish_lane<E, kMode>(pal, pbe, pys, y_enter, o0, o1);
      const uint32_t so = have[hs] ? sb + lane_off : kNoOffset;
      bst16(fin.rr.out0, so, o0);
      if constexpr (kMode == kBwd) bst16(fin.rr.out1, so, o1);
    }
    held_A[hs] = A;
    held_B[hs] = B;
    held_pA[hs] = cur_pA;
    held_pB[hs] = cur_pB;
    have[hs] = cur_live;

    // (4) wave 0: load the predecessor words of the tile finished in the next step (reduced
    // D - 1 steps ago, or just now when D = 1) now, before the refill below: vector loads
    // complete in issue order, so waiting for these words in the next step does not wait
    // for the refill. Loading as late as that gives the workgroups that claimed the
    // predecessors, just before that tile was claimed, D steps to publish them. Lanes before
    // the row start (and all other waves) read 0: the constant map 0, the zero initial
    // state.
    {
      const TileSlot<kMode>& nxt = ring[(u + 3) % N];
      const bool nxt_live = nxt.tile < ntiles;
      const int64_t q = nxt.tile - 64 + lane;
      const bool mine = w == 0 && nxt_live && nxt.seg > 0 && q >= nxt.tile - nxt.seg;
      held_word = status_load(st, mine ? (uint32_t)(q * sizeof(uint64_t)) : kNoOffset);
    }
    // claim the refill two steps ahead now, behind the status words and ahead of the
    // operand loads, so that its return does not wait for them
    pending[u] = claims.issue(st, leader && !claims_done);
    // (5) refill the finished slot with the tile claimed two steps ago
    tile_setup<E, kMode, TW>(a, fin, refill, ntiles, tpr_log2, w, lane_off);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Whether anything is left to finish: a deferred tile or a live slot (uniform: the tile
  // indices come from one lane).
  auto busy = [&]() __attribute__((always_inline)) {
    bool b = false;
#pragma unroll
    for (int i = 0; i < D; ++i) b = b || have[i];
#pragma unroll
    for (int i = 0; i < N; ++i) b = b || ring[i].tile < ntiles;
    return b;
  };
  // Steady state: the exit test sits after whole rings. With an exit inside the unrolled
  // body, the compiler's wait counts at the loop head collapse to waiting for every load in
  // flight. Only the claim stream ends the loop, never an empty ring: while a workgroup moves
  // between used-up groups its refills can be bubbles for a whole ring, and the claims it
  // issued in the last two steps may still hold tiles; leaving then would drop those tiles
  // (never reduced, published or written), and every later tile of their rows would wait out
  // the spin limit. Once a claim comes back kDone, the claims still in flight were made to
  // the same used-up group after it, so they hold no tile.
  for (;;) {
#pragma unroll
    for (int u = 0; u < N; ++u) step(u);
    if (all_claimed) break;
  }
  if (!busy()) return;
  // Drain: no tile is claimed any more, so nothing is loaded and waiting for everything in
  // flight costs nothing; the workgroup leaves after its last finish instead of running the
  // ring to its end (each step past it waits for the previous step's stores, about 1.7 us).
  // The tile refilled last is finished N - 1 steps after the step that found no claim left,
  // so at most N - 1 steps run here. The steps are written out: a loop with an exit in its
  // body is not unrolled, and a ring slot picked at run time would put the ring in scratch.
  static_assert(N == 4, "the drain below is written out for a ring of four slots");
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

// ---------------------------------------------------------------------------------------
// Short rows: G lanes per row (seqlen = G * V), 64/G rows per wave, 4 waves per block.
// ---------------------------------------------------------------------------------------
template <class E, int kMode, int G, class Gp = GatePlain>
__global__ void __launch_bounds__(256) scan_short_rows(const Args a) {
  constexpr int V = E::V;
  constexpr bool kReverse = kMode != kFwd;
  constexpr int kRowsPerWave = 64 / G;
  constexpr int kRowsPerBlock = 4 * kRowsPerWave;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sl = lane & (G - 1);
  const int seg = lane / G;
  const int vec = kReverse ? G - 1 - sl : sl;
  const int64_t ngroups = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;

  for (int64_t grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {
    const int64_t wave_row0 = grp * kRowsPerBlock + (int64_t)wave * kRowsPerWave;
    if (wave_row0 >= a.rows) break;  // wave-uniform
    const int64_t row = wave_row0 + seg;
    const bool valid = row < a.rows;
    const int64_t base = valid ? row_offset(a, row) : 0;

    Slot<kMode> s;
    if (valid) {
      const int64_t e = base + (int64_t)vec * V;
      s.v[0] = ld16(a.in0, e, E::kSize);
      s.v[1] = ld16(a.in1, e, E::kSize);
      if constexpr (kMode == kBwd) s.v[2] = ld16(a.in2, e, E::kSize);
    } else {
#pragma unroll
      for (int i = 0; i < (kMode == kBwd ? 3 : 2); ++i) s.v[i] = u32x4{0u, 0u, 0u, 0u};
    }
    float rate = 0.0f, rate_sum = 0.0f;
    if constexpr (Gp::kFused) rate = valid ? a.rate[row % a.dim] : 0.0f;
    float al[V], be[V], ysh[V];
    typename Gp::template Aux<V> aux;
    make_maps<E, kMode, Gp>(s, al, be, ysh, 1.0f, 0.0f, sl == 0, sl == G - 1, rate, &aux);
    if (kMode != kBwd && sl == 0) al[0] = 1.0f;
    float A, B;
    lane_aggregate<E>(al, be, A, B);
    segment_scan<G>(A, B, sl);
    float y_enter = dpp<kWaveShr1>(0.0f, B);
    y_enter = (sl == 0) ? 0.0f : y_enter;
    u32x4 o0, o1;
    finish_lane<E, kMode, Gp>(al, be, ysh, y_enter, o0, o1, &aux, &rate_sum);
    if (valid) {
      st16(a.out0, base + (int64_t)vec * V, E::kSize, o0);
      if constexpr (kMode == kBwd) st16(a.out1, base + (int64_t)vec * V, E::kSize, o1);
    }
    if constexpr (Gp::kFused && kMode == kBwd) {
      const float tot = segment_sum<G>(rate_sum, sl);  // the row's last lane holds its sum
      if (valid && sl == G - 1 && a.grad_rate_rows != nullptr) a.grad_rate_rows[row] = tot;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------
// Process-wide tuning and test hooks (fpscan_set_launch_override, fpscan_set_tiling,
// fpscan_set_lookback_test_hook); every setting computes the same recurrence.
std::atomic<int> g_override_w{0};
std::atomic<int> g_override_u{0};
std::atomic<int> g_tiling{0};  // 0 automatic, 1 row streaming only, 2 tiled when possible
std::atomic<int64_t> g_hook_skip_publish{-1};
std::atomic<int> g_hook_spin_limit{0};  // 0: kSpinLimit

// Tiled path geometry: TW sub-chunks per tile, at most 64 tiles per row (one look-back window)
constexpr int kTileWaves = 16;
// Steps between a tile's reduce and its finish: a workgroup a step or two behind its
// neighbours then rarely makes them wait (measured at B8 D1024 L65536: see the kernel notes).
constexpr int kTileDefer = 2;
// Below this many bytes per tensor the row-streaming kernels win: a tiled launch costs about
// 10-15 us more than its streaming time (the status clear, start-up claims, filling and
// draining the four-tile pipeline), which dozens of tiles per workgroup amortise. Measured on
// MI355X: at 128 MiB per tensor streaming wins (fp32 B2 D256 L65536 forward 72 us against
// 87), at 512 MiB tiling wins by 6 % (fp32 B8 D1024 L16384) and at 1-2 GiB by 8-10 %.
// Every shape quoted in these notes can be rerun with each path forced:
// `python bench.py --workload rows --dtype D --shape B,D,L --tiling 1|2`.
constexpr int64_t kTiledMinBytes = 512ll << 20;
// The fused backward moves 5 tensors per tile instead of 3, so the same fixed cost is a smaller
// share, and the streaming backward slows down on long rows (one workgroup per row streaming
// 64 KiB or more per tensor). There tiling wins from 256 MiB per tensor. Measured on MI355X
// with the backward's claim groups served by every XCD (same buffers, streaming and tiled
// forced alternately, median of 5, us): 128 KiB rows bf16 B2 D1024 L65536 216-221 against
// 238-240, fp32 B2 D1024 L32768 220.5 against 239.0; 64 KiB rows bf16 (4, 1024, 32768)
// 216.1-216.5 against 229.3-231.0, (8, 512, 32768) 227.8 against 232.7, (2, 2048, 32768)
// 215.1 against 233.0, fp32 (4, 1024, 16384) and (8, 512, 16384) even (221-222 against
// 223); 32 KiB rows still stream faster (bf16 (8, 1024, 16384) 219.5 against 228.3, fp32
// (8, 1024, 8192) 215.9 against 223.9), and at 128 MiB the two paths are within 5 % either way.
constexpr int64_t kTiledMinBytesBwdLongRows = 256ll << 20;
constexpr int64_t kLongRowBytes = 64ll << 10;
// Rows of one tile (16 sub-chunks) stream as 8-wave rows, which keep up with the tiles to
// about 1 GiB per tensor: at 512 MiB streaming measured 3-8 % faster (bf16 32768 rows of L8192
// forward / backward 255 / 420 us against 261-278 / 438; fp32 32768 rows of L4096 256 / 428
// against 267 / 459), at 1 GiB the tiles 2.5 % faster forward (509 against 522 us). The
// 2-byte backward on such rows streams at every size: with the backward's claim groups served
// by every XCD (same buffers, alternated, median of 5) bf16 L8192 streamed 854.5 against 872.1
// us at 1 GiB and 1745.9 against 1809.5 at 2 GiB, while the fp32 backward on L4096 rows tiled
// 842.8 against 847.2 and 1716.0 against 1772.8.
constexpr int64_t kTiledMinBytesOneTileRows = 1ll << 30;

struct TilePlan {
  bool use;
  int tpr;         // tiles per row
  int64_t ntiles;  // rows * tpr
  size_t bytes;    // workspace: one status word per tile + overrun and tile counters
};

// The forward/reverse scan and the backward use the same tile geometry; only the automatic
// size threshold differs (`bwd`).
TilePlan plan_tiles(int64_t rows, int64_t seqlen, int size, int tiling, bool bwd) {
  TilePlan t{false, 0, 0, 0};
  const int64_t sub = 64 * (16 / size);
  const int64_t nsub = seqlen / sub;
  if (tiling == 1 || nsub < kTileWaves) return t;
  t.tpr = (int)(nsub / kTileWaves);
  if (t.tpr > 64) return t;
  if (tiling == 0 && t.tpr == 1 && bwd && size == 2) return t;  // streams at every size
  const int64_t min_bytes =
      t.tpr == 1 ? kTiledMinBytesOneTileRows
                 : (bwd && seqlen * size >= kLongRowBytes ? kTiledMinBytesBwdLongRows
                                                          : kTiledMinBytes);
  if (tiling == 0 && rows * seqlen * size < min_bytes) return t;
  t.ntiles = rows * t.tpr;
  if ((t.ntiles + kStatusExtraWords) * (int64_t)sizeof(uint64_t) > INT32_MAX) return t;
  t.use = true;
  t.bytes = (size_t)(t.ntiles + kStatusExtraWords) * sizeof(uint64_t);
  return t;
}

constexpr int kMaxDevices = 64;
constexpr int kTiledKernels = 9;  // 3 element types x 3 modes
std::atomic<int> g_resident_blocks[kMaxDevices][kTiledKernels];

// Workgroups of `kernel` that fit on the current device at once (CUs x blocks per CU); 0 if
// the device cannot be queried. Cached per device and kernel.
int resident_blocks(const void* kernel, int slot, int threads) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kMaxDevices) {
    const int cached = g_resident_blocks[dev][slot].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
      cus <= 0 || per_cu <= 0)
    return 0;
  const int n = cus * per_cu;
  if (dev < kMaxDevices) g_resident_blocks[dev][slot].store(n, std::memory_order_relaxed);
  return n;
}

int launch(const void* kernel, int64_t groups, int threads, const Args& a, hipStream_t stream) {
  // One group per block; very large problems loop inside the kernel (grid-stride) so the
  // dispatch stays below 2^31 work-items.
  const int64_t max_blocks = ((int64_t)1 << 31) / threads;
  const unsigned int blocks = (unsigned int)(groups < max_blocks ? groups : max_blocks);
  Args copy = a;
  void* params[] = {&copy};
  const hipError_t err =
      hipLaunchKernel(kernel, dim3(blocks), dim3(threads), params, 0, stream);
  return err == hipSuccess ? FPSCAN_OK : FPSCAN_ERR_LAUNCH;
}

template <class E, int kMode, int W, class Gp>
const void* long_kernel(int u) {
  if constexpr (W == 1) {
    if (u >= 4) return reinterpret_cast<const void*>(&scan_long_rows<E, kMode, W, 4, Gp>);
  }
  // W = 16 keeps three sub-chunks in flight per wave: measured 2-5 % faster than two on
  // rows of 4 or more rounds (bf16 B8 D1024 L65536 forward 552 us against 568, backward 928
  // against 972). The forward and reverse keep four on rows of 8 rounds or more (the
  // caller's choice of u): 1-3 % faster than three (fp32 B2 D256 L32768 forward 38.4 -> 37.4
  // us, fused-gate bf16 B8 D1024 L65536 556.4 -> 547.6), within 64 VGPRs; the backward at
  // four (79-97 VGPRs) measured 0.5-1 % slower than three. Other W keep at most two: their
  // waves already multiply the bytes in flight. So does the fused-gate backward: at three (126
  // VGPRs in bf16, no spills, the same one workgroup per CU) it measured within 0.5 % of two
  // in bf16 and fp32 at (8, 1024, 65536), (2, 512, 65536) and (4, 256, 32768).
  if constexpr (W == 16 && kMode != kBwd) {
    if (u >= 4) return reinterpret_cast<const void*>(&scan_long_rows<E, kMode, W, 4, Gp>);
  }
  if constexpr (W == 16 && (!Gp::kFused || kMode != kBwd)) {
    if (u >= 3) return reinterpret_cast<const void*>(&scan_long_rows<E, kMode, W, 3, Gp>);
  }
  if (u >= 2) return reinterpret_cast<const void*>(&scan_long_rows<E, kMode, W, 2, Gp>);
  return reinterpret_cast<const void*>(&scan_long_rows<E, kMode, W, 1, Gp>);
}

template <class E, int kMode, class Gp>
const void* long_kernel(int w, int u) {
  switch (w) {
    case 1: return long_kernel<E, kMode, 1, Gp>(u);
    case 2: return long_kernel<E, kMode, 2, Gp>(u);
    case 4: return long_kernel<E, kMode, 4, Gp>(u);
    case 8: return long_kernel<E, kMode, 8, Gp>(u);
    default: return long_kernel<E, kMode, 16, Gp>(u);
  }
}

template <class E, int kMode, class Gp>
const void* short_kernel(int g) {
  switch (g) {
    case 4: return reinterpret_cast<const void*>(&scan_short_rows<E, kMode, 4, Gp>);
    case 8: return reinterpret_cast<const void*>(&scan_short_rows<E, kMode, 8, Gp>);
    case 16: return reinterpret_cast<const void*>(&scan_short_rows<E, kMode, 16, Gp>);
    default: return reinterpret_cast<const void*>(&scan_short_rows<E, kMode, 32, Gp>);
  }
}

// Chooses the launch for one problem. Rows are independent; long rows are owned by W waves
// (W = 16 when the row has at least 16 sub-chunks) with U sub-chunks in flight per wave. The
// ring depths are the deepest that keep every variant within 64 VGPRs (8 waves per SIMD).
// Tiled launch: clear the status words and counters, then the persistent grid, one workgroup
// per resident slot (more would only queue behind them; fewer is also correct, since tiles
// are claimed dynamically). Returns -1 when the occupancy query fails, so that the caller
// streams rows instead.
template <class E, int kMode>
int run_tiled(const Args& a, const TilePlan& plan, void* workspace, hipStream_t stream, int slot) {
  const void* kernel = reinterpret_cast<const void*>(&scan_tiles<E, kMode, kTileWaves, kTileDefer>);
  const int threads = 64 * kTileWaves;
  const int resident = resident_blocks(kernel, slot, threads);
  if (resident <= 0) return -1;
  uint64_t* status = static_cast<uint64_t*>(workspace);
  int64_t ntiles = plan.ntiles;
  const int64_t nwords = ntiles + kStatusExtraWords;
  const int64_t clear_blocks = (nwords + 255) / 256 < 1024 ? (nwords + 255) / 256 : 1024;
  void* cargs[] = {&status, &ntiles};
  if (hipLaunchKernel(reinterpret_cast<const void*>(&clear_status), dim3((unsigned)clear_blocks),
                      dim3(256), cargs, 0, stream) != hipSuccess)
    return FPSCAN_ERR_LAUNCH;
  const int64_t grid = plan.ntiles < resident ? plan.ntiles : resident;
  Args copy = a;
  copy.skip_publish = g_hook_skip_publish.load(std::memory_order_relaxed);
  const int spin = g_hook_spin_limit.load(std::memory_order_relaxed);
  copy.spin_limit = spin > 0 ? spin : kSpinLimit;
  int tpr_log2 = 0;
  while ((1 << tpr_log2) < plan.tpr) ++tpr_log2;
  void* kargs[] = {&copy, &status, &tpr_log2, &ntiles};
  const hipError_t err =
      hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), kargs, 0, stream);
  return err == hipSuccess ? FPSCAN_OK : FPSCAN_ERR_LAUNCH;
}

// Fused-gate calls (Gp = GateSoftplus) always stream rows: the tiled kernel rebuilds a tile's
// maps at its deferred finish, which would evaluate the gate transform twice.
template <class E, int kMode, class Gp = GatePlain>
int run(const Args& a, void* workspace, size_t ws_bytes, hipStream_t stream) {
  constexpr int V = E::V;
  constexpr int kSub = 64 * V;
  const int L = a.seqlen;
  const TilePlan plan =
      plan_tiles(a.rows, L, E::kSize, g_tiling.load(std::memory_order_relaxed), kMode == kBwd);
  if (!Gp::kFused && plan.use && workspace != nullptr && ws_bytes >= plan.bytes) {
    const int st = run_tiled<E, kMode>(a, plan, workspace, stream,
                                       E::kSlot * 3 + kMode);
    if (st >= 0) return st;
  }
  if (L < kSub) {
    const int g = L / V;
    const int64_t rows_per_block = 4 * (64 / g);
    return launch(short_kernel<E, kMode, Gp>(g), (a.rows + rows_per_block - 1) / rows_per_block,
                  256, a, stream);
  }
  const int nsub = L / kSub;
  // Up to 16 waves share a row: each round then touches W KiB of each tensor contiguously
  // and 16x fewer rows are in flight than with one wave per row, which is what the HBM
  // controllers and address translation reward. Few-row problems also fill the device this
  // way (rows * 16 waves).
  int w = nsub < 16 ? nsub : 16;
  // 8 waves per row where 16 measured slower: rows of 16-64 sub-chunks (one to four 16-wave
  // rounds) in tensors of 16-64 MiB; from 16 MiB up, rows of 16 sub-chunks in the forward and
  // reverse, and rows of 16-32 sub-chunks in the fused-gate backward. Each wave then keeps two
  // sub-chunks in flight over 2-8 rounds instead of filling and draining its ring within one
  // to four. Measured on MI355X (p50 of one call, same buffers, 16 waves -> 8): at 16-64 MiB
  // forward 1-12 % faster (fp32 512 rows of L16384 20.4 -> 18.8 us, bf16 2048 rows of L8192
  // 21.2 -> 19.0) and backward 2-13 % (the fp32 shape 31.8 -> 29.9, bf16 1024 rows of L8192
  // 18.8 -> 17.6); forward on rows of 16 sub-chunks at 128-256 MiB 3-6 % (bf16 8192 rows of
  // L8192 68.1 -> 64.8); fused-gate backward on rows of 16-32 sub-chunks at 16-256 MiB 11-25 %
  // (bf16 8192 rows of L8192 152.4 -> 117.4). Elsewhere 8 waves measured slower (2-9 % on
  // rows of 2-8 rounds at 128-256 MiB, up to 5 % below 16 MiB, where a call takes about 7 us)
  // or even (the plain backward on rows of 16 at 128-256 MiB).
  const int64_t kib = a.rows * nsub;  // tensor size: a sub-chunk is 1 KiB
  const bool from16 = kib >= (16 << 10);
  const bool eight = (nsub >= 16 && nsub <= 64 && from16 && kib <= (64 << 10)) ||
                     (kMode != kBwd && nsub == 16 && from16) ||
                     (Gp::kFused && kMode == kBwd && nsub >= 16 && nsub <= 32 && from16);
  if (eight) w = 8;
  int u_max = (w == 1 && kMode != kBwd) ? 4
              : (w == 16 && kMode != kBwd && nsub >= 8 * 16) ? 4
              : (w == 16 && (!Gp::kFused || kMode != kBwd) ? 3 : 2);
  const int ow = g_override_w.load(std::memory_order_relaxed);
  const int ou = g_override_u.load(std::memory_order_relaxed);
  if (ow > 0) w = ow <= nsub ? ow : nsub;
  if (ou > 0) u_max = ou;
  const int nrounds = nsub / w;
  const int u = u_max < nrounds ? u_max : nrounds;
  if (w == 1) {
    // Rows of one sub-chunk, from 32 MiB per tensor (the backward from 64 MiB): one row per
    // 64-thread block, so that every wave slot that frees up takes the next row at once.
    // Measured on MI355X against 4 rows per 256-thread block (p50 of one call, same buffers,
    // outputs bit for bit equal): fp32 262144 rows of L256 (config 5) forward 127.7-132.1 ->
    // 119.6-120.9 us, backward 224.1-233.5 -> 208.3-209.8; forward 4-10 % faster from 32 MiB,
    // backward 3-10 % from 128 MiB, even at 64 MiB and 1-3 % slower at 32 MiB; at 8 MiB
    // 7-10 % slower.
    // The fused-gate kernels gain as much (fp32 config 5 shape forward 125.6 -> 121.6 us,
    // backward 224.4 -> 208.7; bf16 (64, 4096, 512) 133.3 / 223.9 -> 121.6 / 213.8).
    if (nsub == 1 && ow == 0 && ou == 0 && a.rows >= (kMode == kBwd ? 64 << 10 : 32 << 10))
      return launch(reinterpret_cast<const void*>(&scan_long_rows<E, kMode, 1, 1, Gp, 1>),
                    a.rows, 64, a, stream);
    return launch(long_kernel<E, kMode, Gp>(1, u), (a.rows + 3) / 4, 256, a, stream);
  }
  return launch(long_kernel<E, kMode, Gp>(w, u), a.rows, 64 * w, a, stream);
}

template <int kMode, class Gp = GatePlain>
int dispatch(int dtype, const Args& a, void* ws, size_t ws_bytes, hipStream_t stream) {
  switch (dtype) {
    case FPSCAN_DTYPE_F32: return run<F32, kMode, Gp>(a, ws, ws_bytes, stream);
    case FPSCAN_DTYPE_F16: return run<F16, kMode, Gp>(a, ws, ws_bytes, stream);
    case FPSCAN_DTYPE_BF16: return run<BF16, kMode, Gp>(a, ws, ws_bytes, stream);
    default: return FPSCAN_ERR_DTYPE;
  }
}

int itemsize(int dtype) {
  switch (dtype) {
    case FPSCAN_DTYPE_F32: return 4;
    case FPSCAN_DTYPE_F16: return 2;
    case FPSCAN_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Scratch of fpscan_scan_fwd_noalloc: the tiled path's status words and counters for up to
// kScratchTiles tiles (2 MiB + 1152 bytes per device, held until the process ends). Host code
// never uses the name as an address: each device's copy is found with hipGetSymbolAddress.
constexpr int64_t kScratchTiles = 1ll << 18;
constexpr int64_t kScratchWords = kScratchTiles + kStatusExtraWords;
static __device__ __align__(256) uint64_t scratch[kScratchWords];
std::atomic<uintptr_t> g_scratch_ptr[kMaxDevices];

// This device's copy of `scratch`, looked up once per device with that device current.
int scratch_on_current_device(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FPSCAN_ERR_DEVICE;
  uintptr_t p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == 0) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || q == nullptr)
      return FPSCAN_ERR_DEVICE;
    p = reinterpret_cast<uintptr_t>(q);
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *ptr = reinterpret_cast<void*>(p);
  return FPSCAN_OK;
}

// Shared argument validation. Mirrors the reference's checks where it has them
// (seqlen table full_scan.cu:207-233, dtype full_scan.cu:245-256) and adds the ones it
// lacks (shape, alignment, null pointers).
int validate(int64_t batch, int64_t dim, int64_t seqlen, int64_t stride_b, int64_t stride_d,
             int dtype, Args* a) {
  if (seqlen < 32 || seqlen > 65536 || (seqlen & (seqlen - 1)) != 0) return FPSCAN_ERR_SEQLEN;
  const int size = itemsize(dtype);
  if (size == 0) return FPSCAN_ERR_DTYPE;
  if (batch < 0 || dim < 0 || stride_b < 0 || stride_d < 0) return FPSCAN_ERR_SHAPE;
  // the row count and the element span (batch-1)*stride_b + (dim-1)*stride_d + seqlen, with
  // every product and sum checked, so that no size the caller passes can wrap around; the
  // span's bytes must stay below 2^48 (256 TiB, far above any device memory)
  int64_t rows = 0, over_b = 0, over_d = 0, span = 0;
  if (__builtin_mul_overflow(batch, dim, &rows) ||
      __builtin_mul_overflow(batch > 0 ? batch - 1 : 0, stride_b, &over_b) ||
      __builtin_mul_overflow(dim > 0 ? dim - 1 : 0, stride_d, &over_d) ||
      __builtin_add_overflow(over_b, over_d, &span) ||
      __builtin_add_overflow(span, seqlen, &span) || span > ((int64_t)1 << 48) / size)
    return FPSCAN_ERR_SHAPE;
  if (dim > 1 && stride_d < seqlen) return FPSCAN_ERR_SHAPE;
  if (batch > 1 && dim > 0 && stride_b < over_d + seqlen) return FPSCAN_ERR_SHAPE;
  // strides of size-1 dimensions are never used
  if (batch > 1 && ((stride_b * size) & 15) != 0) return FPSCAN_ERR_ALIGN;
  if (dim > 1 && ((stride_d * size) & 15) != 0) return FPSCAN_ERR_ALIGN;
  a->rows = rows;
  a->dim = dim > 0 ? dim : 1;
  a->stride_b = stride_b;
  a->stride_d = stride_d;
  a->seqlen = (int32_t)seqlen;
  // row r starts at r * seqlen exactly when both strides are the packed ones
  a->contiguous = (dim <= 1 || stride_d == seqlen) && (batch <= 1 || stride_b == dim * seqlen);
  return FPSCAN_OK;
}

}  // namespace

// Path selection set by fpscan_set_tiling and the look-back test hook, read by the
// channel-last and dimwise launchers as well; their counters of given-up waits.
namespace fpscan_detail {
int tiling_mode() { return g_tiling.load(std::memory_order_relaxed); }
int64_t hook_skip_publish() { return g_hook_skip_publish.load(std::memory_order_relaxed); }
int hook_spin_limit() {
  const int spin = g_hook_spin_limit.load(std::memory_order_relaxed);
  return spin > 0 ? spin : kSpinLimit;
}
int cl_overruns(unsigned long long* count);  // fpscan_scan_cl.hip
int dw_overruns(unsigned long long* count);  // fpscan_dimwise.hip
}  // namespace fpscan_detail

namespace fpscan_detail {
// The row kernel's counter of given-up waits on the current device (a synchronous copy).
int row_overruns(unsigned long long* count) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_row_overruns)) != hipSuccess || p == nullptr)
    return FPSCAN_ERR_DEVICE;
  if (hipMemcpy(count, p, sizeof(*count), hipMemcpyDeviceToHost) != hipSuccess)
    return FPSCAN_ERR_DEVICE;
  return FPSCAN_OK;
}
}  // namespace fpscan_detail

extern "C" {

int fpscan_scan_fwd(const void* gates, const void* tokens, void* out, int64_t batch, int64_t dim,
                    int64_t seqlen, int64_t stride_b, int64_t stride_d, int dtype, int reverse,
                    void* workspace, size_t workspace_bytes, void* stream) {
  Args a{};
  const int st = validate(batch, dim, seqlen, stride_b, stride_d, dtype, &a);
  if (st != FPSCAN_OK) return st;
  if (a.rows == 0) return FPSCAN_OK;
  if (!gates || !tokens || !out) return FPSCAN_ERR_NULL;
  if (!aligned16(gates) || !aligned16(tokens) || !aligned16(out)) return FPSCAN_ERR_ALIGN;
  a.in0 = gates;
  a.in1 = tokens;
  a.out0 = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return reverse ? dispatch<kRev>(dtype, a, workspace, workspace_bytes, s)
                 : dispatch<kFwd>(dtype, a, workspace, workspace_bytes, s);
}

int fpscan_scan_bwd(const void* gates, const void* out, const void* grad_out, void* grad_gates,
                    void* grad_tokens, int64_t batch, int64_t dim, int64_t seqlen,
                    int64_t stride_b, int64_t stride_d, int dtype, void* workspace,
                    size_t workspace_bytes, void* stream) {
  Args a{};
  const int st = validate(batch, dim, seqlen, stride_b, stride_d, dtype, &a);
  if (st != FPSCAN_OK) return st;
  if (a.rows == 0) return FPSCAN_OK;
  if (!gates || !out || !grad_out || !grad_gates || !grad_tokens) return FPSCAN_ERR_NULL;
  if (!aligned16(gates) || !aligned16(out) || !aligned16(grad_out) || !aligned16(grad_gates) ||
      !aligned16(grad_tokens))
    return FPSCAN_ERR_ALIGN;
  a.in0 = gates;
  a.in1 = grad_out;
  a.in2 = out;
  a.out0 = grad_tokens;
  a.out1 = grad_gates;
  return dispatch<kBwd>(dtype, a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int fpscan_scan_fwd_noalloc(const void* gates, const void* tokens, void* out, int64_t batch,
                            int64_t dim, int64_t seqlen, int64_t stride_b, int64_t stride_d,
                            int dtype, int reverse, void* stream) {
  Args a{};
  const int st = validate(batch, dim, seqlen, stride_b, stride_d, dtype, &a);
  if (st != FPSCAN_OK) return st;
  if (a.rows == 0) return FPSCAN_OK;
  if (!gates || !tokens || !out) return FPSCAN_ERR_NULL;
  if (!aligned16(gates) || !aligned16(tokens) || !aligned16(out)) return FPSCAN_ERR_ALIGN;
  const TilePlan plan = plan_tiles(a.rows, seqlen, itemsize(dtype),
                                   g_tiling.load(std::memory_order_relaxed), false);
  if (plan.use && plan.bytes > sizeof(scratch)) return FPSCAN_ERR_SCRATCH;
  void* ws = nullptr;
  const int sst = scratch_on_current_device(&ws);
  if (sst != FPSCAN_OK) return sst;
  a.in0 = gates;
  a.in1 = tokens;
  a.out0 = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return reverse ? dispatch<kRev>(dtype, a, ws, sizeof(scratch), s)
                 : dispatch<kFwd>(dtype, a, ws, sizeof(scratch), s);
}

int fpscan_scan_fwd_softplus(const void* z, const float* rate, const void* tokens, void* out,
                             int64_t batch, int64_t dim, int64_t seqlen, int64_t stride_b,
                             int64_t stride_d, int dtype, int reverse, void* stream) {
  Args a{};
  const int st = validate(batch, dim, seqlen, stride_b, stride_d, dtype, &a);
  if (st != FPSCAN_OK) return st;
  if (a.rows == 0) return FPSCAN_OK;
  if (!z || !rate || !tokens || !out) return FPSCAN_ERR_NULL;
  if (!aligned16(z) || !aligned16(tokens) || !aligned16(out) ||
      (reinterpret_cast<uintptr_t>(rate) & 3u) != 0)
    return FPSCAN_ERR_ALIGN;
  a.in0 = z;
  a.in1 = tokens;
  a.out0 = out;
  a.rate = rate;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return reverse ? dispatch<kRev, GateSoftplus>(dtype, a, nullptr, 0, s)
                 : dispatch<kFwd, GateSoftplus>(dtype, a, nullptr, 0, s);
}

int fpscan_scan_bwd_softplus(const void* z, const float* rate, const void* out,
                             const void* grad_out, void* grad_z, void* grad_tokens,
                             float* grad_rate_rows, int64_t batch, int64_t dim, int64_t seqlen,
                             int64_t stride_b, int64_t stride_d, int dtype, void* stream) {
  Args a{};
  const int st = validate(batch, dim, seqlen, stride_b, stride_d, dtype, &a);
  if (st != FPSCAN_OK) return st;
  if (a.rows == 0) return FPSCAN_OK;
  if (!z || !rate || !out || !grad_out || !grad_z || !grad_tokens) return FPSCAN_ERR_NULL;
  if (!aligned16(z) || !aligned16(out) || !aligned16(grad_out) || !aligned16(grad_z) ||
      !aligned16(grad_tokens) || (reinterpret_cast<uintptr_t>(rate) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(grad_rate_rows) & 3u) != 0)
    return FPSCAN_ERR_ALIGN;
  a.in0 = z;
  a.in1 = grad_out;
  a.in2 = out;
  a.out0 = grad_tokens;
  a.out1 = grad_z;
  a.rate = rate;
  a.grad_rate_rows = grad_rate_rows;
  return dispatch<kBwd, GateSoftplus>(dtype, a, nullptr, 0, static_cast<hipStream_t>(stream));
}

size_t fpscan_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int dtype, int op) {
  const int size = itemsize(dtype);
  if (size == 0 || batch <= 0 || dim <= 0 || seqlen < 32 || seqlen > 65536 ||
      (seqlen & (seqlen - 1)) != 0)
    return 0;
  if (op != FPSCAN_OP_FWD && op != FPSCAN_OP_BWD) return 0;
  int64_t rows = 0, elems = 0;
  if (__builtin_mul_overflow(batch, dim, &rows) || __builtin_mul_overflow(rows, seqlen, &elems) ||
      elems > ((int64_t)1 << 48) / size)
    return 0;  // no call of this size passes validation
  const TilePlan plan = plan_tiles(rows, seqlen, size,
                                   g_tiling.load(std::memory_order_relaxed), op == FPSCAN_OP_BWD);
  return plan.use ? plan.bytes : 0;
}

const char* fpscan_strerror(int status) {
  switch (status) {
    case FPSCAN_OK: return "success";
    case FPSCAN_ERR_SEQLEN: return "seqlen must be a power of 2, >= 32, <= 65536";
    case FPSCAN_ERR_DTYPE: return "Unsupported tensor dtype: expecting bfloat16, float16 or float32";
    case FPSCAN_ERR_SHAPE:
      return "invalid shape or strides: rows must not overlap and a tensor must span less than "
             "2^48 bytes";
    case FPSCAN_ERR_ALIGN: return "data pointers and row strides must be 16-byte aligned";
    case FPSCAN_ERR_NULL: return "null data pointer";
    case FPSCAN_ERR_WORKSPACE: return "workspace too small";
    case FPSCAN_ERR_LAUNCH: return "HIP kernel launch failed";
    case FPSCAN_ERR_DEVICE: return "could not query the current HIP device";
    case FPSCAN_ERR_SCRATCH:
      return "problem needs more tile-status scratch than fpscan_scan_fwd_noalloc holds "
             "(262144 tiles)";
    default: return "unknown fpscan status";
  }
}

int fpscan_lookback_overruns(unsigned long long* count) {
  if (count == nullptr) return FPSCAN_ERR_NULL;
  if (hipDeviceSynchronize() != hipSuccess) return FPSCAN_ERR_DEVICE;
  unsigned long long rows = 0, cl = 0, dw = 0;
  int st = fpscan_detail::row_overruns(&rows);
  if (st != FPSCAN_OK) return st;
  st = fpscan_detail::cl_overruns(&cl);
  if (st != FPSCAN_OK) return st;
  st = fpscan_detail::dw_overruns(&dw);
  if (st != FPSCAN_OK) return st;
  *count = rows + cl + dw;
  return FPSCAN_OK;
}

int fpscan_set_lookback_test_hook(int64_t unpublished_tile, int spin_limit) {
  if (spin_limit < 0) return FPSCAN_ERR_SHAPE;
  g_hook_skip_publish.store(unpublished_tile < 0 ? -1 : unpublished_tile,
                            std::memory_order_relaxed);
  g_hook_spin_limit.store(spin_limit, std::memory_order_relaxed);
  return FPSCAN_OK;
}

int fpscan_abi_version(void) { return FPSCAN_ABI_VERSION; }

int fpscan_set_tiling(int mode) {
  if (mode < 0 || mode > 2) return FPSCAN_ERR_SHAPE;
  g_tiling.store(mode, std::memory_order_relaxed);
  return FPSCAN_OK;
}

int fpscan_set_launch_override(int waves_per_row, int ring_depth) {
  const bool w_ok = waves_per_row == 0 || waves_per_row == 1 || waves_per_row == 2 ||
                    waves_per_row == 4 || waves_per_row == 8 || waves_per_row == 16;
  const bool u_ok = ring_depth >= 0 && ring_depth <= 4;
  if (!w_ok || !u_ok) return FPSCAN_ERR_SHAPE;
  g_override_w.store(waves_per_row, std::memory_order_relaxed);
  g_override_u.store(ring_depth, std::memory_order_relaxed);
  return FPSCAN_OK;
}

}  // extern "C"

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
//   When batch x strips alone cannot fill the device, the time axis is cut into segments and
//   three launches run: per-segment per-column aggregates (A, B) into the workspace, a carry
//   pass over the segments of each column, then the segments again with their carry-in.
//   That moves 5 N s bytes for the forward scan instead of 3 N s, still without transposes.
// All arithmetic is fp32; half types are widened exactly on load and rounded to nearest even
// once on store.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fpscan_hip.h"
#include "scan_common.h"

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
};

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
__global__ void __launch_bounds__(256) scan_cl(const ClArgs a) {
  constexpr int V = E::V;
  constexpr bool kReverse = kMode != kFwd;

  const int lane = threadIdx.x & 63;
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
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
// Host side
// ---------------------------------------------------------------------------------------
constexpr int kClWaves = 4;  // independent waves per block
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

template <class E, int kMode>
int run_cl(ClArgs a, void* workspace, size_t ws_bytes, hipStream_t stream) {
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
  if (stride_t < dim || stride_b < (seqlen - 1) * stride_t + dim) return FPSCAN_ERR_SHAPE;
  if (stride_t * size > (INT32_MAX / 3)) return FPSCAN_ERR_SHAPE;
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
  return plan_cl(batch, seqlen, dim, stride_t, size).bytes;
}

}  // extern "C"

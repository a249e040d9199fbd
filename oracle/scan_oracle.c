/*
 * scan_oracle.c -- TEST INFRASTRUCTURE ONLY. The CPU checker for the HIP scan; nothing on
 * the product path (fpscan_amd/) may link, load or call it. Only tests/, the smoke check of
 * __graft_entry__ and the cpu_baseline leg of bench.py use it.
 *
 * Restates saeeddhqan/fpscan's algorithm for the path y[t] = gates[t]*y[t-1] + tokens[t]:
 *
 *   oracle_scan_f64      eval/baselines.py:20-37 (sequential_scan): float64 serial loop,
 *                        zero initial state, reverse = flip / scan / flip.
 *   oracle_scan_bwd_f64  the gradients PScan.backward computes (fpscan/ops.py:69-83):
 *                        grad_tokens = reverse scan of grad_out over gates shifted left by one
 *                        (gates[L] := 1), grad_gates[t] = grad_tokens[t] * y[t-1] (y[-1] := 0),
 *                        in float64.
 *   oracle_refkernel_f32 the reference CUDA kernel's fp32 arithmetic, operation by operation
 *                        (csrc/full_scan/full_scan.cu:50-177, tile table :207-233, with nvcc's
 *                        default a*b+c -> fma contraction): used to state the reference
 *                        kernel's own error on the same inputs, not as the pass criterion.
 *
 * Rows are contiguous runs of L values. Rows are independent and are split over OpenMP
 * threads when the library is built with -fopenmp.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oracle_scan_f64(const double* g, const double* x, double* y, int64_t rows, int64_t L,
                     int reverse) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const double* gr = g + r * L;
    const double* xr = x + r * L;
    double* yr = y + r * L;
    double acc = 0.0;
    if (!reverse) {
      for (int64_t t = 0; t < L; ++t) {
        acc = gr[t] * acc + xr[t];
        yr[t] = acc;
      }
    } else {
      for (int64_t t = L - 1; t >= 0; --t) {
        acc = gr[t] * acc + xr[t];
        yr[t] = acc;
      }
    }
  }
}

void oracle_scan_bwd_f64(const double* g, const double* y, const double* go, double* gg,
                         double* gx, int64_t rows, int64_t L) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const double* gr = g + r * L;
    const double* yr = y + r * L;
    const double* gor = go + r * L;
    double* ggr = gg + r * L;
    double* gxr = gx + r * L;
    double acc = 0.0;
    for (int64_t t = L - 1; t >= 0; --t) {
      const double shifted_gate = (t + 1 < L) ? gr[t + 1] : 1.0;
      acc = shifted_gate * acc + gor[t];
      gxr[t] = acc;
      ggr[t] = acc * ((t > 0) ? yr[t - 1] : 0.0);
    }
  }
}

/* The reference's compile-time tile table (full_scan.cu:207-233): elements per thread S,
 * chunks per row C; threads per block = L / S / C, warps of 32. Returns 0 for a seqlen the
 * reference rejects. */
static int ref_tiles(int64_t L, int* S, int* C) {
  switch (L) {
    case 32: *S = 1; *C = 1; return 1;
    case 64: *S = 2; *C = 1; return 1;
    case 128: *S = 1; *C = 1; return 1;
    case 256: *S = 1; *C = 1; return 1;
    case 512: *S = 4; *C = 1; return 1;
    case 1024: *S = 4; *C = 1; return 1;
    case 2048: *S = 4; *C = 1; return 1;
    case 4096: *S = 4; *C = 1; return 1;
    case 8192: *S = 4; *C = 2; return 1;
    case 16384: *S = 4; *C = 4; return 1;
    case 32768: *S = 4; *C = 8; return 1;
    case 65536: *S = 4; *C = 16; return 1;
    default: return 0;
  }
}

/* Per-row emulation. Work arrays hold one value per (thread, step): ag/at[tid*S + i]. */
static void refkernel_row(const float* g, const float* x, float* y, int64_t L, int reverse,
                          int S, int C, float* ag, float* at, float* pg, float* pt) {
  const int T = (int)(L / S / C);
  const int nwarps = (T + 31) / 32;
  const int chunklen = T * S;
  float warp_g[32], warp_t[32];
  float chunk_g = 1.0f, chunk_t = 0.0f;
  for (int chunk = 0; chunk < C; ++chunk) {
    const int offset = (reverse ? C - 1 - chunk : chunk) * chunklen;
    /* thread-serial combine (full_scan.cu:84-111) */
    for (int tid = 0; tid < T; ++tid) {
      const int vec = reverse ? T - 1 - tid : tid;
      for (int i = 0; i < S; ++i) {
        const int c = reverse ? S - 1 - i : i;
        const float gate = g[offset + vec * S + c];
        const float tok = x[offset + vec * S + c];
        float* AG = ag + tid * S;
        float* AT = at + tid * S;
        if (i == 0) {
          if (chunk == 0) {
            AG[0] = (tid == 0) ? 1.0f : gate;
            AT[0] = tok;
          } else if (tid == 0) {
            AG[0] = chunk_g * gate;
            AT[0] = fmaf(chunk_t, gate, tok);
          } else {
            AG[0] = gate;
            AT[0] = tok;
          }
        } else {
          AG[i] = AG[i - 1] * gate;
          AT[i] = fmaf(AT[i - 1], gate, tok);
        }
      }
    }
    /* warp Kogge-Stone on each lane's last pair (full_scan.cu:113-125): every lane reads
     * the pre-step value of lane - delta */
    for (int delta = 1; delta < 32; delta *= 2) {
      for (int tid = 0; tid < T; ++tid) {
        pg[tid] = ag[tid * S + S - 1];
        pt[tid] = at[tid * S + S - 1];
      }
      for (int tid = 0; tid < T; ++tid) {
        const int lane = tid % 32;
        if (lane < delta) continue;
        const float prev_g = pg[tid - delta];
        const float prev_t = pt[tid - delta];
        for (int i = 0; i < S; ++i) {
          at[tid * S + i] = fmaf(prev_t, ag[tid * S + i], at[tid * S + i]);
          ag[tid * S + i] = prev_g * ag[tid * S + i];
        }
      }
    }
    /* warp totals and their scan by warp 0 (full_scan.cu:129-155) */
    for (int w = 0; w < 32; ++w) {
      const int last = w * 32 + 31;
      warp_g[w] = (w < nwarps) ? ag[last * S + S - 1] : 1.0f;
      warp_t[w] = (w < nwarps) ? at[last * S + S - 1] : 0.0f;
    }
    for (int delta = 1; delta < 32; delta *= 2) {
      float old_g[32], old_t[32];
      memcpy(old_g, warp_g, sizeof old_g);
      memcpy(old_t, warp_t, sizeof old_t);
      for (int lane = delta; lane < 32; ++lane) {
        warp_t[lane] = fmaf(old_t[lane - delta], old_g[lane], old_t[lane]);
        warp_g[lane] = old_g[lane - delta] * old_g[lane];
      }
    }
    /* apply the previous warps' prefix and store (full_scan.cu:159-170) */
    for (int tid = 0; tid < T; ++tid) {
      const int w = tid / 32;
      const int vec = reverse ? T - 1 - tid : tid;
      for (int i = 0; i < S; ++i) {
        if (w > 0) {
          at[tid * S + i] = fmaf(warp_t[w - 1], ag[tid * S + i], at[tid * S + i]);
          ag[tid * S + i] = warp_g[w - 1] * ag[tid * S + i];
        }
        const int c = reverse ? S - 1 - i : i;
        y[offset + vec * S + c] = at[tid * S + i];
      }
    }
    /* chunk carry from the last thread (full_scan.cu:172-175) */
    chunk_g = ag[(T - 1) * S + S - 1];
    chunk_t = at[(T - 1) * S + S - 1];
  }
}

/* Returns 0 on success, 1 for a seqlen the reference rejects, 2 for an allocation failure. */
int oracle_refkernel_f32(const float* g, const float* x, float* y, int64_t rows, int64_t L,
                         int reverse) {
  int S, C;
  if (!ref_tiles(L, &S, &C)) return 1;
  const int T = (int)(L / S / C);
  int failed = 0;
#pragma omp parallel
  {
    float* ag = (float*)malloc(sizeof(float) * (size_t)T * S);
    float* at = (float*)malloc(sizeof(float) * (size_t)T * S);
    float* pg = (float*)malloc(sizeof(float) * (size_t)T);
    float* pt = (float*)malloc(sizeof(float) * (size_t)T);
    const int ok = ag && at && pg && pt;
    if (!ok) {
#pragma omp atomic write
      failed = 1;
    }
    /* every thread reaches the worksharing loop; one without buffers skips its rows */
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
      if (ok) refkernel_row(g + r * L, x + r * L, y + r * L, L, reverse, S, C, ag, at, pg, pt);
    free(ag);
    free(at);
    free(pg);
    free(pt);
  }
  return failed ? 2 : 0;
}

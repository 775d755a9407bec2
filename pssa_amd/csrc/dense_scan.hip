// Dense-transition linear recurrence h_t = A_t h_(t-1) + b_t for gfx950.
//
// There is no counterpart in the reference (its SSM is diagonal); this is the
// standalone dense kernel.  The work is dominated by streaming the transition
// matrices (s*s floats per step) from HBM exactly once, so the kernel is
// built around bandwidth, not flops: one 256-thread workgroup walks one
// sequence in time order, every thread owns S/TPR columns of one row of A_t
// and keeps a ring of DEPTH future steps of its slice in registers, so the
// loads for step t+DEPTH are in flight while step t is reduced.  h_(t-1) is
// double-buffered in LDS (one barrier per step); the TPR partial dot products
// of a row meet through lane shuffles.  A two-level chunked scan would need
// s^3 flops per step for the A_2 A_1 combines (64x the sequential work at
// s=64) and still read A once, so time-sequential is the roofline choice
// whenever batch * (bytes per step) saturates HBM.
#include "common.h"

namespace pssa {

template <int S, int DEPTH>
__global__ __launch_bounds__(256) void dense_scan_kernel(const float* __restrict__ A,
                                                         const float* __restrict__ Bv,
                                                         const float* __restrict__ H0,
                                                         float* __restrict__ H, int L, int s) {
  constexpr int TPR = 256 / S;  // threads per row
  constexpr int CPT = S / TPR;  // columns per thread
  static_assert(CPT % 4 == 0 || CPT < 4, "column slice");
  __shared__ __attribute__((aligned(16))) float sh[2][S];

  const int tid = threadIdx.x;
  const int row = tid / TPR, part = tid % TPR;
  const int c0 = part * CPT;
  const int seq = blockIdx.x;
  const bool rvalid = row < s;
  const size_t ss = (size_t)s * s;
  const float* Aseq = A + (size_t)seq * L * ss;
  const float* bseq = Bv + (size_t)seq * L * s;
  float* hseq = H + (size_t)seq * L * s;

  if (tid < S) sh[0][tid] = (tid < s && H0) ? H0[(size_t)seq * s + tid] : 0.0f;

  float ring[DEPTH][CPT];
  float bring[DEPTH];
  auto fetch = [&](int t, int slot) {
    const float* arow = Aseq + (size_t)t * ss + (size_t)row * s;
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int col = c0 + q;
      ring[slot][q] = (rvalid && col < s) ? __builtin_nontemporal_load(arow + col) : 0.0f;
    }
    bring[slot] = (rvalid && part == 0) ? bseq[(size_t)t * s + row] : 0.0f;
  };
#pragma unroll
  for (int q = 0; q < DEPTH; ++q)
    if (q < L) fetch(q, q);
  __syncthreads();

  int cur = 0;
  for (int t0 = 0; t0 < L; t0 += DEPTH) {
#pragma unroll
    for (int q = 0; q < DEPTH; ++q) {
      const int t = t0 + q;
      if (t < L) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CPT; ++c) acc = fmaf(ring[q][c], sh[cur][c0 + c], acc);
#pragma unroll
        for (int off = TPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
        const float hv = acc + bring[q];
        if (part == 0 && rvalid) {
          sh[cur ^ 1][row] = hv;
          hseq[(size_t)t * s + row] = hv;
        }
        if (t + DEPTH < L) fetch(t + DEPTH, q);
        __syncthreads();
        cur ^= 1;
      }
    }
  }
}

Status launch_dense_scan(hipStream_t stream, const float* A, const float* B, const float* H0, float* H,
                         int batch, int L, int s) {
  if (batch <= 0 || L <= 0 || s <= 0) return Status::Invalid("dense scan: dimensions must be positive");
  if (s <= 16)
    dense_scan_kernel<16, 16><<<batch, 256, 0, stream>>>(A, B, H0, H, L, s);
  else if (s <= 32)
    dense_scan_kernel<32, 16><<<batch, 256, 0, stream>>>(A, B, H0, H, L, s);
  else if (s <= 64)
    dense_scan_kernel<64, 8><<<batch, 256, 0, stream>>>(A, B, H0, H, L, s);
  else
    return Status{PSSA_HIP_EUNSUPPORTED, "dense scan: d_state above 64 is not supported"};
  PSSA_LAUNCH_CHECK("dense_scan");
  return Status::Ok();
}

}  // namespace pssa

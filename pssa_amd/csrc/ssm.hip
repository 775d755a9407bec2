// Fused diagonal SSM for gfx950 (the reference's per-token recurrence,
// src/pssa.rs:1131-1144, and its staged twin, src/gpu_batch.rs:392-437):
//
//   bar_a = exp(delta_ti * rate_ij),  bar_b = delta_ti * B_tj,
//   h_tij = bar_a * h_(t-1)ij + bar_b * x_ti,   y_ti = sum_j h_tij * C_tj.
//
// With lanes*d*s independent channels (6.3M at the 105M prefill shape) a
// time-sequential walk per channel is work-optimal: no scan tree, no
// materialised states.  Mapping: a workgroup owns one lane b and 64
// consecutive channels i; its four waves split a range of 4*J states j, and
// each lane of a wave keeps its J states h_ij and rates in registers for the
// whole sequence.  Per time chunk the workgroup stages delta/x (per i) and
// B/C (per j) in LDS; B_tj and C_tj are read by every lane of a wave at the
// same address (LDS broadcast).  Per element the VALU work is one multiply
// for the exponent, one v_exp_f32, one multiply and two FMAs.  The four
// waves' partial sums over j meet in LDS and are added in a fixed order.
#include "ssm.h"

namespace pssa {

constexpr int SSM_TC = 16;  // time steps staged per chunk

template <int J, bool MAT>
__global__ __launch_bounds__(256) void ssm_scan_kernel(SsmArgs a) {
  __shared__ float sD[SSM_TC][64];
  __shared__ float sX[SSM_TC][64];
  __shared__ __attribute__((aligned(16))) float sB[SSM_TC][4 * J];
  __shared__ __attribute__((aligned(16))) float sC[SSM_TC][4 * J];
  __shared__ float sY[4][SSM_TC][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i0 = blockIdx.x * 64;
  const int b = blockIdx.y;
  const int jb = blockIdx.z * 4 * J;
  const int i = i0 + lane;
  const int jw = jb + wave * J;  // first state of this wave
  const bool ivalid = i < a.d;
  const int T = a.T, d = a.d, s = a.s;
  const size_t row0 = (size_t)b * T;

  float h[J], r2[J];
  float* carry = a.carry + (size_t)b * a.carry_stride;
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    const bool ok = ivalid && j < s;
    h[q] = ok ? carry[(size_t)i * s + j] : 0.0f;
    r2[q] = ok ? a.rates2[(size_t)i * s + j] : 0.0f;
  }
  if constexpr (MAT) {
    if (blockIdx.z == 0 && wave == 0) {
      // states[0] = h0 for this lane's channels (all j of row i).
      for (int j = 0; j < s && ivalid; ++j)
        a.states[(size_t)b * (T + 1) * d * s + (size_t)i * s + j] = carry[(size_t)i * s + j];
    }
  }

  for (int t0 = 0; t0 < T; t0 += SSM_TC) {
    // ---- stage the chunk ----
    for (int e = tid; e < SSM_TC * 64; e += 256) {
      const int tt = e >> 6, ii = e & 63;
      const int t = t0 + tt, gi = i0 + ii;
      const bool ok = t < T && gi < d;
      const size_t r = row0 + t;
      sD[tt][ii] = ok ? a.delta[r * a.ld_delta + gi] : 0.0f;
      sX[tt][ii] = ok ? a.xn[r * a.ld_x + gi] : 0.0f;
    }
    for (int e = tid; e < SSM_TC * 4 * J; e += 256) {
      const int tt = e / (4 * J), jj = e % (4 * J);
      const int t = t0 + tt, gj = jb + jj;
      const bool ok = t < T && gj < s;
      const size_t r = row0 + t;
      sB[tt][jj] = ok ? a.bproj[r * a.ld_b + gj] : 0.0f;
      sC[tt][jj] = ok ? a.cproj[r * a.ld_c + gj] : 0.0f;
    }
    __syncthreads();
    // ---- recurrence over the chunk ----
    const int steps = min(SSM_TC, T - t0);
    for (int tt = 0; tt < steps; ++tt) {
      const float dl = sD[tt][lane];
      const float u = dl * sX[tt][lane];
      const float* bt = &sB[tt][wave * J];
      const float* ct = &sC[tt][wave * J];
      float yp = 0.0f;
#pragma unroll
      for (int q = 0; q < J; ++q) {
        const float ab = __builtin_amdgcn_exp2f(dl * r2[q]);
        h[q] = fmaf(ab, h[q], u * bt[q]);
        yp = fmaf(h[q], ct[q], yp);
        if constexpr (MAT) {
          const int j = jw + q;
          if (ivalid && j < s) {
            const size_t c = (size_t)i * s + j;
            const size_t base = (size_t)b * T * d * s + (size_t)(t0 + tt) * d * s;
            a.bar_a[base + c] = ab;
            a.bar_b[base + c] = dl * bt[q];
            a.states[(size_t)b * (T + 1) * d * s + (size_t)(t0 + tt + 1) * d * s + c] = h[q];
          }
        }
      }
      sY[wave][tt][lane] = yp;
    }
    __syncthreads();
    // ---- combine the four waves' partial sums over j ----
    for (int e = tid; e < steps * 64; e += 256) {
      const int tt = e >> 6, ii = e & 63;
      const int gi = i0 + ii;
      if (gi < d) {
        const float v = ((sY[0][tt][ii] + sY[1][tt][ii]) + sY[2][tt][ii]) + sY[3][tt][ii];
        float* dst = a.y + (row0 + t0 + tt) * a.ld_y + gi;
        if (gridDim.z > 1)
          atomicAdd(dst, v);
        else
          *dst = v;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    if (ivalid && j < s) carry[(size_t)i * s + j] = h[q];
  }
}

static int pick_j(int s) { return s >= 128 ? 32 : (s >= 32 ? 8 : 2); }

bool ssm_needs_zeroed_y(int s) {
  const int J = pick_j(s);
  return s > 4 * J;
}

template <int J>
static void launch_j(hipStream_t stream, const SsmArgs& a, bool mat) {
  dim3 grid((a.d + 63) / 64, a.lanes, (a.s + 4 * J - 1) / (4 * J));
  if (mat)
    ssm_scan_kernel<J, true><<<grid, 256, 0, stream>>>(a);
  else
    ssm_scan_kernel<J, false><<<grid, 256, 0, stream>>>(a);
}

Status launch_ssm_scan(hipStream_t stream, const SsmArgs& a) {
  if (a.T <= 0 || a.d <= 0 || a.s <= 0 || a.lanes <= 0) return Status::Invalid("ssm: empty shape");
  const bool mat = a.bar_a && a.bar_b && a.states;
  switch (pick_j(a.s)) {
    case 32:
      launch_j<32>(stream, a, mat);
      break;
    case 8:
      launch_j<8>(stream, a, mat);
      break;
    default:
      launch_j<2>(stream, a, mat);
      break;
  }
  PSSA_LAUNCH_CHECK("ssm_scan");
  return Status::Ok();
}

__global__ void scale_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n,
                             float scale) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = in[i] * scale;
}

Status launch_scale(hipStream_t stream, const float* in, float* out, size_t n, float scale) {
  if (n == 0) return Status::Ok();
  scale_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(in, out, n, scale);
  PSSA_LAUNCH_CHECK("scale");
  return Status::Ok();
}

}  // namespace pssa

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

// ---------------------------------------------------------------------------
// Unpipelined variant: with MAT it also writes bar_a, bar_b and every state
// h_t (stage API, small diagnostic shapes); without MAT it serves sequences
// shorter than one pipelined chunk (single-token decode), where it runs
// exactly T steps.
constexpr int MAT_TC = 16;

template <int J, bool MAT>
__global__ __launch_bounds__(256) void ssm_materialize_kernel(SsmArgs a) {
  __shared__ float sD[MAT_TC][64];
  __shared__ float sX[MAT_TC][64];
  __shared__ float sB[MAT_TC][4 * J];
  __shared__ float sC[MAT_TC][4 * J];
  constexpr int GS = J < 16 ? J : 16;  // readout group, as in the production scan
  constexpr int NG = J / GS;
  __shared__ float sY[4 * NG][MAT_TC][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i0 = blockIdx.x * 64;
  const int b = blockIdx.y;
  const int jb = blockIdx.z * 4 * J;
  const int i = i0 + lane;
  const int jw = jb + wave * J;
  const bool ivalid = i < a.d;
  const int T = a.T, d = a.d, s = a.s;
  const size_t row0 = (size_t)b * T;
  const size_t ds = (size_t)d * s;

  float h[J], r2[J];
  float* carry = a.carry + (size_t)b * a.carry_stride;
  const CarryCol cc = carry_col(jw, i, d, s);
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    const bool ok = ivalid && j < s;
    h[q] = ok ? carry[cc.base + q * cc.stride] : 0.0f;
    r2[q] = ok ? a.rates2[(size_t)j * d + i] : 0.0f;
  }
  if (MAT && blockIdx.z == 0 && wave == 0 && ivalid)
    for (int j = 0; j < s; ++j) a.states[(size_t)b * (T + 1) * ds + (size_t)i * s + j] = carry[carry_at(j, i, d, s)];

  for (int t0 = 0; t0 < T; t0 += MAT_TC) {
    for (int e = tid; e < MAT_TC * 64; e += 256) {
      const int tt = e >> 6, ii = e & 63;
      const int t = t0 + tt, gi = i0 + ii;
      const bool ok = t < T && gi < d;
      const size_t r = row0 + t;
      sD[tt][ii] = ok ? a.delta[r * a.ld_delta + gi] : 0.0f;
      sX[tt][ii] = ok ? a.xn[r * a.ld_x + gi] : 0.0f;
    }
    for (int e = tid; e < MAT_TC * 4 * J; e += 256) {
      const int tt = e / (4 * J), jj = e % (4 * J);
      const int t = t0 + tt, gj = jb + jj;
      const bool ok = t < T && gj < s;
      const size_t r = row0 + t;
      sB[tt][jj] = ok ? a.bproj[r * a.ld_b + gj] : 0.0f;
      sC[tt][jj] = ok ? a.cproj[r * a.ld_c + gj] : 0.0f;
    }
    __syncthreads();
    const int steps = min(MAT_TC, T - t0);
    for (int tt = 0; tt < steps; ++tt) {
      const float dl = sD[tt][lane];
      const float u = dl * sX[tt][lane];
      // Readout in the production scan's order (groups of GS states, four
      // partial sums each), so that a run of single-token steps equals one
      // prefill bit for bit.
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float yp4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int qq = 0; qq < GS; ++qq) {
          const int q = g * GS + qq;
          const float bq = sB[tt][wave * J + q];
          const float ab = __builtin_amdgcn_exp2f(dl * r2[q]);
          h[q] = fmaf(ab, h[q], u * bq);
          yp4[qq & 3] = fmaf(h[q], sC[tt][wave * J + q], yp4[qq & 3]);
          const int j = jw + q;
          if (MAT && ivalid && j < s) {
            const size_t c = (size_t)i * s + j;
            const size_t base = (size_t)b * T * ds + (size_t)(t0 + tt) * ds;
            a.bar_a[base + c] = ab;
            a.bar_b[base + c] = dl * bq;
            a.states[(size_t)b * (T + 1) * ds + (size_t)(t0 + tt + 1) * ds + c] = h[q];
          }
        }
        sY[wave * NG + g][tt][lane] = (yp4[0] + yp4[1]) + (yp4[2] + yp4[3]);
      }
    }
    __syncthreads();
    for (int e = tid; e < steps * 64; e += 256) {
      const int tt = e >> 6, ii = e & 63;
      const int gi = i0 + ii;
      if (gi < d) {
        float v = sY[0][tt][ii];
#pragma unroll
        for (int g = 1; g < 4 * NG; ++g) v += sY[g][tt][ii];
        const size_t r = row0 + t0 + tt;
        if (!MAT && a.y_part)
          a.y_part[((size_t)blockIdx.z * a.rows + r) * a.d + gi] = v;
        else if (gridDim.z > 1)
          atomicAdd(a.y + r * a.ld_y + gi, v);
        else
          a.y[r * a.ld_y + gi] = v;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    if (ivalid && j < s) carry[cc.base + q * cc.stride] = h[q];
  }
}

// ---------------------------------------------------------------------------
// One time step (decode): no staging, just the carry update.  A workgroup
// owns LPB lanes and 64 channels, and NB consecutive state blocks of 4*J
// states (four waves each); with NB covering all of d_state it also finishes
// the readout, adding the block sums in block order as the multi-block paths
// do, and writes y (and its bf16 copy) directly.  The arithmetic and the
// readout order are those of the kernels above, so a step here equals the
// same step inside a prefill bit for bit.  The traffic is the carry read and
// written once, streamed past the caches, plus the rates, which the LPB
// lanes of a workgroup share: they load from L2 once per workgroup, and the
// next lane's carry, B/C, delta and x loads are issued before this lane's
// carry stores, so the loads of consecutive lanes overlap.
template <int J, int NB, int LPB>
__global__ __launch_bounds__(NB * 256) void ssm_step_kernel(SsmArgs a) {
  constexpr int GS = J < 16 ? J : 16;
  constexpr int NG = J / GS;
  static_assert(J <= 32, "one B/C load per wave covers at most 32 states");
  __shared__ float sY[LPB][NB * 4 * NG][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i0 = blockIdx.x * 64, b0 = blockIdx.y * LPB;
  const int jw = blockIdx.z * NB * 4 * J + wave * J;
  const int i = i0 + lane;
  const bool ivalid = i < a.d;
  const int d = a.d, s = a.s;
  const int jb = jw + (lane & 31);
  // One lane's step inputs: the wave's B values (lanes 0..J-1) and C values
  // (lanes 32..32+J-1) in one load, broadcast with readlane; delta, the
  // input term u = delta * x and the J carries.
  struct LaneIn {
    float h[J];
    float bc, dl, u;
  };
  auto load_lane = [&](int b, LaneIn& L) {
    const size_t r = b;  // T == 1: lane b's row
    const float* carry = a.carry + (size_t)b * a.carry_stride;
    L.bc = 0.0f;
    if ((lane & 31) < J && jb < s) L.bc = lane < 32 ? a.bproj[r * a.ld_b + jb] : a.cproj[r * a.ld_c + jb];
    L.dl = ivalid ? a.delta[r * a.ld_delta + i] : 0.0f;
    L.u = L.dl * (ivalid ? a.xn[r * a.ld_x + i] : 0.0f);
#pragma unroll
    for (int q = 0; q < J; ++q) {
      const int j = jw + q;
      L.h[q] = (ivalid && j < s) ? __builtin_nontemporal_load(&carry[carry_at(j, i, d, s)]) : 0.0f;
    }
  };
  float r2[J];
  LaneIn cur, nxt;
  load_lane(b0, cur);
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    r2[q] = (ivalid && j < s) ? a.rates2[(size_t)j * d + i] : 0.0f;
  }
#pragma unroll
  for (int l = 0; l < LPB; ++l) {
    const int b = b0 + l;
    if (b >= a.lanes) break;  // uniform over the workgroup
    LaneIn& L = (l & 1) ? nxt : cur;
    LaneIn& N = (l & 1) ? cur : nxt;
    if (l + 1 < LPB && b + 1 < a.lanes) load_lane(b + 1, N);
    float* carry = a.carry + (size_t)b * a.carry_stride;
    const int bc_bits = __float_as_int(L.bc);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float yp4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int qq = 0; qq < GS; ++qq) {
        const int q = g * GS + qq;
        const int j = jw + q;
        const float bq = __int_as_float(__builtin_amdgcn_readlane(bc_bits, q));
        const float cq = __int_as_float(__builtin_amdgcn_readlane(bc_bits, 32 + q));
        const float ab = __builtin_amdgcn_exp2f(L.dl * r2[q]);
        const float hv = fmaf(ab, L.h[q], L.u * bq);
        yp4[qq & 3] = fmaf(hv, cq, yp4[qq & 3]);
        if (ivalid && j < s) __builtin_nontemporal_store(hv, &carry[carry_at(j, i, d, s)]);
      }
      sY[l][wave * NG + g][lane] = (yp4[0] + yp4[1]) + (yp4[2] + yp4[3]);
    }
  }
  __syncthreads();
  // Wave l finishes lane b0 + l's readout (LPB <= NB * 4 waves).
  static_assert(LPB <= NB * 4, "one wave per lane for the readout");
  const int b = b0 + wave;
  if (wave < LPB && b < a.lanes && ivalid) {
    const size_t r = b;
    float v = 0.0f;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      float bv = sY[wave][blk * 4 * NG][lane];
#pragma unroll
      for (int g = 1; g < 4 * NG; ++g) bv += sY[wave][blk * 4 * NG + g][lane];
      v = blk == 0 ? bv : v + bv;
    }
    if (a.y_part) {
      a.y_part[((size_t)blockIdx.z * a.rows + r) * a.d + i] = v;
    } else if (gridDim.z > 1) {
      atomicAdd(a.y + r * a.ld_y + i, v);
    } else {
      a.y[r * a.ld_y + i] = v;
      if (a.y16) a.y16[r * a.ld_y16 + i] = bf16_bits_dev(v);
    }
  }
}

// ---------------------------------------------------------------------------
// Production scan.  The next TC time steps' inputs are fetched into registers
// while the current TC steps run out of LDS, so the global-memory latency of
// the staging hides behind the recurrence.  Time steps past the end of a lane
// read delta = x = 0: the update is then h <- exp2(0) h + 0 = h, so whole
// chunks run unguarded and only the stores check t < T.  Per state the inner
// loop batches GS independent exponentials before the dependent FMAs.
//
// NW waves of J states each cover one state block of NW*J states (128 for
// J >= 32 with four waves and J = 16 with eight).  Every variant sums the
// readout in the same order (readout_group_size): per group of GS states four
// partial sums over j = p (mod 4), combined as (p0 + p1) + (p2 + p3), then the
// group sums of the block added one after another in state order.  The
// variant can therefore be chosen by occupancy alone without changing a bit
// of the result, and a run of single-token steps still equals one prefill.
#ifndef PSSA_SSM_TC
#define PSSA_SSM_TC 4
#endif
constexpr int SSM_TC = PSSA_SSM_TC;

template <int J, int NW, int WPE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE))) void ssm_scan_kernel(SsmArgs a) {
  // Steps staged per chunk: with few states per lane a chunk's compute is
  // short, so 16 steps stand between a chunk's input loads and their use.
  constexpr int TC = J <= 8 ? 4 * SSM_TC : SSM_TC;
  constexpr int NT = NW * 64;
  constexpr int GS = J < 16 ? J : 16;        // states per readout group
  constexpr int NG = J / GS;                 // readout groups per wave
  constexpr int SB = NW * J;                 // states per block
  constexpr int NDX = (TC * 64 + NT - 1) / NT;  // delta/x values staged per thread
  constexpr int NBC = (TC * SB + NT - 1) / NT;  // B/C values staged per thread
  __shared__ float sD[TC][64];
  __shared__ float sX[TC][64];
  __shared__ __attribute__((aligned(16))) float sB[TC][SB];
  __shared__ __attribute__((aligned(16))) float sC[TC][SB];
  __shared__ float sY[NW * NG][TC][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i0 = blockIdx.x * 64;
  const int b = blockIdx.y;
  const int jb = blockIdx.z * SB;
  const int i = i0 + lane;
  const int jw = jb + wave * J;
  const bool ivalid = i < a.d;
  const int T = a.T, d = a.d, s = a.s;
  const size_t row0 = (size_t)b * T;

  float h[J], r2[J];
  float* carry = a.carry + (size_t)b * a.carry_stride;
  const CarryCol cc = carry_col(jw, i, d, s);
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    const bool ok = ivalid && j < s;
    h[q] = ok ? carry[cc.base + q * cc.stride] : 0.0f;
    r2[q] = ok ? a.rates2[(size_t)j * d + i] : 0.0f;
  }

  float pd[NDX], px[NDX], pb[NBC], pc[NBC];
  auto load = [&](int t0) {
#pragma unroll
    for (int k = 0; k < NDX; ++k) {
      const int e = tid + NT * k;
      const int t = t0 + (e >> 6), gi = i0 + (e & 63);
      const bool ok = e < TC * 64 && t < T && gi < d;
      const size_t r = row0 + t;
      pd[k] = ok ? a.delta[r * a.ld_delta + gi] : 0.0f;
      px[k] = ok ? a.xn[r * a.ld_x + gi] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < NBC; ++k) {
      const int e = tid + NT * k;
      const int t = t0 + e / SB, gj = jb + e % SB;
      const bool ok = e < TC * SB && t < T && gj < s;
      const size_t r = row0 + t;
      pb[k] = ok ? a.bproj[r * a.ld_b + gj] : 0.0f;
      pc[k] = ok ? a.cproj[r * a.ld_c + gj] : 0.0f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int k = 0; k < NDX; ++k) {
      const int e = tid + NT * k;
      if (e < TC * 64) {
        sD[e >> 6][e & 63] = pd[k];
        sX[e >> 6][e & 63] = px[k];
      }
    }
#pragma unroll
    for (int k = 0; k < NBC; ++k) {
      const int e = tid + NT * k;
      if (e < TC * SB) {
        sB[e / SB][e % SB] = pb[k];
        sC[e / SB][e % SB] = pc[k];
      }
    }
  };

  load(0);
  store();
  __syncthreads();
  for (int t0 = 0; t0 < T; t0 += TC) {
    if (t0 + TC < T) load(t0 + TC);
    if constexpr (J <= 8) {
      // Few states per lane (small d_state, where a grid of few lanes is
      // bound by the step chain): per four steps the exponentials and input
      // terms first, all independent of h, then the recurrence and readout.
      // The same operations as below (one readout group), so the same bits.
      for (int t4 = 0; t4 < TC; t4 += 4) {
        float ab[4][J], ub[4][J];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dl = sD[t4 + i][lane];
          const float u = dl * sX[t4 + i][lane];
          const float* bt = &sB[t4 + i][wave * J];
#pragma unroll
          for (int q = 0; q < J; ++q) {
            ab[i][q] = __builtin_amdgcn_exp2f(dl * r2[q]);
            ub[i][q] = u * bt[q];
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float* ct = &sC[t4 + i][wave * J];
          float yp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int q = 0; q < J; ++q) h[q] = fmaf(ab[i][q], h[q], ub[i][q]);
#pragma unroll
          for (int q = 0; q < J; ++q) yp[q & 3] = fmaf(h[q], ct[q], yp[q & 3]);
          sY[wave][t4 + i][lane] = (yp[0] + yp[1]) + (yp[2] + yp[3]);
        }
      }
    } else
    for (int tt = 0; tt < TC; ++tt) {
      const float dl = sD[tt][lane];
      const float u = dl * sX[tt][lane];
      const float* bt = &sB[tt][wave * J];
      const float* ct = &sC[tt][wave * J];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const int g0 = g * GS;
        float ab[GS];
        float yp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < GS; ++q) ab[q] = dl * r2[g0 + q];
#pragma unroll
        for (int q = 0; q < GS; ++q) ab[q] = __builtin_amdgcn_exp2f(ab[q]);
#pragma unroll
        for (int q = 0; q < GS; ++q) h[g0 + q] = fmaf(ab[q], h[g0 + q], u * bt[g0 + q]);
#pragma unroll
        for (int q = 0; q < GS; ++q) yp[q & 3] = fmaf(h[g0 + q], ct[g0 + q], yp[q & 3]);
        sY[wave * NG + g][tt][lane] = (yp[0] + yp[1]) + (yp[2] + yp[3]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NDX; ++k) {
      const int e = tid + NT * k;
      const int tt = e >> 6, gi = i0 + (e & 63);
      const int t = t0 + tt;
      if (e < TC * 64 && t < T && gi < d) {
        float v = sY[0][tt][e & 63];
#pragma unroll
        for (int g = 1; g < NW * NG; ++g) v += sY[g][tt][e & 63];
        const size_t r = row0 + t;
        if (a.y_part)
          a.y_part[((size_t)blockIdx.z * a.rows + r) * a.d + gi] = v;
        else if (gridDim.z > 1)
          atomicAdd(a.y + r * a.ld_y + gi, v);
        else
          a.y[r * a.ld_y + gi] = v;
      }
    }
    if (t0 + TC < T) store();
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < J; ++q) {
    const int j = jw + q;
    if (ivalid && j < s) carry[cc.base + q * cc.stride] = h[q];
  }
}

// y = sum over state blocks of the partial readouts, in block order.
__global__ void ssm_reduce_kernel(const float* __restrict__ part, int nz, size_t rows, int d,
                                  float* __restrict__ y, int ld_y) {
  const size_t n = rows * (size_t)d;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
    float v = part[e];
    for (int z = 1; z < nz; ++z) v += part[(size_t)z * n + e];
    y[(e / d) * ld_y + e % d] = v;
  }
}

static int pick_j(int s) { return s >= 128 ? 32 : (s >= 32 ? 8 : 2); }

bool ssm_step_writes_y(int T, int s) { return T == 1 && ssm_state_blocks(s) <= 2; }

int ssm_state_blocks(int s) {
  const int J = pick_j(s);
  return (s + 4 * J - 1) / (4 * J);
}

bool ssm_needs_zeroed_y(int s) { return ssm_state_blocks(s) == 2; }

// Workgroups at which the four-wave J = 32 scan holds three waves per SIMD on
// the 256 CUs; below that the eight-wave J = 16 variant (same state blocks,
// twice the waves, half the registers per lane) keeps the SIMDs fed.
constexpr long kScanFullGrid = 768;

// Lanes per decode-step workgroup (they share the rate loads).
#ifndef PSSA_SSM_STEP_LPB
#define PSSA_SSM_STEP_LPB 4
#endif

template <int J>
static void launch_j(hipStream_t stream, const SsmArgs& a, bool mat) {
  dim3 grid((a.d + 63) / 64, a.lanes, (a.s + 4 * J - 1) / (4 * J));
  if (mat) {
    ssm_materialize_kernel<J, true><<<grid, 256, 0, stream>>>(a);
  } else if (a.T == 1) {
    // At most one lane per wave of the workgroup (the readout's waves).
    constexpr int LPB2 = PSSA_SSM_STEP_LPB < 8 ? PSSA_SSM_STEP_LPB : 8;
    constexpr int LPB1 = PSSA_SSM_STEP_LPB < 4 ? PSSA_SSM_STEP_LPB : 4;
    if (grid.z == 2) {
      grid.z = 1;
      grid.y = (a.lanes + LPB2 - 1) / LPB2;
      ssm_step_kernel<J, 2, LPB2><<<grid, 512, 0, stream>>>(a);
    } else {
      grid.y = (a.lanes + LPB1 - 1) / LPB1;
      ssm_step_kernel<J, 1, LPB1><<<grid, 256, 0, stream>>>(a);
    }
  } else if (a.T < SSM_TC) {
    ssm_materialize_kernel<J, false><<<grid, 256, 0, stream>>>(a);
  } else if constexpr (J == 32) {
    if ((long)grid.x * grid.y * grid.z < kScanFullGrid && !a.concurrent)
      ssm_scan_kernel<16, 8, 4><<<grid, 512, 0, stream>>>(a);
    else
      ssm_scan_kernel<32, 4, 3><<<grid, 256, 0, stream>>>(a);
  } else if constexpr (J <= 8) {
    // Few states per lane: a small model's grid of a few workgroups, each
    // bound by its step chain, so occupancy gives nothing and the register
    // budget of two waves per SIMD keeps the 16-step staging out of scratch.
    ssm_scan_kernel<J, 4, 2><<<grid, 256, 0, stream>>>(a);
  } else {
    ssm_scan_kernel<J, 4, 3><<<grid, 256, 0, stream>>>(a);
  }
}

Status launch_ssm_scan(hipStream_t stream, const SsmArgs& a_in) {
  SsmArgs a = a_in;
  if (a.T <= 0 || a.d <= 0 || a.s <= 0 || a.lanes <= 0) return Status::Invalid("ssm: empty shape");
  const bool mat = a.bar_a && a.bar_b && a.states;
  const int nz = ssm_state_blocks(a.s);
  a.rows = (size_t)a.lanes * a.T;
  if (mat || nz <= 2) {
    a.y_part = nullptr;
  } else if (!a.y_part) {
    return Status::Invalid("ssm: more than two state blocks need a partial-sum buffer");
  }
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
  if (a.y_part) {
    const size_t n = a.rows * (size_t)a.d;
    size_t g = (n + 255) / 256;
    if (g > 16384) g = 16384;
    ssm_reduce_kernel<<<(unsigned)g, 256, 0, stream>>>(a.y_part, nz, a.rows, a.d, a.y, a.ld_y);
    PSSA_LAUNCH_CHECK("ssm_reduce");
  }
  return Status::Ok();
}

__global__ void scale_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n,
                             float scale) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = in[i] * scale;
}

// 32x32 tiles through LDS; blockIdx.z = matrix.
__global__ void transpose_kernel(const float* __restrict__ in, float* __restrict__ out, int rows, int cols,
                                 float scale) {
  __shared__ float tile[32][33];
  const size_t base = (size_t)blockIdx.z * rows * cols;
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  for (int k = threadIdx.y; k < 32; k += blockDim.y) {
    const int r = r0 + k, c = c0 + threadIdx.x;
    if (r < rows && c < cols) tile[k][threadIdx.x] = in[base + (size_t)r * cols + c];
  }
  __syncthreads();
  for (int k = threadIdx.y; k < 32; k += blockDim.y) {
    const int c = c0 + k, r = r0 + threadIdx.x;
    if (r < rows && c < cols) out[base + (size_t)c * rows + r] = tile[threadIdx.x][k] * scale;
  }
}

Status launch_transpose(hipStream_t stream, const float* in, float* out, size_t count, int rows,
                        int cols, float scale) {
  if (!count || rows <= 0 || cols <= 0) return Status::Ok();
  if (count > 65535) return Status::Invalid("transpose: too many matrices");
  dim3 grid((cols + 31) / 32, (rows + 31) / 32, (unsigned)count), block(32, 8);
  transpose_kernel<<<grid, block, 0, stream>>>(in, out, rows, cols, scale);
  PSSA_LAUNCH_CHECK("transpose");
  return Status::Ok();
}

// Carries between the reference's [d, s] per matrix and the device's
// channel-blocked layout (carry_at): one 64-channel x 64-state tile per
// workgroup through LDS, so both sides move contiguous runs.
__global__ __launch_bounds__(256) void carry_convert_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                            int d, int s, int to_device) {
  __shared__ float tile[64][65];
  const size_t m = blockIdx.z, ds = (size_t)d * s;
  const float* src = in + m * ds;
  float* dst = out + m * ds;
  const int i0 = blockIdx.x * 64, j0 = blockIdx.y * 64;
  const int w = min(64, d - i0), hs = min(64, s - j0);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if (to_device) {
    for (int r = ty; r < w; r += 4)
      if (tx < hs) tile[r][tx] = src[(size_t)(i0 + r) * s + j0 + tx];
    __syncthreads();
    float* blk = dst + (size_t)i0 * s;  // the channel block's run: state j at + j * w
    for (int r = ty; r < hs; r += 4)
      if (tx < w) blk[(size_t)(j0 + r) * w + tx] = tile[tx][r];
  } else {
    const float* sb = src + (size_t)i0 * s;
    for (int r = ty; r < hs; r += 4)
      if (tx < w) tile[tx][r] = sb[(size_t)(j0 + r) * w + tx];
    __syncthreads();
    for (int r = ty; r < w; r += 4)
      if (tx < hs) dst[(size_t)(i0 + r) * s + j0 + tx] = tile[r][tx];
  }
}

Status launch_carry_convert(hipStream_t stream, const float* in, float* out, size_t count, int d, int s,
                            bool to_device) {
  if (!count || d <= 0 || s <= 0) return Status::Ok();
  for (size_t m0 = 0; m0 < count; m0 += 65535) {
    const size_t cnt = count - m0 < 65535 ? count - m0 : 65535, off = m0 * (size_t)d * s;
    dim3 grid((d + 63) / 64, (s + 63) / 64, (unsigned)cnt);
    carry_convert_kernel<<<grid, 256, 0, stream>>>(in + off, out + off, d, s, to_device ? 1 : 0);
    PSSA_LAUNCH_CHECK("carry_convert");
  }
  return Status::Ok();
}

Status launch_scale(hipStream_t stream, const float* in, float* out, size_t n, float scale) {
  if (n == 0) return Status::Ok();
  scale_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(in, out, n, scale);
  PSSA_LAUNCH_CHECK("scale");
  return Status::Ok();
}

}  // namespace pssa

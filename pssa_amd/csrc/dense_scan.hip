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

// ---------------------------------------------------------------------------
// d_state = 64 with the operands 16-byte aligned: the transition streams
// through a ring of DS_RING LDS slots, each holding one step's A_t (16 KiB)
// and b_t, filled by direct-to-LDS loads (global_load_lds_dwordx4).  Waves
// 0-3 only compute: every thread owns 16 columns of one row (4 threads a
// row), the row's partial dot products meet through DPP quad permutes, and
// one barrier per step publishes h_t; wave 0 also writes h_(t-1) out.  Waves
// 4 and 5 only load (9 and 8 instructions a slot), so their s_waitcnt counts
// cover loads alone and no load instruction sits on the compute waves'
// per-step path.  Ring depth 9 keeps 7 slots (116 KiB) in flight per
// sequence; 7 x 9 = 63 instructions is the most a wave can count.
constexpr int DS_S = 64;
constexpr int DS_RING = 9;
constexpr int DS_SLOT = DS_S * DS_S + DS_S;       // floats per ring slot (A_t then b_t)
constexpr int DS_CHUNKS = DS_SLOT / 4;            // 16-byte chunks per slot (1040)
constexpr int DS_LOADERS = 2;                     // waves issuing the ring's loads
constexpr int DS_NI0 = 9;                         // instructions per slot, first loader
constexpr int DS_NI1 = (DS_CHUNKS - DS_NI0 * 64 + 63) / 64;  // second loader (8)
constexpr int DS_THREADS = (4 + DS_LOADERS) * 64;
static_assert(DS_NI0 >= DS_NI1, "loader 0 carries the larger share");

// s_waitcnt immediate for vmcnt(v) alone (gfx9: vmcnt bits [3:0] and [15:14],
// expcnt and lgkmcnt left at their no-wait maxima).
constexpr int vmcnt_only(int v) { return (v & 0xF) | (((v >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8); }
static_assert((DS_RING - 2) * DS_NI0 <= 63, "vmcnt holds at most 63");

__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // quad_perm 1,0,3,2
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // quad_perm 2,3,0,1
  return v;
}

__global__ __launch_bounds__(DS_THREADS) void dense_scan_ring_kernel(const float* __restrict__ A,
                                                                     const float* __restrict__ Bv,
                                                                     const float* __restrict__ H0,
                                                                     float* __restrict__ H, int L) {
  __shared__ __attribute__((aligned(1024))) float ring_s[DS_RING][DS_SLOT];
  __shared__ __attribute__((aligned(16))) float sh_s[2][DS_S];
  float* ring = &ring_s[0][0];
  float* sh = &sh_s[0][0];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool loader = wave >= 4;
  const int row = (tid >> 2) & (DS_S - 1), part = tid & 3, c0 = part * 16;
  const int seq = blockIdx.x;
  const float* Aseq = A + (size_t)seq * L * DS_S * DS_S;
  const float* bseq = Bv + (size_t)seq * L * DS_S;
  float* hseq = H + (size_t)seq * L * DS_S;

  // Loader w (wave 4 + w) moves chunks first_w + 64 i + lane of a slot; the
  // source of chunk c at step t is src[i] + t * (A or b stride).
  const int lw = loader ? wave - 4 : 0;
  const int ni = lw == 0 ? DS_NI0 : DS_NI1;
  const int first = lw * DS_NI0 * 64;
  const float* src[DS_NI0];
  size_t stride[DS_NI0];
#pragma unroll
  for (int i = 0; i < DS_NI0; ++i) {
    const int c = min(first + i * 64 + lane, DS_CHUNKS - 1);
    const bool in_a = c < DS_S * DS_S / 4;
    src[i] = in_a ? Aseq + 4 * c : bseq + 4 * (c - DS_S * DS_S / 4);
    stride[i] = in_a ? (size_t)DS_S * DS_S : (size_t)DS_S;
  }
  auto issue = [&](int t) {
    float* slot = ring + (t % DS_RING) * DS_SLOT;
#pragma unroll
    for (int i = 0; i < DS_NI0; ++i) {
      const int c = first + i * 64;
      if (i < ni && c + lane < DS_CHUNKS)
        __builtin_amdgcn_global_load_lds((const void*)(src[i] + (size_t)t * stride[i]),
                                         (__attribute__((address_space(3))) void*)(slot + 4 * c), 16, 0, 0);
    }
  };
  if (tid < DS_S) sh[tid] = H0 ? H0[(size_t)seq * DS_S + tid] : 0.0f;
  if (loader)
    for (int t = 0; t < DS_RING - 1 && t < L; ++t) issue(t);

  int cur = 0;
  for (int t = 0; t < L; ++t) {
    if (loader) {
      // Slot t is complete once only the slots issued after it are in flight.
      if (t + DS_RING - 2 < L) {
        if (lw == 0)
          __builtin_amdgcn_s_waitcnt(vmcnt_only((DS_RING - 2) * DS_NI0));
        else
          __builtin_amdgcn_s_waitcnt(vmcnt_only((DS_RING - 2) * DS_NI1));
      } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // near the end
      }
    } else {
      // This wave's LDS writes are done; meet the others (a plain barrier: a
      // __syncthreads fence would also drain the ring's loads).
      __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8) | (0xF) | (0x3 << 14));  // lgkmcnt(0)
    }
    asm volatile("s_barrier" ::: "memory");
    if (loader) {
      // Every compute wave finished step t - 1: refill its slot.
      if (t + DS_RING - 1 < L) issue(t + DS_RING - 1);
      continue;
    }

    const float* slot = ring + (t % DS_RING) * DS_SLOT;
    const float* arow = slot + row * DS_S + c0;
    const float* h = sh + cur * DS_S + c0;
    float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 av = *reinterpret_cast<const float4*>(arow + 4 * q);
      const float4 hv = *reinterpret_cast<const float4*>(h + 4 * q);
      p[q] = fmaf(av.x, hv.x, p[q]);
      p[q] = fmaf(av.y, hv.y, p[q]);
      p[q] = fmaf(av.z, hv.z, p[q]);
      p[q] = fmaf(av.w, hv.w, p[q]);
    }
    const float acc = quad_sum((p[0] + p[1]) + (p[2] + p[3]));
    if (part == 0) sh[(cur ^ 1) * DS_S + row] = acc + slot[DS_S * DS_S + row];
    // Off the step's critical path: write h_(t-1) out.
    if (wave == 0 && t > 0) hseq[(size_t)(t - 1) * DS_S + lane] = sh[cur * DS_S + lane];
    cur ^= 1;
  }
  __syncthreads();
  if (wave == 0) hseq[(size_t)(L - 1) * DS_S + lane] = sh[(L & 1) * DS_S + lane];
}

static bool ring_fits(const float* A, const float* B, int s) {
  return s == DS_S && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0;
}

Status init_dense_scan_attributes() { return Status::Ok(); }

Status launch_dense_scan(hipStream_t stream, const float* A, const float* B, const float* H0, float* H,
                         int batch, int L, int s) {
  if (batch <= 0 || L <= 0 || s <= 0) return Status::Invalid("dense scan: dimensions must be positive");
  if (ring_fits(A, B, s)) {
    dense_scan_ring_kernel<<<batch, DS_THREADS, 0, stream>>>(A, B, H0, H, L);
  } else if (s <= 16)
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

// Dense-transition linear recurrence h_t = A_t h_(t-1) + b_t for gfx950.
//
// There is no counterpart in the reference (its SSM is diagonal); this is the
// standalone dense kernel.  Two schedules:
//
//  - Time-sequential (dense_scan_ring_kernel, dense_scan_kernel): one
//    workgroup walks one sequence in time order and reads every A_t once.
//    With one workgroup per sequence only `batch` CUs stream, and a CU
//    streams about 22 B/clk from HBM (3.3 TB/s with 64 CUs, measured), so
//    this bounds long sequences of few lanes.
//
//  - Chunked two-level (dense_twolevel_kernel, d_state 64): time is cut into
//    windows of TL_SUB sub-chunks of TL_LC steps.  Level 1 composes each
//    sub-chunk's affine map (P, q) = (A_last ... A_first, local response from
//    zero) with matrix-core products P <- A_t P; level 2 carries the window's
//    entry state through the composed maps (h <- P h + q) so every sub-chunk
//    of the window knows its entry state, and re-runs its steps exactly in
//    fp32.  Launch l composes window l and re-runs window l - 1, so a
//    window's transitions are read the second time shortly after the first,
//    while they are still in the device's last-level cache.
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

// ---------------------------------------------------------------------------
// Chunked two-level scan, d_state 64.  One launch runs two roles side by side
// (workgroup-uniform): the re-run role for window w_rerun (TL_SUB workgroups
// per sequence) and the compose role for window w_agg (TL_SUB - 1 per
// sequence: the last sub-chunk's map is never needed, the next window starts
// from the exact re-run state).  Both stream one step's A_t and b_t per LDS
// ring slot with direct-to-LDS loads from two loader waves, as the ring
// kernel does; the slot's A_t rows keep their sixteen 16-byte chunks
// XOR-swizzled by the row index, so 16 lanes reading one chunk column of 16
// rows hit 16 distinct bank groups.
//
// Compose role, per step (four compute waves):
//  - q <- A_t q + b_t in fp32 (four threads a row, DPP quad sums);
//  - P <- A_t P on the matrix cores: wave c computes rows 16c .. 16c+15 of
//    the new P (one 16-row tile, four 16-column tiles, 16x16 accumulator
//    layout: lane l holds column l%16 and rows 4(l/16)+r).  Both operands are
//    split into bf16 hi + lo parts (x = hi + lo to about 2^-17 relative) and
//    three v_mfma_f32_16x16x32_bf16 products (lo.hi, hi.lo, hi.hi) accumulate
//    each 16x16x32 block in fp32.  The waves exchange P through LDS as
//    ready-split B fragments: the k slots of a 32-row block are rows
//    4(l/16)+r of its first and second 16-row tiles, which lane l of waves
//    2kb and 2kb+1 hold, so every lane reads the 16 bytes its own lane index
//    wrote and A_t's fragments use the same k order.  Over a sub-chunk of
//    contracting transitions the composed map shrinks (about 0.9^32 at
//    config 2), so its relative error of a few 1e-5 moves the carried state
//    by a few 1e-6 of its size; the re-run of every step is exact fp32.
// A map that is not finite, or does not contract (Frobenius norm above 1:
// its split rounding would reach the later states undamped), is marked
// unusable, and a re-run that would need it replays the earlier sub-chunks
// of its window in fp32 instead.
constexpr int TL_SUB = 4;                          // sub-chunks per window
constexpr int TL_LC = 32;                          // steps per sub-chunk
constexpr int TL_W = TL_SUB * TL_LC;               // steps per window
constexpr int TL_RING = 7;                         // LDS ring slots (one step each)
constexpr int TL_AGG = DS_S * DS_S + DS_S + 4;     // P [64][64], q [64], unusable flag, pad

// s_waitcnt vmcnt(after * NI): the loads of a slot have landed once at most
// the `after` slots issued later are in flight.
template <int NI>
__device__ __forceinline__ void tl_wait_loads(int after) {
  switch (after) {
    case 7: __builtin_amdgcn_s_waitcnt(vmcnt_only(7 * NI)); break;
    case 6: __builtin_amdgcn_s_waitcnt(vmcnt_only(6 * NI)); break;
    case 5: __builtin_amdgcn_s_waitcnt(vmcnt_only(5 * NI)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_only(4 * NI)); break;
    case 3: __builtin_amdgcn_s_waitcnt(vmcnt_only(3 * NI)); break;
    case 2: __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * NI)); break;
    case 1: __builtin_amdgcn_s_waitcnt(vmcnt_only(NI)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_only(0)); break;
  }
}
static_assert(TL_RING - 2 <= 7, "tl_wait_loads covers up to seven slots in flight");

typedef __bf16 tl_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float tl_f32x4_t __attribute__((ext_vector_type(4)));

struct TwoLevelArgs {
  const float* A;
  const float* B;
  const float* H0;
  float* H;
  float* agg;   // [2][batch][TL_SUB - 1][TL_AGG] composed maps, by window parity
  float* hend;  // [2][batch][DS_S] state after a window, by window parity
  int L, batch;
  int w_rerun, w_agg;  // windows re-run / composed by this launch (-1: none)
};

// Float offset of 16-byte chunk `c` of row `r` of an A_t slot.
__device__ __forceinline__ int tl_off(int r, int c) { return 4 * (r * 16 + (c ^ (r & 15))); }

// x = hi + lo in bf16 (round to nearest even both times).
__device__ __forceinline__ void tl_split(const float (&x)[8], tl_bf16x8_t& hi, tl_bf16x8_t& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = (__bf16)x[e];
    hi[e] = h;
    lo[e] = (__bf16)(x[e] - (float)h);
  }
}

// One exact fp32 step: out[row] = A_t[row, :] . h + b_t[row] (four threads a
// row, 16 columns each, DPP quad sum).
__device__ __forceinline__ void tl_exact_step(const float* slot, const float* h, float* out, int row, int part) {
  float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = 4 * part + q;
    const float4 av = *reinterpret_cast<const float4*>(slot + tl_off(row, c));
    const float4 hv = *reinterpret_cast<const float4*>(h + 4 * c);
    p[q] = fmaf(av.x, hv.x, p[q]);
    p[q] = fmaf(av.y, hv.y, p[q]);
    p[q] = fmaf(av.z, hv.z, p[q]);
    p[q] = fmaf(av.w, hv.w, p[q]);
  }
  const float acc = quad_sum((p[0] + p[1]) + (p[2] + p[3]));
  if (part == 0) out[row] = acc + slot[DS_S * DS_S + row];
}

constexpr int TL_CW = 8;                      // compute waves (two per SIMD)
constexpr int TL_LOADERS = 4;                 // loader waves: 16 rows of A_t each, the first also b_t
constexpr int TL_NI = DS_S * DS_S / 4 / 64 / TL_LOADERS;  // A instructions per loader per slot (4)
constexpr int TL_THREADS = (TL_CW + TL_LOADERS) * 64;
static_assert((TL_RING - 2) * (TL_NI + 1) <= 63, "vmcnt holds at most 63");

__global__ __launch_bounds__(TL_THREADS) void dense_twolevel_kernel(TwoLevelArgs a) {
  __shared__ __attribute__((aligned(1024))) float ring_s[TL_RING][DS_SLOT];
  __shared__ __attribute__((aligned(16))) float vec_s[2][DS_S];   // compose: q
  __shared__ __attribute__((aligned(16))) float vecR_s[2][DS_S];  // re-run: h
  // P as B fragments, [buffer][hi/lo][k block][16-column tile][lane]
  __shared__ __attribute__((aligned(16))) tl_bf16x8_t pf_s[2][2][2][4][64];
  __shared__ int bad_s;
  __shared__ float nrm_s[TL_CW];
  float* ring = &ring_s[0][0];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool loader = wave >= TL_CW;
  const bool rowwave = wave < 4;  // the exact steps: four threads a row
  const int seq = blockIdx.x / TL_SUB, j = blockIdx.x % TL_SUB;
  const int L = a.L;
  const float* Aseq = a.A + (size_t)seq * L * DS_S * DS_S;
  const float* bseq = a.B + (size_t)seq * L * DS_S;
  const int row = (tid >> 2) & (DS_S - 1), part = tid & 3;
  const size_t hb = (size_t)a.batch * DS_S;

  // Loader w (wave TL_CW + w) moves A_t rows 16w .. 16w+15 of a slot (TL_NI
  // instructions of four rows), loader 0 also b_t (one instruction, 16 lanes).
  const int lw = loader ? wave - TL_CW : 0;
  const float* asrc[TL_NI];
#pragma unroll
  for (int i = 0; i < TL_NI; ++i) {
    const int c = (lw * TL_NI + i) * 64 + lane;  // LDS chunk of the slot
    const int r = c >> 4, p = c & 15;
    asrc[i] = Aseq + r * DS_S + 4 * (p ^ (r & 15));
  }
  const float* bsrc = bseq + 4 * min(lane, DS_S / 4 - 1);
  // Loads step t's A_t and b_t into ring slot `slot` (loader waves).
  auto issue_step = [&](int slot_i, size_t t) {
    float* slot = ring + slot_i * DS_SLOT;
#pragma unroll
    for (int i = 0; i < TL_NI; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(asrc[i] + t * (DS_S * DS_S)),
                                       (__attribute__((address_space(3))) void*)(slot + 4 * (lw * TL_NI + i) * 64),
                                       16, 0, 0);
    if (lw == 0 && lane < DS_S / 4)
      __builtin_amdgcn_global_load_lds((const void*)(bsrc + t * DS_S),
                                       (__attribute__((address_space(3))) void*)(slot + DS_S * DS_S), 16, 0, 0);
  };
  // The loader waves' wait for the slot whose loads are followed by `after`
  // more slots in flight; the compute waves' LDS writes of the last step
  // complete before the barrier.
  auto step_wait = [&](int after) {
    if (loader) {
      if (lw == 0)
        tl_wait_loads<TL_NI + 1>(after);
      else
        tl_wait_loads<TL_NI>(after);
    } else {
      __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8) | (0xF) | (0x3 << 14));  // lgkmcnt(0)
    }
    asm volatile("s_barrier" ::: "memory");
  };
  // Streams steps ts .. ts+nst-1 through the ring; compute(k, slot) runs on
  // the compute waves once step ts+k has landed, one barrier per step.
  auto stream = [&](int ts, int nst, auto&& compute) {
    if (loader)
      for (int k = 0; k < TL_RING - 1 && k < nst; ++k) issue_step(k % TL_RING, (size_t)(ts + k));
    for (int k = 0; k < nst; ++k) {
      step_wait(min(TL_RING - 2, nst - 1 - k));
      if (loader) {
        if (k + TL_RING - 1 < nst) issue_step((k + TL_RING - 1) % TL_RING, (size_t)(ts + k + TL_RING - 1));
        continue;
      }
      compute(k, ring + (k % TL_RING) * DS_SLOT);
    }
    __syncthreads();
  };

  // ---- the two roles of a launch, each in three parts (start, one step,
  // finish) so that they can share one barrier chain ----
  // Re-run: sub-chunk j of window w_rerun, its steps exactly in fp32 from
  // its entry state.
  const int wr = a.w_rerun;
  const int wr_start = wr * TL_W, wr_end = wr >= 0 ? min(L, wr_start + TL_W) : 0;
  const int tr0 = wr_start + j * TL_LC;
  const int nr = wr >= 0 ? max(0, min(wr_end, tr0 + TL_LC) - tr0) : 0;
  // Compose: the map (P, q) of sub-chunk j < TL_SUB - 1 of window w_agg.
  const int wc = a.w_agg;
  const int tc0 = wc * TL_W + j * TL_LC;
  const int nc = (wc >= 0 && j < TL_SUB - 1) ? max(0, min(min(L, wc * TL_W + TL_W), tc0 + TL_LC) - tc0) : 0;
  float* Hseq = a.H + (size_t)seq * L * DS_S;
  const float* rmaps = a.agg + ((size_t)(wr & 1) * a.batch + seq) * (TL_SUB - 1) * TL_AGG;
  bool rusable = true;  // every map before sub-chunk j of the re-run's window
  if (nr > 0)
    for (int i = 0; i < j; ++i) rusable = rusable && rmaps[(size_t)i * TL_AGG + DS_S * DS_S + DS_S] == 0.0f;
  int curR = 0, curC = 0, pb = 0;
  const int g = lane >> 4, cl = lane & 15;
  // Compute wave cw owns the 16-row tile rt = cw % 4 of the new P and the
  // 16-column tiles 2 (cw / 4) and 2 (cw / 4) + 1.
  const int rt = wave & 3, nt0 = 2 * (wave >> 2);
  tl_f32x4_t pm[2];  // this wave's tile rows of P, column tiles nt0, nt0 + 1

  // Re-run start: the window's entry state carried through the composed
  // maps of sub-chunks 0 .. j-1 (h <- P h + q), or, when one of them is
  // unusable, those sub-chunks replayed exactly (streamed on their own).
  auto rerun_start = [&]() {
    if (tid < DS_S)
      vecR_s[0][tid] = wr == 0 ? (a.H0 ? a.H0[(size_t)seq * DS_S + tid] : 0.0f)
                               : a.hend[(size_t)((wr - 1) & 1) * hb + (size_t)seq * DS_S + tid];
    __syncthreads();
    if (rusable) {
      for (int i = 0; i < j; ++i) {
        if (rowwave) {
          const float* P = rmaps + (size_t)i * TL_AGG;
          const float* h = &vecR_s[curR][0];
          float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 pv = *reinterpret_cast<const float4*>(P + row * DS_S + 16 * part + 4 * q);
            const float4 hv = *reinterpret_cast<const float4*>(h + 16 * part + 4 * q);
            p[q] = fmaf(pv.x, hv.x, p[q]);
            p[q] = fmaf(pv.y, hv.y, p[q]);
            p[q] = fmaf(pv.z, hv.z, p[q]);
            p[q] = fmaf(pv.w, hv.w, p[q]);
          }
          const float acc = quad_sum((p[0] + p[1]) + (p[2] + p[3]));
          if (part == 0) vecR_s[curR ^ 1][row] = acc + P[DS_S * DS_S + row];
        }
        __syncthreads();
        curR ^= 1;
      }
    } else {
      stream(wr_start, tr0 - wr_start, [&](int, const float* slot) {
        if (rowwave) tl_exact_step(slot, vecR_s[curR], vecR_s[curR ^ 1], row, part);
        curR ^= 1;
      });
    }
  };
  auto rerun_step = [&](int k, const float* slot) {
    if (wave == 0 && k > 0) Hseq[(size_t)(tr0 + k - 1) * DS_S + lane] = vecR_s[curR][lane];
    if (rowwave) tl_exact_step(slot, vecR_s[curR], vecR_s[curR ^ 1], row, part);
    curR ^= 1;
  };
  auto rerun_finish = [&]() {  // after a barrier that follows the last step
    if (wave == 0) {
      Hseq[(size_t)(tr0 + nr - 1) * DS_S + lane] = vecR_s[curR][lane];
      if (tr0 + nr == wr_end) a.hend[(size_t)(wr & 1) * hb + (size_t)seq * DS_S + lane] = vecR_s[curR][lane];
    }
  };

  // Compose: P <- A_t P on the matrix cores (both operands split into bf16
  // hi + lo), q <- A_t q + b_t in exact fp32 beside it.
  // This wave's values of P as bf16 halves of B fragments: values r = 0..3
  // of tile nt go to k block rt/2, slots 4 (rt%2) + r.
  auto put_rows = [&](int buf, const tl_f32x4_t (&v)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      __bf16 h[4], l[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        h[r] = (__bf16)v[u][r];
        l[r] = (__bf16)(v[u][r] - (float)h[r]);
      }
      __bf16* ph = reinterpret_cast<__bf16*>(&pf_s[buf][0][rt >> 1][nt0 + u][lane]) + 4 * (rt & 1);
      __bf16* pl = reinterpret_cast<__bf16*>(&pf_s[buf][1][rt >> 1][nt0 + u][lane]) + 4 * (rt & 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) ph[r] = h[r], pl[r] = l[r];
    }
  };
  auto compose_start = [&]() {  // a barrier must follow before the first step
    if (tid < DS_S) vec_s[0][tid] = 0.0f;
    if (tid == 0) bad_s = 0;
    if (!loader) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) pm[u][r] = (16 * rt + 4 * g + r == 16 * (nt0 + u) + cl) ? 1.0f : 0.0f;
      put_rows(0, pm);
    }
  };
  auto compose_step = [&](int, const float* slot) {
    // B fragments of the previous P for this wave's column tiles.
    tl_bf16x8_t bh[2][2], bl[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        bh[u][kb] = pf_s[pb][0][kb][nt0 + u][lane];
        bl[u][kb] = pf_s[pb][1][kb][nt0 + u][lane];
      }
    // A_t fragments of this wave's rows: row 16 rt + l%16, columns
    // 32 kb + 4 g .. +3 and 32 kb + 16 + 4 g .. +3.
    tl_bf16x8_t ah[2], al[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const float4 u = *reinterpret_cast<const float4*>(slot + tl_off(16 * rt + cl, 8 * kb + g));
      const float4 v = *reinterpret_cast<const float4*>(slot + tl_off(16 * rt + cl, 8 * kb + 4 + g));
      const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
      tl_split(x, ah[kb], al[kb]);
    }
    if (rowwave) tl_exact_step(slot, vec_s[curC], vec_s[curC ^ 1], row, part);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      tl_f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[kb], bh[u][kb], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[kb], bl[u][kb], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[kb], bh[u][kb], acc, 0, 0, 0);
      }
      pm[u] = acc;
    }
    put_rows(pb ^ 1, pm);
    pb ^= 1;
    curC ^= 1;
  };
  auto compose_finish = [&]() {  // after a barrier that follows the last step
    bool bad = false;
    float sq = 0.0f;  // this lane's share of |P|_F^2
    if (!loader)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          bad = bad || !(fabsf(pm[u][r]) <= 3.0e38f);
          sq = fmaf(pm[u][r], pm[u][r], sq);
        }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sq += __shfl_xor(sq, off, 64);
    if (!loader && lane == 0) nrm_s[wave] = sq;
    if (!loader && (bad || (tid < DS_S && !(fabsf(vec_s[curC][tid]) <= 3.0e38f)))) atomicOr(&bad_s, 1);
    __syncthreads();
    float* out = a.agg + (((size_t)(wc & 1) * a.batch + seq) * (TL_SUB - 1) + j) * TL_AGG;
    if (!loader) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          out[(16 * rt + 4 * g + r) * DS_S + 16 * (nt0 + u) + cl] = pm[u][r];
      if (tid < DS_S) out[DS_S * DS_S + tid] = vec_s[curC][tid];
      if (tid == 0) {
        // A map that does not contract (|P|_F > 1) would carry its split
        // rounding undamped into the states after it: replayed instead.
        float f2 = 0.0f;
        for (int w2 = 0; w2 < TL_CW; ++w2) f2 += nrm_s[w2];
        out[DS_S * DS_S + DS_S] = (bad_s || !(f2 <= 1.0f)) ? 1.0f : 0.0f;
      }
    }
    __syncthreads();
  };

  if (nr > 0 && !rusable) {
    // A map the re-run needs is unusable: the re-run replays and streams
    // on its own, then the compose streams.
    rerun_start();
    stream(tr0, nr, rerun_step);
    rerun_finish();
    __syncthreads();
    if (nc > 0) {
      compose_start();
      __syncthreads();
      stream(tc0, nc, compose_step);
      compose_finish();
    }
    return;
  }

  // Both roles in one barrier chain: step k runs compose step k (8 waves,
  // matrix cores) and re-run step k (4 waves, exact fp32) on two ring slots,
  // so a launch costs max(nc, nr) dependent steps instead of nc + nr.  The
  // ring holds loads in order: compose step k's slot before re-run step k's.
  if (nr > 0) rerun_start();
  if (nc > 0) compose_start();
  __syncthreads();
  const int K = max(nc, nr), n_load = nc + nr;
  auto before = [&](int k) { return min(k, nc) + min(k, nr); };  // loads of the steps before k
  // The loaders' cursor: the next load is step lk's compose (lrole 0) or
  // re-run (lrole 1) slot.
  int issued = 0, lk = 0, lrole = nc > 0 ? 0 : 1;
  auto issue_next = [&]() {
    issue_step(issued % TL_RING, (size_t)(lrole == 0 ? tc0 + lk : tr0 + lk));
    ++issued;
    if (lrole == 0 && lk < nr) {
      lrole = 1;
    } else {
      ++lk;
      lrole = lk < nc ? 0 : 1;
    }
  };
  if (loader)
    while (issued < min(n_load, TL_RING)) issue_next();
  for (int k = 0; k < K; ++k) {
    // This step's loads are complete once at most the loads issued after
    // them are in flight (at most TL_RING - 1 slots).
    step_wait(issued - before(k + 1));
    if (loader) {
      // The slots of the steps before k are free.
      const int lim = min(n_load, before(k) + TL_RING);
      while (issued < lim) issue_next();
      continue;
    }
    const int p0 = before(k);
    if (k < nc) compose_step(k, ring + (p0 % TL_RING) * DS_SLOT);
    if (k < nr) rerun_step(k, ring + ((p0 + (k < nc ? 1 : 0)) % TL_RING) * DS_SLOT);
  }
  __syncthreads();
  if (nr > 0) rerun_finish();
  if (nc > 0) compose_finish();
}

size_t dense_scan_scratch_bytes(int batch, int L, int s) {
  if (s != DS_S || L < 2 * TL_W) return 0;
  return ((size_t)2 * batch * (TL_SUB - 1) * TL_AGG + (size_t)2 * batch * DS_S) * sizeof(float);
}

static bool ring_fits(const float* A, const float* B, int s) {
  return s == DS_S && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0;
}

Status init_dense_scan_attributes() { return Status::Ok(); }

Status launch_dense_scan(hipStream_t stream, const float* A, const float* B, const float* H0, float* H,
                         int batch, int L, int s, void* scratch, size_t scratch_bytes) {
  if (batch <= 0 || L <= 0 || s <= 0) return Status::Invalid("dense scan: dimensions must be positive");
  const size_t need = dense_scan_scratch_bytes(batch, L, s);
  if (need && ring_fits(A, B, s) && scratch && scratch_bytes >= need) {
    // Two-level: launch l composes window l and re-runs window l - 1.
    TwoLevelArgs ta;
    ta.A = A;
    ta.B = B;
    ta.H0 = H0;
    ta.H = H;
    ta.agg = static_cast<float*>(scratch);
    ta.hend = ta.agg + (size_t)2 * batch * (TL_SUB - 1) * TL_AGG;
    ta.L = L;
    ta.batch = batch;
    const int nw = (L + TL_W - 1) / TL_W;
    const long blocks = (long)batch * TL_SUB;
    if (blocks > INT32_MAX) return Status::Invalid("dense scan: too many workgroups");
    for (int l = 0; l <= nw; ++l) {
      ta.w_agg = l < nw ? l : -1;
      ta.w_rerun = l - 1;
      dense_twolevel_kernel<<<(unsigned)blocks, TL_THREADS, 0, stream>>>(ta);
      PSSA_LAUNCH_CHECK("dense_twolevel");
    }
    return Status::Ok();
  }
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

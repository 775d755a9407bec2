// Poincare-ball memory read for gfx950.
//
// One wave per query, one lane per group of slots.  Everything that decides
// which slots are read -- the projection into the ball, the squared norms and
// the distances -- is computed in f64 in the reference's own order
// (sequential sums, no fused multiply-add, Rust's asinh formula), so the f32
// distances, and with them the top-k indices, agree with the reference
// (src/memory.rs:181-262).  The softmax weights and the value mix are fp32.
#include "memory.h"

#include <algorithm>
#include <cfloat>

namespace pssa {

__device__ __forceinline__ double rust_asinh(double x) {
  // Rust std f64::asinh: ln_1p(|x| + |x| / (hypot(1, 1/|x|) + 1/|x|)), sign of x.
  const double ax = fabs(x);
  const double ix = 1.0 / ax;
  return copysign(log1p(ax + (ax / (hypot(1.0, ix) + ix))), x);
}

// Sequential f64 sum of squares (squared_norm_f64, src/memory.rs:188-192).
__device__ __forceinline__ double sumsq_f64(const float* p, int n) {
#pragma clang fp contract(off)
  double acc = 0.0;
  for (int i = 0; i < n; ++i) {
    const double v = (double)p[i];
    acc = acc + v * v;
  }
  return acc;
}

__device__ __forceinline__ float bank_norm_sq(const float* p, int n) {
  const double v = sumsq_f64(p, n);
  if (v < 1.0 && (float)v == 1.0f) return __uint_as_float(0x3f7fffffu);
  return (float)v;
}

// poincare_distance (src/memory.rs:242-262).
__device__ __forceinline__ float poincare_dist(const float* __restrict__ q, float q_sq,
                                               const float* __restrict__ key, float k_sq, int n) {
#pragma clang fp contract(off)
  double sq = 0.0;
  int i = 0;
  if (((uintptr_t)key & 15) == 0) {
    for (; i + 4 <= n; i += 4) {
      const float4 kv = *reinterpret_cast<const float4*>(key + i);
      double t;
      t = (double)q[i] - (double)kv.x;
      sq = sq + t * t;
      t = (double)q[i + 1] - (double)kv.y;
      sq = sq + t * t;
      t = (double)q[i + 2] - (double)kv.z;
      sq = sq + t * t;
      t = (double)q[i + 3] - (double)kv.w;
      sq = sq + t * t;
    }
  }
  for (; i < n; ++i) {
    const double t = (double)q[i] - (double)key[i];
    sq = sq + t * t;
  }
  const double den = (1.0 - (double)q_sq) * (1.0 - (double)k_sq);
  return (float)(2.0 * rust_asinh(sqrt(sq / den)));
}

// Orders this wave's LDS writes before its subsequent LDS reads.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, 64);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ uint16_t bf16_bits(float f) { return bf16_bits_dev(f); }

__device__ __forceinline__ void put_weight(const RetrieveArgs& a, int n, int s, float w) {
  const size_t o = (size_t)n * a.capacity + s;
  if (a.weights) a.weights[o] = w;
  if (a.weights16) a.weights16[o] = bf16_bits(w);
}

constexpr double kMaxRadius = 1.0 - 8.0 * (double)FLT_EPSILON;  // src/memory.rs:173

// Hybrid read recency factor of slot s for query row n (src/memory.rs:632-633):
// (float)exp(age * ln(lam)) in f64, the age saturating at 2^64 - 1.
__device__ __forceinline__ float hybrid_decay(const RetrieveArgs& a, int s, int n) {
  unsigned long long age = a.hage ? a.hage[s] : 0ull;
  const unsigned long long add =
      a.age_base + (a.age_T > 0 ? (unsigned long long)(n % a.age_T) + 1ull : 0ull);
  age = age > ~0ull - add ? ~0ull : age + add;
  return (float)exp((double)age * a.log_lam);
}

// Several waves per query: each computes the distances of every
// RETRIEVE_WPQ-th 64-slot block (the per-slot sums are the only long chains,
// and a 512-query prefill would otherwise leave half the SIMDs idle); the
// first wave then selects, weights and reads out alone, as a one-wave read
// would.  The waves of a query meet at workgroup barriers, so every wave of
// a workgroup runs the same number of iterations.
#ifndef RETRIEVE_QPB
#define RETRIEVE_QPB 2
#endif
constexpr int RETRIEVE_WPQ = 4 / RETRIEVE_QPB;  // waves per query (4-wave workgroups)
__global__ __launch_bounds__(256) void retrieve_kernel(RetrieveArgs a) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pair = wave / RETRIEVE_WPQ, half = wave % RETRIEVE_WPQ;
  const int dk_pad = (a.dk + 3) & ~3;
  float* sq = smem + pair * (dk_pad + a.capacity);  // this query's projection, then distances
  float* sdist = sq + dk_pad;
  __shared__ uint32_t ssel[RETRIEVE_QPB][kMaxTopK];
  __shared__ float spart[RETRIEVE_QPB][RETRIEVE_WPQ];
  const int cnt = a.count_dev ? a.count_dev[0] : a.count;

  for (int n0 = blockIdx.x * RETRIEVE_QPB; n0 < a.n; n0 += gridDim.x * RETRIEVE_QPB) {
    const int n = n0 + pair;
    const bool live = n < a.n;
    if (live && half == 0) {
      const float* qrow = a.q + (size_t)n * a.ld_q;
      for (int i = lane; i < a.dk; i += 64) sq[i] = qrow[i];
      wave_sync();
      // ---- diffeomorphic_project (src/memory.rs:194-211) ----
      if (a.project) {
        const double r = sqrt(sumsq_f64(sq, a.dk));
        const double scale = r == 0.0 ? 1.0 : fmin(r / (1.0 + r), kMaxRadius) / r;
        wave_sync();
        for (int i = lane; i < a.dk; i += 64) sq[i] = (float)((double)sq[i] * scale);
        if (a.q_norm && lane == 0) a.q_norm[n] = (float)fmin(r, (double)FLT_MAX);
        wave_sync();
      }
      if (a.q_pnc)
        for (int i = lane; i < a.dk; i += 64) a.q_pnc[(size_t)n * a.dk + i] = sq[i];
    }
    __syncthreads();
    // ---- distances: 64-slot blocks dealt round the query's waves ----
    float q_sq = 0.0f;
    if (live && cnt > 0) {
      q_sq = bank_norm_sq(sq, a.dk);
      float local_min = FLT_MAX;
      for (int s = lane + 64 * half; s < cnt; s += 64 * RETRIEVE_WPQ) {
        const float dist = poincare_dist(sq, q_sq, a.keys + (size_t)s * a.dk, a.norm_sq[s], a.dk);
        sdist[s] = dist;
        local_min = fminf(local_min, dist);
      }
      const float wmin = wave_min(local_min);
      if (lane == 0) spart[pair][half] = wmin;
    }
    __syncthreads();
    if (live && half == 0) {
      if (cnt == 0) {
        for (int s = lane; s < a.capacity; s += 64) put_weight(a, n, s, 0.0f);
        if (a.out_val)
          for (int j = lane; j < a.dv; j += 64) a.out_val[(size_t)n * a.dv + j] = 0.0f;
        if (a.out_min && lane == 0) a.out_min[n] = 0.0f;
        if (a.out_idx)
          for (int r = lane; r < a.top_k; r += 64) a.out_idx[(size_t)n * a.top_k + r] = 0xFFFFFFFFu;
      } else {
        float min_dist = spart[pair][0];
        for (int h = 1; h < RETRIEVE_WPQ; ++h) min_dist = fminf(min_dist, spart[pair][h]);
        if (a.out_min && lane == 0) a.out_min[n] = min_dist;

        if (a.top_k > 0 && a.top_k < cnt) {
          // ---- exact top-k by (distance bits, slot) (src/memory.rs:380-392) ----
          const int k = a.top_k;
          for (int r = 0; r < k; ++r) {
            unsigned long long best = ~0ull;
            for (int s = lane; s < cnt; s += 64) {
              const uint32_t bits = __float_as_uint(sdist[s]);
              const unsigned long long key = ((unsigned long long)bits << 32) | (unsigned)s;
              bool taken = false;
              for (int p = 0; p < r; ++p) taken |= ssel[pair][p] == (uint32_t)s;
              if (!taken && key < best) best = key;
            }
            best = wave_min_u64(best);
            if (lane == 0) ssel[pair][r] = (uint32_t)(best & 0xFFFFFFFFu);
            wave_sync();
          }
          if (lane == 0) {  // ascending slot order
            for (int x = 1; x < k; ++x) {
              const uint32_t v = ssel[pair][x];
              int y = x - 1;
              while (y >= 0 && ssel[pair][y] > v) {
                ssel[pair][y + 1] = ssel[pair][y];
                --y;
              }
              ssel[pair][y + 1] = v;
            }
          }
          wave_sync();
          // Hybrid read: (e * gate) * decay per live slot, unless every live
          // weight is zero (then the plain softmax, src/memory.rs:640-650).
          auto hyb_w = [&](int s, float e) { return (e * a.hgate[s]) * hybrid_decay(a, s, n); };
          bool hyb = a.hgate != nullptr;
          float sum = 0.0f;
          if (hyb) {
            for (int r = 0; r < k; ++r) {
              const int s = ssel[pair][r];
              sum += hyb_w(s, expf((min_dist - sdist[s]) / a.tau));
            }
            hyb = sum != 0.0f;
          }
          if (!hyb) {
            sum = 0.0f;
            for (int r = 0; r < k; ++r) sum += expf((min_dist - sdist[ssel[pair][r]]) / a.tau);
          }
          auto weight_of = [&](int s) {
            const float e = expf((min_dist - sdist[s]) / a.tau);
            return (hyb ? hyb_w(s, e) : e) / sum;
          };
          if (a.weights || a.weights16) {
            for (int s = lane; s < a.capacity; s += 64) {
              bool chosen = false;
              for (int r = 0; r < k; ++r) chosen |= ssel[pair][r] == (uint32_t)s;
              put_weight(a, n, s, chosen ? weight_of(s) : 0.0f);
            }
          }
          if (a.out_idx)
            for (int r = lane; r < k; r += 64) a.out_idx[(size_t)n * k + r] = ssel[pair][r];
          if (a.out_val) {
            for (int j = lane; j < a.dv; j += 64) {
#pragma clang fp contract(off)
              float acc = 0.0f;
              for (int r = 0; r < k; ++r) {
                const uint32_t s = ssel[pair][r];
                const float w = weight_of((int)s);
                acc = acc + w * a.values[(size_t)s * a.dv + j];
              }
              a.out_val[(size_t)n * a.dv + j] = acc;
            }
          }
        } else {
          // ---- full soft read (src/memory.rs:409-425); hybrid: every slot live ----
          float part = 0.0f, part_h = 0.0f;
          for (int s = lane; s < cnt; s += 64) {
            const float e = expf((min_dist - sdist[s]) / a.tau);
            sdist[s] = e;
            part += e;
            if (a.hgate) part_h += (e * a.hgate[s]) * hybrid_decay(a, s, n);
          }
          const float sum_p = wave_sum(part);
          const float sum_h = a.hgate ? wave_sum(part_h) : 0.0f;
          const bool hyb = a.hgate && sum_h != 0.0f;
          const float sum = hyb ? sum_h : sum_p;
          wave_sync();
          for (int s = lane; s < a.capacity; s += 64) {
            float w = 0.0f;
            if (s < cnt) w = (hyb ? (sdist[s] * a.hgate[s]) * hybrid_decay(a, s, n) : sdist[s]) / sum;
            if (s < cnt) sdist[s] = w;
            put_weight(a, n, s, w);
          }
          wave_sync();
          if (a.out_val) {
            for (int j = lane; j < a.dv; j += 64) {
              float acc = 0.0f;
              for (int s = 0; s < cnt; ++s) acc = fmaf(sdist[s], a.values[(size_t)s * a.dv + j], acc);
              a.out_val[(size_t)n * a.dv + j] = acc;
            }
          }
          if (a.out_idx)
            for (int r = lane; r < a.top_k; r += 64)
              a.out_idx[(size_t)n * a.top_k + r] = r < cnt ? (uint32_t)r : 0xFFFFFFFFu;
        }
      }
    }
    // The next query's projection and distances overwrite this one's.
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Full soft read for the model path (no top-k, small banks).  The bank's keys
// stay in LDS for the whole launch, transposed so that lane j of a wave reads
// slot j + 64q of key dimension i at consecutive addresses, next to
// 1/(1 - |k|^2) and the exact key norm sum_i k_i^2 per slot in f64.
//
// Each wave owns a contiguous range of queries.  Their projections follow the
// reference's sequential f64 order exactly (src/memory.rs:181-211), one query
// per lane, so the two dependent 32-step chains are paid once per 64 queries
// rather than once per query.  The squared distance of QG queries at a time
// is then |q|^2 + |k|^2 - 2 q.k with every term in f64: the products of two
// f32 values are exact in f64 and each sum has relative error below
// d_key * 2^-53, so the absolute error of |q - k|^2 stays near 1e-14 (the
// distance of even coincident points moves by < 1e-6).  One key element read
// from LDS and converted once serves QG queries' fused multiply-adds; the
// query values enter them as wave-uniform f64 operands (readlane from the
// lane that holds that dimension).
//
// Only the soft weights depend on the distances (no ranking), so the rest is
// evaluated in f32 with the hardware square root, log2 and exp2:
//   d = 2 asinh(sqrt(x)) = 2 ln(sqrt(x) + sqrt(1 + x)) = 2 ln2 * l,
//   l = log2(sqrt(x) + sqrt(1 + x)),  x = |q-k|^2 / ((1-|q|^2)(1-|k|^2)),
//   exp((d_min - d) / tau) = exp2((l_min - l) * 2 / tau),
// which moves a weight by a few 1e-6 relative, far inside the 1e-4 parity
// gate; the softmax sums over slots run as wave reductions and every weight
// is scaled by one reciprocal of the sum.  Writes the [n, capacity] weights;
// the value readout is a GEMM.  A query's arithmetic does not depend on its
// position in the batch or on QG, so one token at a time and a whole prefill
// give the same bits.
constexpr int SOFT_SPL = 8;            // slots per lane: capacity <= 512
constexpr int SOFT_MAX_KEYS = 16384;   // dk * capacity floats held in LDS (64 KiB)
constexpr int SOFT_MAX_DK = 64;
constexpr int SOFT_WAVES = 8;
#ifndef SOFT_WAVES_FEW
#define SOFT_WAVES_FEW 4               // waves per workgroup for few queries (measured: 1, 2, 8 slower)
#endif
constexpr int SOFT_FEW_QUERIES = 2048;
constexpr int SOFT_QG = 4;             // queries sharing one pass over the keys

// Slots per lane for a bank of `cap` slots (a power of two up to SOFT_SPL).
__host__ __device__ __forceinline__ int soft_spl(int cap) {
  return cap <= 64 ? 1 : cap <= 128 ? 2 : cap <= 256 ? 4 : 8;
}
// keyT rows hold every slot a lane reads (64 * spl, so no read needs a
// clamp) and have an odd pitch: the transposing stores of a wave
// (consecutive key dimensions) and the slot reads (consecutive slots) both
// fall in distinct banks.
__host__ __device__ __forceinline__ int soft_pitch(int cap) { return 64 * soft_spl(cap) + 1; }
__host__ __device__ __forceinline__ size_t soft_keys_floats(int dk, int cap) {
  return (((size_t)dk * soft_pitch(cap) + 1) & ~(size_t)1);  // keep the f64 arrays 8-byte aligned
}
// Dynamic LDS: keyT, then 1/(1-|k|^2) and |k|^2 (f64), then each wave's QG
// projected queries (f32).
static size_t soft_read_lds(int dk, int cap, int qg, int nwv) {
  return soft_keys_floats(dk, cap) * sizeof(float) + 2 * (size_t)cap * sizeof(double) +
         (size_t)nwv * qg * dk * sizeof(float);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// The fused query product's LDS (after the soft read's own): each wave's raw
// query row (32 floats), then the bf16 panels, 16-byte aligned: 32 weight
// rows (clamped past d_key) and the workgroup's query rows, qk elements
// each, chunk c of panel row r at position c ^ (r & 15).
constexpr int SOFT_QP_ROWS = 32;
static size_t soft_qp_lds(int qk, int nwv) {
  return (size_t)nwv * 32 * sizeof(float) + 16 + (size_t)(SOFT_QP_ROWS + nwv) * qk * sizeof(uint16_t);
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)b, l);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

template <int QG, int SPL, bool HYB, int NWV, bool QP = false>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(4))) void soft_read_kernel(
    RetrieveArgs a) {
  extern __shared__ float smem[];
  const int cap = a.capacity, dk = a.dk, cnt = a.count_dev ? a.count_dev[0] : a.count;
  if constexpr (QP) __builtin_amdgcn_s_setprio(2);  // a decode-step product, as gemm_few_kernel
  float* keyT = smem;                                                  // [dk][kp]
  const int kp = soft_pitch(cap);
  double* rk = reinterpret_cast<double*>(smem + soft_keys_floats(dk, cap));  // [cap]
  double* kk = rk + cap;                                               // [cap]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* pw = reinterpret_cast<float*>(kk + cap) + wave * QG * dk;     // [QG][dk]
  const int nw = gridDim.x * NWV;
  const int per = (a.n + nw - 1) / nw;
  const int qb = (blockIdx.x * NWV + wave) * per;
  const int qe = min(a.n, qb + per);
  // One query per wave (a decode step): its row loads now, across the lanes,
  // so the round trip overlaps the key staging below.
  const bool one = QG == 1 && per == 1;
  float qlane = 0.0f;
  // Fused query product (QP, one query per wave): the weight panel and the
  // workgroup's query rows go to LDS by direct loads issued first; wave 0
  // forms the products while the other waves finish the key terms.
  static_assert(!QP || (QG == 1 && NWV > 1), "the fused query product serves one query per wave");
  const size_t pq_off = soft_keys_floats(dk, cap) + 4 * (size_t)cap + (size_t)NWV * QG * dk;
  float* pq = smem + pq_off;                                                         // [NWV][32]
  uint16_t* sq = reinterpret_cast<uint16_t*>(smem + ((pq_off + NWV * 32 + 3) & ~(size_t)3));
  float qx[16];
  if constexpr (QP) {
    const int cpr = a.qk / 8;                     // 16-byte chunks per panel row
    const int n_ins = (SOFT_QP_ROWS + NWV) * cpr / 64;
    for (int ins = wave; ins < n_ins; ins += NWV) {
      const int e = ins * 64 + lane, r = e / cpr, c = (e - r * cpr) ^ (r & 15);
      const uint16_t* src = r < SOFT_QP_ROWS
                                ? a.qw + (size_t)min(r, dk - 1) * a.qk + c * 8
                                : a.qa + (size_t)min((int)blockIdx.x * NWV + r - SOFT_QP_ROWS, a.n - 1) * a.ld_qa + c * 8;
      __builtin_amdgcn_global_load_lds((const void*)src,
                                       (__attribute__((address_space(3))) void*)(sq + (size_t)ins * 512), 16, 0, 0);
    }
    // The addend of the rows wave 0's lanes will hold (see below).
    const int l32 = lane & 31, qrow = min((int)blockIdx.x * NWV + min(l32, NWV - 1), a.n - 1);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      qx[i] = a.qaux[(size_t)qrow * a.ld_qaux + min(8 * (i / 4) + 4 * (lane >> 5) + i % 4, dk - 1)];
  } else {
    if (one && qb < qe) qlane = a.q[(size_t)qb * a.ld_q + min(lane, dk - 1)];
  }
  // Coalesced reads of the row-major keys, transposed on the way into LDS;
  // KU loads per thread are issued before their stores (a four-wave
  // workgroup holds a 512 x 32 bank in one round of sixteen).
  constexpr int KU = NWV <= 4 ? 16 : 8;
  if (dk % 4 == 0 && ((uintptr_t)a.keys & 15) == 0) {
    const int nv = cnt * dk / 4;
    for (int e0 = tid; e0 < nv; e0 += KU * 64 * NWV) {
      float4 v[KU];
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int e = e0 + u * 64 * NWV;
        v[u] = e < nv ? reinterpret_cast<const float4*>(a.keys)[e] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int e = e0 + u * 64 * NWV;
        if (e < nv) {
          const int sl = (4 * e) / dk, i = 4 * e - sl * dk;
          keyT[i * kp + sl] = v[u].x;
          keyT[(i + 1) * kp + sl] = v[u].y;
          keyT[(i + 2) * kp + sl] = v[u].z;
          keyT[(i + 3) * kp + sl] = v[u].w;
        }
      }
    }
  } else {
    for (int e = tid; e < cnt * dk; e += 64 * NWV) {
      const int sl = e / dk, i = e - sl * dk;
      keyT[i * kp + sl] = a.keys[e];
    }
  }
  if constexpr (QP) __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // this wave's panel loads
  __syncthreads();
  if (!QP || wave > 0) {
    const int t0 = QP ? tid - 64 : tid, step = QP ? 64 * (NWV - 1) : 64 * NWV;
    for (int sl = t0; sl < cnt; sl += step) {
      rk[sl] = 1.0 / (1.0 - (double)a.norm_sq[sl]);
      double s2 = 0.0;
      for (int i = 0; i < dk; ++i) {
        const double kv = keyT[i * kp + sl];
        s2 = fma(kv, kv, s2);
      }
      kk[sl] = s2;
    }
  }
  if constexpr (QP) {
    if (wave == 0) {
      // q = qa qw^T + qaux for the workgroup's NWV rows: one 32 x 32 tile
      // whose token rows are those rows (lane l32 reads row min(l32, NWV-1)),
      // K in 16-wide steps in increasing order on v_mfma_f32_32x32x16_bf16
      // with the weights as the first operand, as in the tiled GEMMs; lane
      // l32 < NWV then holds row l32's columns 8*(i/4) + 4*(lane/32) + i%4.
      const int half = lane >> 5, l32 = lane & 31, ra = SOFT_QP_ROWS + min(l32, NWV - 1);
      const uint16_t* wrow = sq + (size_t)l32 * a.qk;
      const uint16_t* arow = sq + (size_t)ra * a.qk;
      const int sw = l32 & 15, sa = ra & 15;
      f32x16_t acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
      for (int k0 = 0; k0 < a.qk; k0 += 64) {
        bf16x8_t fa[4], fb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = k0 / 8 + 2 * q + half;
          fb[q] = *reinterpret_cast<const bf16x8_t*>(wrow + (c ^ sw) * 8);
          fa[q] = *reinterpret_cast<const bf16x8_t*>(arow + (c ^ sa) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[q], fa[q], acc, 0, 0, 0);
      }
      if (l32 < NWV) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int col = 8 * (i / 4) + 4 * half + i % 4;
          if (col < dk) pq[l32 * 32 + col] = acc[i] + qx[i];  // the ADD_AUX epilogue's sum
        }
      }
    }
  }
  __syncthreads();
  if constexpr (QP) {
    if (one && qb < qe) qlane = pq[wave * 32 + min(lane, dk - 1)];
  }

  const float c2 = 2.0f / a.tau;

  for (int c0 = qb; c0 < qe; c0 += 64) {
    const int na = min(64, qe - c0);
    // ---- projection, one query per lane (src/memory.rs:181-211) ----
    double scale = 1.0, qs = 0.0, rq = 1.0;
    if (one) {
#pragma clang fp contract(off)
      // The wave's one query, held across the lanes: the same sequential
      // f64 sums, every lane reading the values in order.
      double r2 = 0.0;
      for (int i = 0; i < dk; ++i) {
        const double v = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(qlane), i));
        r2 = r2 + v * v;
      }
      const double r = sqrt(r2);
      scale = r == 0.0 ? 1.0 : fmin(r / (1.0 + r), kMaxRadius) / r;
      for (int i = 0; i < dk; ++i) {
        const double v = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(qlane), i));
        const double pv = (double)(float)(v * scale);
        qs = qs + pv * pv;
      }
      float q_sq = (float)qs;
      if (qs < 1.0 && q_sq == 1.0f) q_sq = __uint_as_float(0x3f7fffffu);
      rq = 1.0 / (1.0 - (double)q_sq);
    } else if (lane < na) {
#pragma clang fp contract(off)
      const float* qrow = a.q + (size_t)(c0 + lane) * a.ld_q;
      // Sixteen loads in flight before the dependent sums (the sums keep the
      // reference's order).  The loads read clamped in-range addresses and
      // the sums skip the columns past d_key: a load under a per-element
      // guard ended its block with a full wait, one round trip per element.
      double r2 = 0.0;
      for (int i0 = 0; i0 < dk; i0 += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = qrow[min(i0 + k, dk - 1)];
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (i0 + k < dk) r2 = r2 + (double)v[k] * (double)v[k];
      }
      const double r = sqrt(r2);
      scale = r == 0.0 ? 1.0 : fmin(r / (1.0 + r), kMaxRadius) / r;
      for (int i0 = 0; i0 < dk; i0 += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = qrow[min(i0 + k, dk - 1)];
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (i0 + k < dk) {
            const double pv = (double)(float)((double)v[k] * scale);
            qs = qs + pv * pv;
          }
      }
      float q_sq = (float)qs;
      if (qs < 1.0 && q_sq == 1.0f) q_sq = __uint_as_float(0x3f7fffffu);
      rq = 1.0 / (1.0 - (double)q_sq);
    }

    for (int g0 = 0; g0 < na; g0 += QG) {
      const int ng = min(QG, na - g0);
      // Projected queries of this group into LDS (and the q_pnc tap).
      // The group's query values load first, unguarded at a clamped column,
      // and are scaled by every lane; only the stores are guarded (a load
      // used only under `lane < dk` was sunk into that block and waited
      // there, one round trip per query).
      float qvg[QG];
      if (one) {
        qvg[0] = qlane;
      } else {
#pragma unroll
        for (int g = 0; g < QG; ++g)
          qvg[g] = a.q[(size_t)(c0 + (g < ng ? g0 + g : g0)) * a.ld_q + min(lane, dk - 1)];
      }
      // Lane i keeps dimension i of each projected query, widened to f64;
      // the products take it as a wave-uniform operand by readlane (no LDS
      // round trip per query and dimension).
      double pvd[QG];
#pragma unroll
      for (int g = 0; g < QG; ++g) {
        const int src = g < ng ? g0 + g : g0;
        const float pv = (float)((double)qvg[g] * (one ? scale : readlane_f64(scale, src)));
        pvd[g] = (double)pv;
        if (lane < dk && a.q_pnc && g < ng) a.q_pnc[(size_t)(c0 + src) * dk + lane] = pv;
      }
      double dot[QG][SPL];
#pragma unroll
      for (int g = 0; g < QG; ++g)
#pragma unroll
        for (int j = 0; j < SPL; ++j) dot[g][j] = 0.0;
      // Slots >= count read whatever that part of keyT holds; their results
      // are discarded below.
      for (int i = 0; i < dk; ++i) {
        const float* kr = keyT + i * kp + lane;
        double kv[SPL];
#pragma unroll
        for (int j = 0; j < SPL; ++j) kv[j] = (double)kr[64 * j];
#pragma unroll
        for (int g = 0; g < QG; ++g) {
          const double pg = readlane_f64(pvd[g], i);
#pragma unroll
          for (int j = 0; j < SPL; ++j) dot[g][j] = fma(pg, kv[j], dot[g][j]);
        }
      }
#pragma unroll
      for (int g = 0; g < QG; ++g) {
        if (g >= ng) break;
        const int n = c0 + g0 + g;
        const double qs_g = readlane_f64(qs, g0 + g), rq_g = readlane_f64(rq, g0 + g);
        float l[SPL];
        float lm = FLT_MAX;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          const int sl = lane + 64 * j;
          l[j] = 0.0f;
          if (sl < cnt) {
            const double sq = fmax(fma(-2.0, dot[g][j], qs_g + kk[sl]), 0.0);
            const float x = (float)((sq * rq_g) * rk[sl]);
            const float u = __builtin_amdgcn_sqrtf(x) + __builtin_amdgcn_sqrtf(1.0f + x);
            l[j] = __builtin_amdgcn_logf(u);
            lm = fminf(lm, l[j]);
          }
        }
        const float lmin = wave_min(lm);
        float e[SPL];
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          const int sl = lane + 64 * j;
          e[j] = sl < cnt ? __builtin_amdgcn_exp2f((lmin - l[j]) * c2) : 0.0f;
          part += e[j];
        }
        float sum = wave_sum(part);
        if constexpr (HYB) {  // hybrid read: (e * gate) * decay unless all are zero
          float eh[SPL];
          float part_h = 0.0f;
#pragma unroll
          for (int j = 0; j < SPL; ++j) {
            const int sl = lane + 64 * j;
            eh[j] = sl < cnt ? (e[j] * a.hgate[sl]) * hybrid_decay(a, sl, n) : 0.0f;
            part_h += eh[j];
          }
          const float sum_h = wave_sum(part_h);
          if (sum_h != 0.0f) {
#pragma unroll
            for (int j = 0; j < SPL; ++j) e[j] = eh[j];
            sum = sum_h;
          }
        }
        const float inv = 1.0f / sum;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          const int sl = lane + 64 * j;
          if (sl < cap) put_weight(a, n, sl, sl < cnt ? e[j] * inv : 0.0f);
        }
      }
      wave_sync();
    }
  }
}

// ---------------------------------------------------------------------------
// Exact top-k read for wide keys: the search is pruned on the matrix cores
// and decided in the reference's own f64 arithmetic.
//
// 1. ranked_dot_kernel: dot products q.k for all queries x occupied slots
//    from bf16 MFMAs on split operands, x = x_hi + x_lo (x_hi = bf16(x),
//    x_lo = bf16(x - x_hi), |x - x_hi - x_lo| <= 2^-18 |x|), summing
//    hi*hi + lo*hi + hi*lo in fp32.  Their error is at most
//    RK_DOT_ERR * |q| |k| (split remainder ~3 * 2^-18 plus fp32 accumulation
//    of 3 * d_key products, ~(3 d_key + 48) * 2^-24 for d_key <= 1024, both
//    doubled for margin).
// 2. ranked_pick_kernel, per query: z_s = |q - k_s|^2 / (1 - |k_s|^2) orders
//    the slots exactly like the reference's distance (2 asinh(sqrt(z_s /
//    (1 - |q|^2))) is monotone in z_s; the f32 rounding of the distance can
//    only merge neighbours).  From |q - k|^2 = |q|^2 + |k|^2 - 2 q.k the bound
//    gives an interval [L_s, U_s] around z_s.  T is the top_k-th smallest of
//    the 64 per-lane minima of U (each lane holds every 64th slot), so at
//    least top_k slots have z <= T, and every slot of the exact top_k by
//    (distance bits, slot) has L_s <= T (1 + RK_TIE) (the slack covers slots
//    whose larger z rounds to the same f32 distance).  Those are the
//    candidates -- about top_k + 1 per query at the benchmark shape.
// 3. The candidates' distances are recomputed exactly as in
//    poincare_distance (sequential f64 sum, no fused multiply-add, Rust's
//    asinh), one job per thread, together with one sequential |q|^2 chain
//    per query (squared_norm).  The workgroup's query rows and the distinct
//    candidate keys pass through LDS in 32-dimension chunks.
// 4. Selection by (distance bits, slot) through ranks counted over the
//    candidates, softmax over the selected distances, and the value readout
//    in ascending slot order, as retrieve_soft_into (src/memory.rs:344-407).
constexpr int RK_SLOTS = 512;            // occupied slots handled
constexpr int RK_BK = 32;                // key dimensions per slab and per exact chunk
constexpr int RK_MAX_DK = 1024;
constexpr int RK_THREADS = 512;
constexpr int RK_TQ = 256, RK_TS = 256;  // dot tile: queries x slots
constexpr int RK_CHUNK = 32768;          // queries per dot/pick pass (scratch rows)
constexpr double RK_DOT_ERR = 4e-4;
constexpr double RK_TIE = 1.0 / 4096.0;

__device__ __forceinline__ int rk_swizzle(int r) { return (((r & 15) >> 1) ^ ((r & 15) >> 3)) & 3; }
__device__ __forceinline__ uint32_t rk_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

struct RankedScratch {
  uint16_t* khi;  // [RK_SLOTS][dkp] bf16 hi parts (zero past count and past d_key)
  uint16_t* klo;  // [RK_SLOTS][dkp] bf16 lo parts
  float4* terms;  // [RK_SLOTS] {|k|^2, 2 RK_DOT_ERR |k|, 1 / (1 - norm_sq), 0} (stored f32 norm_sq)
  float* zdot;    // [RK_CHUNK][RK_SLOTS] approximate q.k
  double* qq;     // [RK_CHUNK] |q|^2 (any order)
};

__host__ __device__ inline int ranked_dkp(int dk) { return (dk + RK_BK - 1) / RK_BK * RK_BK; }

// Queries per dot/pick pass: RK_CHUNK unless the arguments name a smaller chunk.
static int ranked_chunk(const RetrieveArgs& a) { return a.chunk > 0 && a.chunk < RK_CHUNK ? a.chunk : RK_CHUNK; }

static constexpr size_t ranked_scratch_bytes(int dk, int chunk) {
  return (size_t)RK_SLOTS * ((dk + RK_BK - 1) / RK_BK * RK_BK) * 2 * sizeof(uint16_t) + RK_SLOTS * sizeof(float4) +
         (size_t)chunk * RK_SLOTS * sizeof(float) + (size_t)chunk * sizeof(double);
}

static RankedScratch ranked_scratch(void* base, int dk, int chunk) {
  const size_t row = (size_t)RK_SLOTS * ranked_dkp(dk);
  RankedScratch s;
  s.khi = static_cast<uint16_t*>(base);
  s.klo = s.khi + row;
  s.terms = reinterpret_cast<float4*>(s.klo + row);
  s.zdot = reinterpret_cast<float*>(s.terms + RK_SLOTS);
  s.qq = reinterpret_cast<double*>(s.zdot + (size_t)chunk * RK_SLOTS);
  return s;
}

// The allocation-free retrieval's scratch: one array per device, sized for
// the ranked path at the largest key width and kNoallocChunk queries per
// pass.  Host code reaches it only through the address hipGetSymbolAddress
// returns (noalloc_scratch_address); the symbol itself is not a device
// address on the host.
static_assert(ranked_scratch_bytes(RK_MAX_DK, kNoallocChunk) <= kNoallocScratchBytes, "scratch size");
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

__global__ __launch_bounds__(256) void ranked_prep_kernel(RetrieveArgs a, RankedScratch sc) {
  __shared__ double part[256];
  const int s = blockIdx.x, dkp = ranked_dkp(a.dk);
  const bool live = s < a.count;
  double acc = 0.0;
  for (int i = threadIdx.x; i < dkp; i += 256) {
    const float x = (live && i < a.dk) ? a.keys[(size_t)s * a.dk + i] : 0.0f;
    const uint32_t hb = rk_bf16(x);
    const float lo = x - __uint_as_float(hb << 16);
    sc.khi[(size_t)s * dkp + i] = (uint16_t)hb;
    sc.klo[(size_t)s * dkp + i] = (uint16_t)rk_bf16(lo);
    acc += (double)x * (double)x;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0)
    sc.terms[s] = make_float4((float)part[0], (float)(2.0 * RK_DOT_ERR * sqrt(part[0])),
                              live ? (float)(1.0 / (1.0 - (double)a.norm_sq[s])) : 0.0f, 0.0f);
}

// ---- 1. approximate dot products ------------------------------------------
// A 512-thread workgroup computes a 256-query x 256-slot tile; wave w owns
// queries (w & 1) * 128 .. +128 and slots (w >> 1) * 64 .. +64 (4 x 2 MFMA
// 32x32 tiles).  Key slabs (pre-split) move global -> LDS directly; query
// slabs are loaded as fp32, split into hi/lo in registers and stored.  Two
// slab stages; 64-byte slab rows with the 16-byte chunk index XOR-swizzled.
constexpr int RD_A = RK_TQ * RK_BK * 2;          // bytes of one bf16 query slab (hi or lo)
constexpr int RD_B = RK_TS * RK_BK * 2;          // bytes of one bf16 key slab
constexpr int RD_STAGE = 2 * RD_A + 2 * RD_B;
constexpr int RD_LDS = 2 * RD_STAGE;
static_assert(RD_LDS <= 160 * 1024, "LDS budget");

__global__ __launch_bounds__(RK_THREADS) void ranked_dot_kernel(RetrieveArgs a, RankedScratch sc, int q0, int nq) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char rd_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int wq = wave & 1, ws = wave >> 1;
  const int qb = blockIdx.x * RK_TQ, sb = blockIdx.y * RK_TS;
  const int dk = a.dk, dkp = ranked_dkp(dk);

  // Query staging: thread -> rows tid/8 + 64p, four dimensions at (tid%8)*4.
  const int ar = tid >> 3, ac = (tid & 7) * 4;
  const float* qsrc[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) qsrc[p] = a.q + (size_t)(q0 + min(qb + ar + 64 * p, nq - 1)) * a.ld_q;
  float4 qv[4];
  double qpart[4] = {0.0, 0.0, 0.0, 0.0};
  auto load_q = [&](int k0) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
      qv[p] = (k0 + ac < dk) ? *reinterpret_cast<const float4*>(qsrc[p] + k0 + ac) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto store_q = [&](int stage) {
    uint16_t* ahi = reinterpret_cast<uint16_t*>(rd_smem + stage * RD_STAGE);
    uint16_t* alo = reinterpret_cast<uint16_t*>(rd_smem + stage * RD_STAGE + RD_A);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float x[4] = {qv[p].x, qv[p].y, qv[p].z, qv[p].w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[e] = rk_bf16(x[e]);
        l[e] = rk_bf16(x[e] - __uint_as_float(h[e] << 16));
        qpart[p] += (double)x[e] * (double)x[e];
      }
      const int row = ar + 64 * p;
      const int off = row * RK_BK + (((ac >> 3) ^ rk_swizzle(row)) << 3) + (ac & 7);
      *reinterpret_cast<uint2*>(ahi + off) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      *reinterpret_cast<uint2*>(alo + off) = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
    }
  };
  // Key slabs: 16 rows of 64 bytes per wave instruction, two per array.
  const int lr = lane >> 2, pc = lane & 3;
  auto issue_b = [&](int stage, int k0) {
#pragma unroll
    for (int i = 0; i < RK_TS / 16 / 8; ++i) {
      const int row = (wave + 8 * i) * 16 + lr;
      const int lc = pc ^ rk_swizzle(row);
      const size_t src = (size_t)(sb + row) * dkp + k0 + lc * 8;
      unsigned char* base = rd_smem + stage * RD_STAGE + 2 * RD_A + (wave + 8 * i) * 16 * RK_BK * 2;
      __builtin_amdgcn_global_load_lds((const void*)(sc.khi + src),
                                       (__attribute__((address_space(3))) void*)base, 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(sc.klo + src),
                                       (__attribute__((address_space(3))) void*)(base + RD_B), 16, 0, 0);
    }
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][u][i] = 0.0f;

  const int nk = dkp / RK_BK;
  issue_b(0, 0);
  load_q(0);
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));  // vmcnt(0)
  store_q(0);
  const int fr = rk_swizzle(l32);
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    // This wave's slab loads and LDS stores are complete; meet the others.
    __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));  // vmcnt(0) lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    if (kt + 1 < nk) {
      issue_b(st ^ 1, (kt + 1) * RK_BK);
      load_q((kt + 1) * RK_BK);
    }
    const uint16_t* ahi = reinterpret_cast<const uint16_t*>(rd_smem + st * RD_STAGE);
    const uint16_t* alo = ahi + RK_TQ * RK_BK;
    const uint16_t* bhi = alo + RK_TQ * RK_BK;
    const uint16_t* blo = bhi + RK_TS * RK_BK;
#pragma unroll
    for (int kk = 0; kk < RK_BK / 16; ++kk) {
      const int ch = (kk * 2 + half) ^ fr;
      bf16x8_t fbh[2], fbl[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int brow = (ws * 64 + u * 32 + l32) * RK_BK + ch * 8;
        fbh[u] = *reinterpret_cast<const bf16x8_t*>(bhi + brow);
        fbl[u] = *reinterpret_cast<const bf16x8_t*>(blo + brow);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int arow = (wq * 128 + t * 32 + l32) * RK_BK + ch * 8;
        const bf16x8_t fah = *reinterpret_cast<const bf16x8_t*>(ahi + arow);
        const bf16x8_t fal = *reinterpret_cast<const bf16x8_t*>(alo + arow);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fbh[u], fah, acc[t][u], 0, 0, 0);
          acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fbl[u], fah, acc[t][u], 0, 0, 0);
          acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fbh[u], fal, acc[t][u], 0, 0, 0);
        }
      }
    }
    if (kt + 1 < nk) {
      __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));  // vmcnt(0): the query slab
      store_q(st ^ 1);
    }
  }
  // |q|^2 per row (the slot-half-0 workgroups): eight adjacent lanes per row.
  if (blockIdx.y == 0) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      double v = qpart[p];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      const int row = qb + ar + 64 * p;
      if ((tid & 7) == 0 && row < nq) sc.qq[row] = v;
    }
  }
  // Accumulator layout (keys as the first operand): lane l holds query
  // tile row l%32 and slots 8*(i/4) + 4*(l/32) + i%4.
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = qb + wq * 128 + t * 32 + l32;
    if (row < nq) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int slot = sb + ws * 64 + u * 32 + 8 * g + 4 * half;
          *reinterpret_cast<float4*>(sc.zdot + (size_t)row * RK_SLOTS + slot) =
              make_float4(acc[t][u][4 * g], acc[t][u][4 * g + 1], acc[t][u][4 * g + 2], acc[t][u][4 * g + 3]);
        }
    }
  }
}

// ---- 2-4. candidates, exact distances, selection, readout -----------------
// One wave per query, no workgroup-wide synchronisation.
//  - Candidates: the bounds of every slot from the approximate dot product;
//    T = the top_k-th smallest of the 64 per-lane minima of U.
//  - Distances of the candidates: |q - k|^2 summed in f64 across the wave
//    (coalesced rows, any order).  The reference's sequential sum and this
//    one are both within (d_key - 1) * 2^-53 (relative) of the exact sum of
//    the same nonnegative terms, so the two differ by at most RQ_SUM_REL; the
//    distance's relative sensitivity to the sum is at most 1/2.  When the f32
//    rounding of the distance is the same at both ends of that interval it
//    equals the reference's; otherwise (rare) the wave runs the sequential
//    sum itself.  |q|^2 (squared_norm, with its clamp below 1) likewise.
//  - Ranks by (distance bits, slot) counted over the candidates; softmax and
//    value readout in ascending slot order.
constexpr int RQ_WAVES = 4;                    // independent waves per workgroup
constexpr int RQ_V = RK_MAX_DK / 256;          // float4 per lane for one row
constexpr int RQ_QPW = 2;                      // queries per wave (measured: 1, 4, 8 no faster)
constexpr int RQ_G = 2;                        // candidate rows per step
constexpr int RK_MAX_DV4 = 256;                // vectorised readout: d_val <= 1024
constexpr double RQ_SUM_REL = 4e-13;           // >= 2 * 1024 * 2^-53, with margin
constexpr double RQ_DIST_REL = 4e-13;          // distance interval (relative)

// The reference's sequential f64 sum over a row distributed as lane l holding
// dimensions 256 v + 4 l + e: sum of (x - y)^2 in dimension order.
__device__ double rq_sequential(const float (&x)[RQ_V * 4], const float (&y)[RQ_V * 4], int dk) {
  double acc = 0.0;
#pragma unroll
  for (int v = 0; v < RQ_V; ++v) {
    for (int l = 0; l < 64; ++l) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
        const int i = 256 * v + 4 * l + e;
        if (i < dk) {
          const float xv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[4 * v + e]), l));
          const float yv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(y[4 * v + e]), l));
          const double t = (double)xv - (double)yv;
          acc = acc + t * t;
        }
      }
    }
  }
  return acc;
}

// Lane exchanges inside each row of 16 lanes (DPP; gfx9 dpp_ctrl codes:
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror).  They
// run in the VALU pipe, with none of the LDS round trip of a shuffle.
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_ROW_HALF_MIRROR = 0x141, DPP_ROW_MIRROR = 0x140;
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a fully active wave, the same in every lane:
// pairs, quads, halves and whole rows of 16 lanes by DPP (each exchange adds
// the same two operands in both lanes), then the four row sums as
// (r0 + r1) + (r2 + r3).  Deterministic; the order differs from a
// sequential sum (callers bound the difference).
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<DPP_QUAD_XOR1>(v);
  v += dpp_f64<DPP_QUAD_XOR2>(v);
  v += dpp_f64<DPP_ROW_HALF_MIRROR>(v);
  v += dpp_f64<DPP_ROW_MIRROR>(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// Minimum over the 64 lanes of a fully active wave (order-free), by DPP.
__device__ __forceinline__ float wave_min_dpp(float v) {
  v = fminf(v, dpp_f32<DPP_QUAD_XOR1>(v));
  v = fminf(v, dpp_f32<DPP_QUAD_XOR2>(v));
  v = fminf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
  v = fminf(v, dpp_f32<DPP_ROW_MIRROR>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fminf(fminf(r0, r1), fminf(r2, r3));
}

__device__ __forceinline__ float rq_qsq(double qs) {
  float f = (float)qs;
  if (qs < 1.0 && f == 1.0f) f = __uint_as_float(0x3f7fffffu);
  return f;
}

template <int V>
// Four waves per SIMD (128 VGPRs, a few spills off the common path): the
// per-query chain is latency-bound, and 16 resident waves per CU measure 8%
// faster than 12.
__global__ __launch_bounds__(64 * RQ_WAVES) __attribute__((amdgpu_waves_per_eu(4))) void ranked_pick_kernel(RetrieveArgs a, RankedScratch sc, int q0, int nq,
                                                                    int vec_out) {
  __shared__ uint16_t s_cand[RQ_WAVES][RK_SLOTS];
  __shared__ unsigned long long s_key[RQ_WAVES][RK_SLOTS];
  __shared__ uint32_t s_sel[RQ_WAVES][kMaxTopK];
  __shared__ float s_selw[RQ_WAVES][kMaxTopK];
  __shared__ __attribute__((aligned(16))) float s_lmin[RQ_WAVES][64];
  __shared__ double s_sq[RQ_WAVES][RK_SLOTS];
  __shared__ float s_min[RQ_WAVES];
  constexpr int SPL = RK_SLOTS / 64;
  // The wave index as a uniform value: the per-query row bases below then live
  // in scalar registers and the loads take 32-bit offsets (64-bit per-slot
  // addresses had been hoisted out of the query loop and spilled).
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int dk = a.dk, cnt = a.count, K = a.top_k;
  uint16_t* cand = s_cand[wave];
  unsigned long long* ckey = s_key[wave];
  uint32_t* sel = s_sel[wave];
  float* selw = s_selw[wave];
  double* csq = s_sq[wave];

  const int row0 = (blockIdx.x * RQ_WAVES + wave) * RQ_QPW;
  for (int row = row0; row < min(row0 + RQ_QPW, nq); ++row) {
    const size_t n = (size_t)q0 + row;
    // ---- candidates: bounds in f32 (their rounding, ~1e-7 relative, is far
    // inside the RK_TIE slack) ----
    // The scratch holds RK_SLOTS entries per row, so every slot's loads run
    // unguarded and are in flight together (a load under `s < cnt` waited
    // out its own round trip); slots past the count are masked below.
    // |q|^2 is loaded after them, so its wait does not hold them back.
    float L[SPL];
    float lm = HUGE_VALF;
    float4 tmv[SPL];
    float dtv[SPL];
    const char* tbase = reinterpret_cast<const char*>(sc.terms);
    const char* zbase = reinterpret_cast<const char*>(sc.zdot + (size_t)row * RK_SLOTS);
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      tmv[j] = *reinterpret_cast<const float4*>(tbase + (uint32_t)(16 * (lane + 64 * j)));
      dtv[j] = *reinterpret_cast<const float*>(zbase + (uint32_t)(4 * (lane + 64 * j)));
    }
    const double qq = sc.qq[row];
    const float qqf = (float)qq, qnf = (float)sqrt(qq);
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      const int s = lane + 64 * j;
      L[j] = HUGE_VALF;
      if (s < cnt) {
        const float4 tm = tmv[j];
        const float dot = dtv[j];
        const float sqt = qqf + tm.x - 2.0f * dot;
        const float e = qnf * tm.y + 1e-6f * (qqf + tm.x + 2.0f * fabsf(dot));
        L[j] = (sqt - e) * tm.z;
        lm = fminf(lm, (sqt + e) * tm.z);
      }
    }
    // T = the K-th smallest lane minimum (counted with multiplicity).
    s_lmin[wave][lane] = lm;
    wave_sync();
    int le = 0;
#pragma unroll
    for (int l4 = 0; l4 < 16; ++l4) {
      const float4 v = *reinterpret_cast<const float4*>(&s_lmin[wave][4 * l4]);
      le += (v.x <= lm) + (v.y <= lm) + (v.z <= lm) + (v.w <= lm);
    }
    const float lim = wave_min_dpp(le >= K ? lm : HUGE_VALF) * (1.0f + (float)RK_TIE);
    int m = 0;
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      const bool c = lane + 64 * j < cnt && L[j] <= lim;
      const unsigned long long b = __ballot(c);
      if (c) cand[m + __popcll(b & ((1ull << lane) - 1ull))] = (uint16_t)(lane + 64 * j);
      m += __popcll(b);
    }
    // ---- the query row and |q|^2 ----
    const float* qrow = a.q + n * a.ld_q;
    float qv[V * 4];
    double qs = 0.0;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int i = 256 * v + 4 * lane;
      // Clamped in-range address, masked after: no load under a branch.
      float4 x = *reinterpret_cast<const float4*>(qrow + min(i, dk - 4));
      if (i >= dk) x = make_float4(0.f, 0.f, 0.f, 0.f);
      qv[4 * v] = x.x, qv[4 * v + 1] = x.y, qv[4 * v + 2] = x.z, qv[4 * v + 3] = x.w;
#pragma unroll
      for (int e = 0; e < 4; ++e) qs = fma((double)qv[4 * v + e], (double)qv[4 * v + e], qs);
    }
    qs = wave_sum_f64(qs);
    float q_sq = rq_qsq(qs);
    if (rq_qsq(qs * (1.0 - RQ_SUM_REL)) != rq_qsq(qs * (1.0 + RQ_SUM_REL))) {
      float qf[RQ_V * 4], zero[RQ_V * 4];
#pragma unroll
      for (int e = 0; e < RQ_V * 4; ++e) qf[e] = e < V * 4 ? qv[e < V * 4 ? e : 0] : 0.0f, zero[e] = 0.0f;
      q_sq = rq_qsq(rq_sequential(qf, zero, dk));
    }
    // ---- candidate sums |q - k|^2 across the wave, RQ_G rows at a time
    // (prefetching the next group's rows measured no faster: the sums are
    // bound by the L2 -> CU bandwidth of the key rows, and the extra
    // registers cost waves) ----
    for (int c0 = 0; c0 < m; c0 += RQ_G) {
      float kf[RQ_G][V * 4];
#pragma unroll
      for (int g = 0; g < RQ_G; ++g) {
        const float* krow = a.keys + (size_t)cand[min(c0 + g, m - 1)] * dk;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int i = 256 * v + 4 * lane;
          float4 y = *reinterpret_cast<const float4*>(krow + min(i, dk - 4));
          if (i >= dk) y = make_float4(0.f, 0.f, 0.f, 0.f);
          kf[g][4 * v] = y.x, kf[g][4 * v + 1] = y.y, kf[g][4 * v + 2] = y.z, kf[g][4 * v + 3] = y.w;
        }
      }
      double sq[RQ_G];
#pragma unroll
      for (int g = 0; g < RQ_G; ++g) {
        double acc = 0.0;
#pragma unroll
        for (int e = 0; e < V * 4; ++e) {
          const double t = (double)qv[e] - (double)kf[g][e];
          acc = fma(t, t, acc);
        }
        sq[g] = wave_sum_f64(acc);
      }
      if (lane == 0)
#pragma unroll
        for (int g = 0; g < RQ_G; ++g)
          if (c0 + g < m) csq[c0 + g] = sq[g];
    }
    wave_sync();
    // ---- candidate distances, one candidate per lane; the rare ambiguous
    // rounding is settled by the sequential sum ----
    for (int cb = 0; cb < m; cb += 64) {
      const int c = cb + lane;
      bool ok = true;
      if (c < m) {
        const uint32_t slot = cand[c];
        const double den = (1.0 - (double)q_sq) * (1.0 - (double)a.norm_sq[slot]);
        const double r = 2.0 * rust_asinh(sqrt(csq[c] / den));
        const double dr = RQ_DIST_REL * r;
        ok = (float)(r - dr) == (float)(r + dr);
        ckey[c] = ((unsigned long long)__float_as_uint((float)r) << 32) | slot;
      }
      unsigned long long redo = __ballot(!ok);
      while (redo) {
        const int l = __ffsll((long long)redo) - 1;
        redo &= redo - 1;
        const uint32_t s2 = cand[cb + l];
        float qf[RQ_V * 4], kf[RQ_V * 4];
#pragma unroll
        for (int v = 0; v < RQ_V; ++v) {
          const int i = 256 * v + 4 * lane;
          const bool in = i < dk;
          const float4 x = in ? *reinterpret_cast<const float4*>(qrow + i) : make_float4(0.f, 0.f, 0.f, 0.f);
          const float4 y = in ? *reinterpret_cast<const float4*>(a.keys + (size_t)s2 * dk + i)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
          qf[4 * v] = x.x, qf[4 * v + 1] = x.y, qf[4 * v + 2] = x.z, qf[4 * v + 3] = x.w;
          kf[4 * v] = y.x, kf[4 * v + 1] = y.y, kf[4 * v + 2] = y.z, kf[4 * v + 3] = y.w;
        }
        const double sq2 = rq_sequential(qf, kf, dk);
        const double den2 = (1.0 - (double)q_sq) * (1.0 - (double)a.norm_sq[s2]);
        const float dist = (float)(2.0 * rust_asinh(sqrt(sq2 / den2)));
        if (lane == 0) ckey[cb + l] = ((unsigned long long)__float_as_uint(dist) << 32) | s2;
      }
    }
    if (lane < K) {
      sel[lane] = 0xFFFFFFFFu;
      selw[lane] = 0.0f;
    }
    wave_sync();
    // ---- selection: ranks over the candidates, positions in slot order ----
    int nsel_before = 0;
    for (int cb = 0; cb < m; cb += 64) {
      const int c = cb + lane;
      const unsigned long long key = c < m ? ckey[c] : ~0ull;
      int rank = 0;
      if (c < m)
        for (int c2 = 0; c2 < m; ++c2) rank += ckey[c2] < key;
      const bool chosen = c < m && rank < K;
      if (c < m && rank == 0) s_min[wave] = __uint_as_float((uint32_t)(key >> 32));
      const unsigned long long b = __ballot(chosen);
      if (chosen) {
        const int pos = nsel_before + __popcll(b & ((1ull << lane) - 1ull));
        sel[pos] = (uint32_t)(key & 0xFFFFFFFFull);
        selw[pos] = __uint_as_float((uint32_t)(key >> 32));  // the distance, for now
      }
      nsel_before += __popcll(b);
    }
    wave_sync();
    const float min_dist = s_min[wave];
    const float ev = lane < K && sel[lane] != 0xFFFFFFFFu ? expf((min_dist - selw[lane]) / a.tau) : 0.0f;
    wave_sync();
    if (lane < K) selw[lane] = ev;
    wave_sync();
    float sum = 0.0f;
    for (int t = 0; t < K; ++t) sum += selw[t];
    wave_sync();
    if (lane < K) selw[lane] = ev / sum;
    wave_sync();
    if (a.out_min && lane == 0) a.out_min[n] = min_dist;
    if (a.out_idx && lane < K) a.out_idx[n * K + lane] = sel[lane];
    if (a.weights || a.weights16) {
      for (int s = lane; s < a.capacity; s += 64) {
        float w = 0.0f;
        for (int t = 0; t < K; ++t)
          if (sel[t] == (uint32_t)s) w = selw[t];
        put_weight(a, (int)n, s, w);
      }
    }
    // ---- value readout in ascending slot order, eight rows at a time ----
    if (a.out_val) {
      const int dv = a.dv;
      if (vec_out) {
        float4 o[(RK_MAX_DV4 + 63) / 64];
#pragma unroll
        for (int u = 0; u < (RK_MAX_DV4 + 63) / 64; ++u) o[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int t0 = 0; t0 < K; t0 += 8) {
          const float* vr[8];
          float w[8];
          bool use[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const uint32_t s = t0 + u < K ? sel[t0 + u] : 0xFFFFFFFFu;
            use[u] = s < (uint32_t)cnt;
            w[u] = use[u] ? selw[t0 + u] : 0.0f;
            vr[u] = a.values + (size_t)(use[u] ? s : 0u) * dv;
          }
#pragma unroll
          for (int jj = 0; jj < (RK_MAX_DV4 + 63) / 64; ++jj) {
            const int j4 = lane + 64 * jj;
            if (j4 < dv / 4) {
              float4 v[8];
#pragma unroll
              for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4*>(vr[u] + 4 * j4);
#pragma unroll
              for (int u = 0; u < 8; ++u) {
#pragma clang fp contract(off)
                if (use[u]) {
                  o[jj].x = o[jj].x + w[u] * v[u].x;
                  o[jj].y = o[jj].y + w[u] * v[u].y;
                  o[jj].z = o[jj].z + w[u] * v[u].z;
                  o[jj].w = o[jj].w + w[u] * v[u].w;
                }
              }
            }
          }
        }
#pragma unroll
        for (int jj = 0; jj < (RK_MAX_DV4 + 63) / 64; ++jj) {
          const int j4 = lane + 64 * jj;
          if (j4 < dv / 4) *reinterpret_cast<float4*>(a.out_val + n * dv + 4 * j4) = o[jj];
        }
      } else {
        for (int j = lane; j < dv; j += 64) {
#pragma clang fp contract(off)
          float o = 0.0f;
          for (int t = 0; t < K; ++t) {
            const uint32_t s = sel[t];
            const float v = a.values[(size_t)min(s, (uint32_t)cnt - 1) * dv + j];
            if (s < (uint32_t)cnt) o = o + selw[t] * v;
          }
          a.out_val[n * dv + j] = o;
        }
      }
    }
    wave_sync();
  }
}

// clamp_value (src/memory.rs:150-170) on rows [n_rows, d] with leading
// dimension ld, src -> dst (may alias): a row whose Euclidean norm exceeds
// its cap is scaled to it (f64 scale, f32 rounding), then its nonzero
// components move one ulp toward zero per pass while the rounded row still
// exceeds it.  The squared norm is the reference's left-to-right f64 sum
// (src/memory.rs:190-192), so every decision and bit equals its own.  One
// wave per row, staged in LDS.  Row r takes caps.c[r / rows_per_cap]; a cap
// <= 0 copies the row.  A capped row whose squared norm is not finite is
// copied unchanged and raises *bad (the reference asserts the norm is
// finite, src/memory.rs:151-152).
__global__ __launch_bounds__(64) void clamp_rows_kernel(const float* src, float* dst, int d, size_t ld,
                                                        ValueCaps caps, int rows_per_cap, int* bad) {
  extern __shared__ float srow[];
  __shared__ double s_norm;
  const int row = blockIdx.x, lane = threadIdx.x;
  const float cap = caps.c[row / rows_per_cap];
  const float* in = src + (size_t)row * ld;
  float* out = dst + (size_t)row * ld;
  for (int j = lane; j < d; j += 64) srow[j] = in[j];
  __syncthreads();
  auto norm_sq = [&]() {
    if (lane == 0) {
      double s = 0.0;
      for (int j = 0; j < d; ++j) s += (double)srow[j] * (double)srow[j];
      s_norm = s;
    }
    __syncthreads();
    const double v = s_norm;
    __syncthreads();
    return v;
  };
  if (cap > 0.0f) {
    const double cap_sq = (double)cap * (double)cap;
    const double nsq = norm_sq();
    if (!isfinite(nsq)) {
      if (lane == 0 && bad) bad[0] = 1;
    } else if (nsq > cap_sq) {
      const double scale = (double)cap / sqrt(nsq);
      for (int j = lane; j < d; j += 64) srow[j] = (float)((double)srow[j] * scale);
      __syncthreads();
      // Each pass shrinks every nonzero magnitude; the pass count bounds the
      // loop regardless.
      for (int pass = 0; pass < 1024 && norm_sq() > cap_sq; ++pass) {
        for (int j = lane; j < d; j += 64)
          if (srow[j] != 0.0f) srow[j] = __uint_as_float(__float_as_uint(srow[j]) - 1u);
        __syncthreads();
      }
    }
  }
  for (int j = lane; j < d; j += 64) out[j] = srow[j];
}

Status launch_clamp_rows(hipStream_t stream, const float* src, float* dst, int n_rows, int d, size_t ld,
                         const ValueCaps& caps, int rows_per_cap, int* bad) {
  if (n_rows <= 0 || d <= 0) return Status::Ok();
  if ((size_t)d * 4 > 64 * 1024) return Status::Invalid("value cap: rows wider than 16384");
  clamp_rows_kernel<<<(unsigned)n_rows, 64, (size_t)d * 4, stream>>>(src, dst, d, ld, caps, rows_per_cap, bad);
  PSSA_LAUNCH_CHECK("clamp_rows");
  return Status::Ok();
}

static bool ranked_read_fits(const RetrieveArgs& a) {
  return a.top_k > 0 && !a.hgate && !a.count_dev && a.top_k < a.count && a.count <= RK_SLOTS && !a.project &&
         !a.q_pnc && !a.q_norm && a.dk % 4 == 0 && a.dk <= RK_MAX_DK && a.ld_q % 4 == 0 &&
         ((uintptr_t)a.q & 15) == 0 && ((uintptr_t)a.keys & 15) == 0;
}

size_t retrieve_scratch_bytes(const RetrieveArgs& a) {
  return ranked_read_fits(a) ? ranked_scratch_bytes(a.dk, ranked_chunk(a)) : 0;
}

Status noalloc_scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  PSSA_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return Status::Invalid("allocation-free scratch: device index above 63");
  std::lock_guard<std::mutex> g(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    PSSA_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return Status::Device("hipGetSymbolAddress returned a null scratch address");
    addr[dev] = p;
  }
  *out = addr[dev];
  return Status::Ok();
}

static bool soft_read_fits(const RetrieveArgs& a) {
  return (a.top_k == 0 || (!a.count_dev && a.top_k >= a.count)) && a.project && !a.q_norm && !a.out_val &&
         !a.out_min && !a.out_idx && a.dk <= SOFT_MAX_DK && a.capacity <= 64 * SOFT_SPL &&
         (long)a.dk * soft_pitch(a.capacity) <= SOFT_MAX_KEYS + SOFT_MAX_DK;
}

// Raises the kernel's dynamic-LDS limit to the device maximum once per
// device, before any launch that could be captured into a graph.
static Status allow_large_lds() {
  static std::mutex mu;
  static bool done[64] = {};
  int dev = 0;
  PSSA_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> g(mu);
  if (dev >= 0 && dev < 64 && done[dev]) return Status::Ok();
  const void* soft[] = {
#define PSSA_SOFT_FN(QG, SPL, NWV)                                         \
  reinterpret_cast<const void*>(&soft_read_kernel<QG, SPL, false, NWV>),  \
      reinterpret_cast<const void*>(&soft_read_kernel<QG, SPL, true, NWV>),
      PSSA_SOFT_FN(1, 1, SOFT_WAVES) PSSA_SOFT_FN(1, 2, SOFT_WAVES) PSSA_SOFT_FN(1, 4, SOFT_WAVES)
      PSSA_SOFT_FN(1, 8, SOFT_WAVES) PSSA_SOFT_FN(SOFT_QG, 1, SOFT_WAVES) PSSA_SOFT_FN(SOFT_QG, 2, SOFT_WAVES)
      PSSA_SOFT_FN(SOFT_QG, 4, SOFT_WAVES) PSSA_SOFT_FN(SOFT_QG, 8, SOFT_WAVES)
      PSSA_SOFT_FN(1, 1, SOFT_WAVES_FEW) PSSA_SOFT_FN(1, 2, SOFT_WAVES_FEW) PSSA_SOFT_FN(1, 4, SOFT_WAVES_FEW)
      PSSA_SOFT_FN(1, 8, SOFT_WAVES_FEW)
#undef PSSA_SOFT_FN
#define PSSA_SOFT_QP_FN(SPL)                                                        \
  reinterpret_cast<const void*>(&soft_read_kernel<1, SPL, false, SOFT_WAVES_FEW, true>), \
      reinterpret_cast<const void*>(&soft_read_kernel<1, SPL, true, SOFT_WAVES_FEW, true>),
      PSSA_SOFT_QP_FN(1) PSSA_SOFT_QP_FN(2) PSSA_SOFT_QP_FN(4) PSSA_SOFT_QP_FN(8)
#undef PSSA_SOFT_QP_FN
  };
  for (const void* f : soft)
    PSSA_HIP_TRY(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&ranked_dot_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  if (dev >= 0 && dev < 64) done[dev] = true;
  return Status::Ok();
}

Status init_retrieve_attributes() { return allow_large_lds(); }

Status prepare_retrieve(const RetrieveArgs& a) {
  if (soft_read_fits(a)) return allow_large_lds();
  return Status::Ok();
}


// Launch shape of the soft read: waves per workgroup, workgroups, queries per wave.
static void soft_read_shape(const RetrieveArgs& a, int& nwv, int& blocks, int& per) {
  // Few queries (a decode step): small workgroups spread them over more
  // CUs, each staging the bank for fewer waves.
  nwv = a.n <= SOFT_FEW_QUERIES ? SOFT_WAVES_FEW : SOFT_WAVES;
  blocks = (a.n + nwv - 1) / nwv;
  if (blocks > 512) blocks = 512;
  per = (a.n + blocks * nwv - 1) / (blocks * nwv);
}

bool retrieve_fuses_query(const RetrieveArgs& a) {
  if (!a.qa || !a.qw || !a.qaux || a.n <= 0 || !soft_read_fits(a)) return false;
  int nwv = 0, blocks = 0, per = 0;
  soft_read_shape(a, nwv, blocks, per);
  return nwv == SOFT_WAVES_FEW && per == 1 && a.dk <= 32 && a.qk > 0 && a.qk % 128 == 0 &&
         a.ld_qa % 8 == 0 && ((uintptr_t)a.qa & 15) == 0 && ((uintptr_t)a.qw & 15) == 0 &&
         soft_read_lds(a.dk, a.capacity, 1, nwv) + soft_qp_lds(a.qk, nwv) <= 160 * 1024;
}

Status launch_retrieve(hipStream_t stream, const RetrieveArgs& a) {
  if (a.n <= 0) return Status::Ok();
  if ((a.qa || a.qw || a.qaux) && !retrieve_fuses_query(a))
    return Status::Invalid("retrieve: fused query product outside the few-query soft read");
  if (a.dk <= 0 || a.capacity <= 0 || a.count < 0 || a.count > a.capacity)
    return Status::Invalid("retrieve: bad bank shape");
  if (a.top_k < 0 || a.top_k > kMaxTopK) return Status::Invalid("retrieve: top_k must be in 0..=64");
  if (a.top_k == 0 && !a.weights && !a.weights16 && !a.out_val) return Status::Invalid("retrieve: no output");
  if (soft_read_fits(a)) {
    int nwv = 0, blocks = 0, per = 0;
    soft_read_shape(a, nwv, blocks, per);
    const int qg = per >= SOFT_QG && nwv == SOFT_WAVES ? SOFT_QG : 1;
    const bool qp = a.qw != nullptr;  // retrieve_fuses_query held above
    const size_t lds = soft_read_lds(a.dk, a.capacity, qg, nwv) + (qp ? soft_qp_lds(a.qk, nwv) : 0);
    if (lds > 64 * 1024) PSSA_RETURN_IF(allow_large_lds());
    const int spl = soft_spl(a.capacity);
    if (qp) {
#define PSSA_SOFT_QP_CASE(SPL)                                                                  \
  if (spl == SPL) {                                                                             \
    if (a.hgate)                                                                                \
      soft_read_kernel<1, SPL, true, SOFT_WAVES_FEW, true><<<blocks, 64 * SOFT_WAVES_FEW, lds, stream>>>(a);  \
    else                                                                                        \
      soft_read_kernel<1, SPL, false, SOFT_WAVES_FEW, true><<<blocks, 64 * SOFT_WAVES_FEW, lds, stream>>>(a); \
    PSSA_LAUNCH_CHECK("soft_read");                                                             \
    return Status::Ok();                                                                        \
  }
      PSSA_SOFT_QP_CASE(1) PSSA_SOFT_QP_CASE(2) PSSA_SOFT_QP_CASE(4) PSSA_SOFT_QP_CASE(8)
#undef PSSA_SOFT_QP_CASE
      return Status::Invalid("retrieve: soft read shape");
    }
#define PSSA_SOFT_CASE(QG, SPL, NWV)                                                    \
  if (qg == QG && spl == SPL && nwv == NWV) {                                           \
    if (a.hgate)                                                                        \
      soft_read_kernel<QG, SPL, true, NWV><<<blocks, 64 * NWV, lds, stream>>>(a);       \
    else                                                                                \
      soft_read_kernel<QG, SPL, false, NWV><<<blocks, 64 * NWV, lds, stream>>>(a);      \
    PSSA_LAUNCH_CHECK("soft_read");                                                     \
    return Status::Ok();                                                                \
  }
    PSSA_SOFT_CASE(1, 1, SOFT_WAVES) PSSA_SOFT_CASE(1, 2, SOFT_WAVES) PSSA_SOFT_CASE(1, 4, SOFT_WAVES)
    PSSA_SOFT_CASE(1, 8, SOFT_WAVES) PSSA_SOFT_CASE(SOFT_QG, 1, SOFT_WAVES) PSSA_SOFT_CASE(SOFT_QG, 2, SOFT_WAVES)
    PSSA_SOFT_CASE(SOFT_QG, 4, SOFT_WAVES) PSSA_SOFT_CASE(SOFT_QG, 8, SOFT_WAVES)
    PSSA_SOFT_CASE(1, 1, SOFT_WAVES_FEW) PSSA_SOFT_CASE(1, 2, SOFT_WAVES_FEW) PSSA_SOFT_CASE(1, 4, SOFT_WAVES_FEW)
    PSSA_SOFT_CASE(1, 8, SOFT_WAVES_FEW)
#undef PSSA_SOFT_CASE
    return Status::Invalid("retrieve: soft read shape");
  }
  if (ranked_read_fits(a) && a.scratch && a.scratch_bytes >= retrieve_scratch_bytes(a)) {
    PSSA_RETURN_IF(allow_large_lds());
    const int chunk = ranked_chunk(a);
    const RankedScratch sc = ranked_scratch(a.scratch, a.dk, chunk);
    ranked_prep_kernel<<<RK_SLOTS, 256, 0, stream>>>(a, sc);
    PSSA_LAUNCH_CHECK("ranked_prep");
    const int vec_out = a.dv % 4 == 0 && a.dv <= 4 * RK_MAX_DV4 && ((uintptr_t)a.values & 15) == 0 &&
                        ((uintptr_t)a.out_val & 15) == 0;
    for (int q0 = 0; q0 < a.n; q0 += chunk) {
      const int nq = std::min(chunk, a.n - q0);
      ranked_dot_kernel<<<dim3((nq + RK_TQ - 1) / RK_TQ, (a.count + RK_TS - 1) / RK_TS), RK_THREADS, RD_LDS,
                          stream>>>(a, sc, q0, nq);
      PSSA_LAUNCH_CHECK("ranked_dot");
      const unsigned pg = (nq + RQ_WAVES * RQ_QPW - 1) / (RQ_WAVES * RQ_QPW);
      switch ((a.dk + 255) / 256) {
        case 1:
          ranked_pick_kernel<1><<<pg, 64 * RQ_WAVES, 0, stream>>>(a, sc, q0, nq, vec_out);
          break;
        case 2:
          ranked_pick_kernel<2><<<pg, 64 * RQ_WAVES, 0, stream>>>(a, sc, q0, nq, vec_out);
          break;
        case 3:
          ranked_pick_kernel<3><<<pg, 64 * RQ_WAVES, 0, stream>>>(a, sc, q0, nq, vec_out);
          break;
        default:
          ranked_pick_kernel<4><<<pg, 64 * RQ_WAVES, 0, stream>>>(a, sc, q0, nq, vec_out);
          break;
      }
      PSSA_LAUNCH_CHECK("ranked_pick");
    }
    return Status::Ok();
  }
  const int dk_pad = (a.dk + 3) & ~3;
  const size_t lds = (size_t)RETRIEVE_QPB * (dk_pad + a.capacity) * sizeof(float);
  if (lds > 128 * 1024) return Status::Invalid("retrieve: d_key + capacity too large for LDS");
  int blocks = (a.n + RETRIEVE_QPB - 1) / RETRIEVE_QPB;
  if (blocks > 8192) blocks = 8192;
  retrieve_kernel<<<blocks, 256, lds, stream>>>(a);
  PSSA_LAUNCH_CHECK("retrieve");
  return Status::Ok();
}

}  // namespace pssa

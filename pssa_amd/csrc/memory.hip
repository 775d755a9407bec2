// Poincare-ball memory read for gfx950.
//
// One wave per query, one lane per group of slots.  Everything that decides
// which slots are read -- the projection into the ball, the squared norms and
// the distances -- is computed in f64 in the reference's own order
// (sequential sums, no fused multiply-add, Rust's asinh formula), so the f32
// distances, and with them the top-k indices, agree with the reference
// (src/memory.rs:181-262).  The softmax weights and the value mix are fp32.
#include "memory.h"

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

__device__ __forceinline__ uint16_t bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ void put_weight(const RetrieveArgs& a, int n, int s, float w) {
  const size_t o = (size_t)n * a.capacity + s;
  if (a.weights) a.weights[o] = w;
  if (a.weights16) a.weights16[o] = bf16_bits(w);
}

constexpr double kMaxRadius = 1.0 - 8.0 * (double)FLT_EPSILON;  // src/memory.rs:173

__global__ __launch_bounds__(256) void retrieve_kernel(RetrieveArgs a) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dk_pad = (a.dk + 3) & ~3;
  float* sq = smem + wave * (dk_pad + a.capacity);  // this wave's query, then distances
  float* sdist = sq + dk_pad;
  __shared__ uint32_t ssel[4][kMaxTopK];
  const int cnt = a.count_dev ? a.count_dev[0] : a.count;

  for (int n = blockIdx.x * 4 + wave; n < a.n; n += gridDim.x * 4) {
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
    const float q_sq = bank_norm_sq(sq, a.dk);

    if (cnt == 0) {
      for (int s = lane; s < a.capacity; s += 64) put_weight(a, n, s, 0.0f);
      if (a.out_val)
        for (int j = lane; j < a.dv; j += 64) a.out_val[(size_t)n * a.dv + j] = 0.0f;
      if (a.out_min && lane == 0) a.out_min[n] = 0.0f;
      if (a.out_idx)
        for (int r = lane; r < a.top_k; r += 64) a.out_idx[(size_t)n * a.top_k + r] = 0xFFFFFFFFu;
      wave_sync();
      continue;
    }
    // ---- distances ----
    float local_min = FLT_MAX;
    for (int s = lane; s < cnt; s += 64) {
      const float dist = poincare_dist(sq, q_sq, a.keys + (size_t)s * a.dk, a.norm_sq[s], a.dk);
      sdist[s] = dist;
      local_min = fminf(local_min, dist);
    }
    const float min_dist = wave_min(local_min);
    wave_sync();
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
          for (int p = 0; p < r; ++p) taken |= ssel[wave][p] == (uint32_t)s;
          if (!taken && key < best) best = key;
        }
        best = wave_min_u64(best);
        if (lane == 0) ssel[wave][r] = (uint32_t)(best & 0xFFFFFFFFu);
        wave_sync();
      }
      if (lane == 0) {  // ascending slot order
        for (int x = 1; x < k; ++x) {
          const uint32_t v = ssel[wave][x];
          int y = x - 1;
          while (y >= 0 && ssel[wave][y] > v) {
            ssel[wave][y + 1] = ssel[wave][y];
            --y;
          }
          ssel[wave][y + 1] = v;
        }
      }
      wave_sync();
      float sum = 0.0f;
      for (int r = 0; r < k; ++r) sum += expf((min_dist - sdist[ssel[wave][r]]) / a.tau);
      if (a.weights || a.weights16) {
        for (int s = lane; s < a.capacity; s += 64) {
          bool chosen = false;
          for (int r = 0; r < k; ++r) chosen |= ssel[wave][r] == (uint32_t)s;
          put_weight(a, n, s, chosen ? expf((min_dist - sdist[s]) / a.tau) / sum : 0.0f);
        }
      }
      if (a.out_idx)
        for (int r = lane; r < k; r += 64) a.out_idx[(size_t)n * k + r] = ssel[wave][r];
      if (a.out_val) {
        for (int j = lane; j < a.dv; j += 64) {
#pragma clang fp contract(off)
          float acc = 0.0f;
          for (int r = 0; r < k; ++r) {
            const uint32_t s = ssel[wave][r];
            const float w = expf((min_dist - sdist[s]) / a.tau) / sum;
            acc = acc + w * a.values[(size_t)s * a.dv + j];
          }
          a.out_val[(size_t)n * a.dv + j] = acc;
        }
      }
    } else {
      // ---- full soft read (src/memory.rs:409-425) ----
      float part = 0.0f;
      for (int s = lane; s < cnt; s += 64) {
        const float e = expf((min_dist - sdist[s]) / a.tau);
        sdist[s] = e;
        part += e;
      }
      const float sum = wave_sum(part);
      wave_sync();
      for (int s = lane; s < a.capacity; s += 64) {
        const float w = s < cnt ? sdist[s] / sum : 0.0f;
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
    wave_sync();
  }
}

// ---------------------------------------------------------------------------
// Full soft read for the model path (no top-k, small banks): the bank's keys
// stay in LDS for the whole launch, transposed so that lane j of a wave reads
// slot j + 64q of key dimension i at consecutive addresses, next to
// 1/(1 - |k|^2) per slot in f64.  One wave per query, up to SOFT_SPL slots
// per lane, eight waves per workgroup.  The projection and the query norm
// follow the reference's sequential f64 order exactly; the squared distance
// sum runs in f64, and x = sum / ((1-|q|^2)(1-|k|^2)) is formed with the two
// reciprocals.  Only the soft weights depend on the result (no ranking), so
// 2 asinh(sqrt(x)) is then evaluated in f32 (relative error a few 1e-7, far
// inside the 1e-4 parity gate), followed by the reference's f32 softmax
// whose two sums over slots run as wave reductions.  Writes the
// [n, capacity] weights; the value readout is a GEMM.
constexpr int SOFT_SPL = 8;            // slots per lane: capacity <= 512
constexpr int SOFT_MAX_KEYS = 16384;   // dk * capacity floats held in LDS (64 KiB)
constexpr int SOFT_MAX_DK = 64;
constexpr int SOFT_WAVES = 8;

__device__ __forceinline__ size_t soft_keys_floats(int dk, int cap) {
  return (((size_t)dk * cap + 1) & ~(size_t)1);  // keep the f64 arrays 8-byte aligned
}

__global__ __launch_bounds__(64 * SOFT_WAVES) void soft_read_kernel(RetrieveArgs a) {
  extern __shared__ float smem[];
  const int cap = a.capacity, dk = a.dk, cnt = a.count_dev ? a.count_dev[0] : a.count;
  float* keyT = smem;                                                  // [dk][cap]
  double* rk = reinterpret_cast<double*>(smem + soft_keys_floats(dk, cap));  // [cap]
  double* pq = rk + cap;                                               // [waves][SOFT_MAX_DK]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < cnt * dk; e += 64 * SOFT_WAVES) {
    const int i = e / cnt, sl = e - i * cnt;
    keyT[i * cap + sl] = a.keys[(size_t)sl * dk + i];
  }
  for (int sl = tid; sl < cnt; sl += 64 * SOFT_WAVES) rk[sl] = 1.0 / (1.0 - (double)a.norm_sq[sl]);
  __syncthreads();
  double* p = pq + wave * SOFT_MAX_DK;

  for (int n = blockIdx.x * SOFT_WAVES + wave; n < a.n; n += gridDim.x * SOFT_WAVES) {
    const float* qrow = a.q + (size_t)n * a.ld_q;
    // diffeomorphic_project (src/memory.rs:194-211): sequential f64 norm.
    const float qv = lane < dk ? qrow[lane] : 0.0f;
    p[lane] = (double)qv;
    wave_sync();
    double r2 = 0.0;
    {
#pragma clang fp contract(off)
      for (int i = 0; i < dk; ++i) r2 = r2 + p[i] * p[i];
    }
    const double r = sqrt(r2);
    const double scale = r == 0.0 ? 1.0 : fmin(r / (1.0 + r), kMaxRadius) / r;
    const float pv = (float)((double)qv * scale);
    if (a.q_pnc && lane < dk) a.q_pnc[(size_t)n * dk + lane] = pv;
    wave_sync();
    p[lane] = (double)pv;
    wave_sync();
    // squared_norm of the projected query (src/memory.rs:181-192).
    double qs = 0.0;
    {
#pragma clang fp contract(off)
      for (int i = 0; i < dk; ++i) qs = qs + p[i] * p[i];
    }
    float q_sq = (float)qs;
    if (qs < 1.0 && q_sq == 1.0f) q_sq = __uint_as_float(0x3f7fffffu);
    const double rq = 1.0 / (1.0 - (double)q_sq);

    float dist[SOFT_SPL];
    float local_min = FLT_MAX;
    if (cnt > 0) {
      double sq[SOFT_SPL];
#pragma unroll
      for (int j = 0; j < SOFT_SPL; ++j) sq[j] = 0.0;
      for (int i = 0; i < dk; ++i) {
        const double pi = p[i];
        const float* kr = keyT + i * cap;
#pragma unroll
        for (int j = 0; j < SOFT_SPL; ++j) {
          const int sl = lane + 64 * j;
          const double t = pi - (double)(sl < cnt ? kr[sl] : 0.0f);
          sq[j] = fma(t, t, sq[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < SOFT_SPL; ++j) {
        const int sl = lane + 64 * j;
        if (sl < cnt) {
          const float x = (float)(sq[j] * rq * rk[sl]);
          const float y = sqrtf(x);
          // asinh(y) = log1p(y + y^2 / (1 + sqrt(1 + y^2))), y^2 = x.
          dist[j] = 2.0f * log1pf(y + x / (1.0f + sqrtf(1.0f + x)));
          local_min = fminf(local_min, dist[j]);
        } else {
          dist[j] = 0.0f;
        }
      }
    }
    const float min_dist = wave_min(local_min);
    float e[SOFT_SPL];
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < SOFT_SPL; ++j) {
      const int sl = lane + 64 * j;
      e[j] = sl < cnt ? expf((min_dist - dist[j]) / a.tau) : 0.0f;
      part += e[j];
    }
    const float sum = wave_sum(part);
#pragma unroll
    for (int j = 0; j < SOFT_SPL; ++j) {
      const int sl = lane + 64 * j;
      if (sl < cap) put_weight(a, n, sl, sl < cnt ? e[j] / sum : 0.0f);
    }
    wave_sync();
  }
}

static bool soft_read_fits(const RetrieveArgs& a) {
  return (a.top_k == 0 || (!a.count_dev && a.top_k >= a.count)) && a.project && !a.q_norm && !a.out_val &&
         !a.out_min && !a.out_idx && a.dk <= SOFT_MAX_DK && a.capacity <= 64 * SOFT_SPL &&
         (long)a.dk * a.capacity <= SOFT_MAX_KEYS;
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
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&soft_read_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  if (dev >= 0 && dev < 64) done[dev] = true;
  return Status::Ok();
}

Status init_retrieve_attributes() { return allow_large_lds(); }

Status prepare_retrieve(const RetrieveArgs& a) {
  if (soft_read_fits(a)) return allow_large_lds();
  return Status::Ok();
}


Status launch_retrieve(hipStream_t stream, const RetrieveArgs& a) {
  if (a.n <= 0) return Status::Ok();
  if (a.dk <= 0 || a.capacity <= 0 || a.count < 0 || a.count > a.capacity)
    return Status::Invalid("retrieve: bad bank shape");
  if (a.top_k < 0 || a.top_k > kMaxTopK) return Status::Invalid("retrieve: top_k must be in 0..=64");
  if (a.top_k == 0 && !a.weights && !a.weights16 && !a.out_val) return Status::Invalid("retrieve: no output");
  if (soft_read_fits(a)) {
    const size_t lds = (((size_t)a.dk * a.capacity + 1) & ~(size_t)1) * sizeof(float) +
                       ((size_t)a.capacity + (size_t)SOFT_WAVES * SOFT_MAX_DK) * sizeof(double);
    if (lds > 64 * 1024) PSSA_RETURN_IF(allow_large_lds());
    int blocks = (a.n + SOFT_WAVES - 1) / SOFT_WAVES;
    if (blocks > 512) blocks = 512;
    soft_read_kernel<<<blocks, 64 * SOFT_WAVES, lds, stream>>>(a);
    PSSA_LAUNCH_CHECK("soft_read");
    return Status::Ok();
  }
  const int dk_pad = (a.dk + 3) & ~3;
  const size_t lds = (size_t)4 * (dk_pad + a.capacity) * sizeof(float);
  if (lds > 128 * 1024) return Status::Invalid("retrieve: d_key + capacity too large for LDS");
  int blocks = (a.n + 3) / 4;
  if (blocks > 4096) blocks = 4096;
  retrieve_kernel<<<blocks, 256, lds, stream>>>(a);
  PSSA_LAUNCH_CHECK("retrieve");
  return Status::Ok();
}

}  // namespace pssa

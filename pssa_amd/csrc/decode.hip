// Greedy decode step for gfx950: one token per lane through the whole model
// (forward_inference, src/pssa.rs:2387-2391), the greedy choice
// (src/inference.rs:123-127) and, in plastic mode, the per-step write rules
// applied after the batch in lane order:
//   - refractory-protected bank write of the lane's projected query and block
//     output when the surprise -log softmax(logits)[chosen] exceeds 3.5
//     (insert_protected, src/memory.rs:305-342, with the write rule of
//     insert_training_memory_at, src/pssa.rs:3705-3736);
//   - Hebbian fast-weight update of the adapter with the block output as the
//     target and the adapter output as the prediction (dream_replay_value,
//     src/pssa.rs:1814-1832).
// Every launch reads its inputs from device memory (ids, counts, the step
// counter, the generation position), so one step can be captured into a
// hipGraph and replayed.
#include <cfloat>
#include <cmath>

#include "memory.h"
#include "model.h"

namespace pssa {

namespace {

// f32::total_cmp order: a larger key is a larger value in IEEE total order.
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t b = __float_as_int(f);
  return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

__device__ __forceinline__ void argmax_merge(int32_t& bk, int& bi, int32_t k2, int i2) {
  if (k2 > bk || (k2 == bk && i2 < bi)) {
    bk = k2;
    bi = i2;
  }
}
// Running sum of exp(x - m) with its maximum m: merge (m2, s2) into (m, s).
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  if (mm == -INFINITY) return;
  s = s * expf(m - mm) + s2 * expf(m2 - mm);
  m = mm;
}

constexpr int GR_CHUNK = 16;

// Repetition-penalty window of the greedy choice (sample(),
// src/inference.rs:104-127).  `append_row_id` appends the id the lane just
// consumed (ids[row]) before the window is read.
struct GreedyWindow {
  uint32_t* hist = nullptr;  // [lanes, kHist] ring
  int* hist_n = nullptr;     // [lanes] ids in the ring
  int* hist_pos = nullptr;   // [lanes] next position
  float penalty = 1.0f;
  int append_row_id = 0;
  int* nonfinite = nullptr;  // raised on any non-finite logit
};

// One workgroup per lane, one pass over the logits: greedy id over 1..V-1
// in f32::total_cmp order (ties to the lower id) after the repetition
// penalty, and the surprise logsumexp(logits) - logits[chosen] of the raw
// logits from a running maximum and rescaled sum.  The penalised ids (at
// most 64) are left out of the pass and enter with their penalised values
// at the end: each distinct window id is divided (positive) or multiplied
// (otherwise) by the penalty once per occurrence, as the reference applies
// it in window order.  Partials meet through lane shuffles and then across
// the four waves.
__global__ __launch_bounds__(256) void greedy_kernel(const float* __restrict__ logits, int V,
                                                     uint32_t* __restrict__ ids,
                                                     uint32_t* __restrict__ gen_ids,
                                                     const int* __restrict__ gen_pos, int n_lanes,
                                                     float* __restrict__ surprise, GreedyWindow gw) {
  constexpr int H = pssa_hip_lanes::kHist;
  __shared__ int32_t sk[4];
  __shared__ int si[4];
  __shared__ float smx[4], ssm[4];
  __shared__ uint32_t s_win[H];
  __shared__ float s_val[H];
  __shared__ int s_own[H];
  __shared__ int s_n;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* lg = logits + (size_t)row * V;
  const bool pen = gw.penalty > 1.0f && gw.hist != nullptr;
  if (gw.hist && tid == 0) {
    int n = gw.hist_n[row], pos = gw.hist_pos[row];
    if (gw.append_row_id) {
      gw.hist[(size_t)row * H + pos] = ids[row];
      pos = (pos + 1) % H;
      n = n < H ? n + 1 : H;
      gw.hist_pos[row] = pos;
      gw.hist_n[row] = n;
    }
    s_n = pen ? n : 0;
    for (int j = 0; j < n && pen; ++j) s_win[j] = gw.hist[(size_t)row * H + (pos - n + j + H) % H];
  }
  __syncthreads();
  const int wn = s_n;
  if (wave == 0 && lane < wn) {
    const uint32_t id = s_win[lane];
    int own = 1, c = 0;
    for (int j = 0; j < wn; ++j)
      if (s_win[j] == id) {
        own &= j >= lane;
        ++c;
      }
    float l = id < (uint32_t)V ? lg[id] : 0.0f;
    if (own)
      for (int q = 0; q < c; ++q) l = l > 0.0f ? l / gw.penalty : l * gw.penalty;
    s_val[lane] = l;
    s_own[lane] = own;
  }
  __syncthreads();
  auto in_window = [&](int v) {
    for (int j = 0; j < wn; ++j)
      if (s_win[j] == (uint32_t)v) return true;
    return false;
  };
  int32_t bk = INT32_MIN;
  int bi = V;
  float m = -INFINITY, sacc = 0.0f;
  int bad = 0;
  // Chunks of GR_CHUNK logits per thread are loaded together, then scanned
  // for the maximum and summed as independent exponentials.
  for (int v0 = 0; v0 < V; v0 += 256 * GR_CHUNK) {
    float x[GR_CHUNK];
#pragma unroll
    for (int k = 0; k < GR_CHUNK; ++k) {
      const int v = v0 + k * 256 + tid;
      x[k] = v < V ? lg[v] : -INFINITY;
    }
    float cm = -INFINITY;
#pragma unroll
    for (int k = 0; k < GR_CHUNK; ++k) {
      const int v = v0 + k * 256 + tid;
      if (v < V) bad |= !isfinite(x[k]);
      const int32_t key = total_key(x[k]);
      if (v >= 1 && v < V && (key > bk || (key == bk && v < bi)) && !(wn && in_window(v))) {
        bk = key;
        bi = v;
      }
      cm = fmaxf(cm, x[k]);
    }
    float cs = 0.0f;
    if (cm != -INFINITY) {
#pragma unroll
      for (int k = 0; k < GR_CHUNK; ++k) cs += expf(x[k] - cm);
    }
    lse_merge(m, sacc, cm, cs);
  }
  bad = __syncthreads_or(bad);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    argmax_merge(bk, bi, __shfl_xor(bk, off, 64), __shfl_xor(bi, off, 64));
    lse_merge(m, sacc, __shfl_xor(m, off, 64), __shfl_xor(sacc, off, 64));
  }
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
    smx[wave] = m;
    ssm[wave] = sacc;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) {
      argmax_merge(bk, bi, sk[w], si[w]);
      lse_merge(m, sacc, smx[w], ssm[w]);
    }
    for (int j = 0; j < wn; ++j)
      if (s_own[j] && s_win[j] >= 1u && s_win[j] < (uint32_t)V) argmax_merge(bk, bi, total_key(s_val[j]), (int)s_win[j]);
    const int best = bi < V ? bi : 0;  // V == 1 leaves no candidate
    ids[row] = (uint32_t)best;
    if (gen_ids) gen_ids[(size_t)gen_pos[0] * n_lanes + row] = (uint32_t)best;
    if (surprise) surprise[row] = (m + logf(sacc)) - lg[best];
    if (bad && gw.nonfinite) gw.nonfinite[0] = 1;
  }
}

// Sampling at temperature > 0 (sample(), src/inference.rs:128-178) for one
// lane per workgroup, after the same penalty window as greedy_kernel:
//  - the maximum over ids 1..V-1 of the penalised logits;
//  - probs[v] = exp((logit - max) / T) into the lane's row (LDS, or a global
//    scratch row for large vocabularies), the exponential in f64 rounded once
//    to f32 (the correctly rounded f32 value; the reference's f32::exp is
//    within half an ulp plus a hair of it);
//  - their f32 sum in id order by one thread, as the reference adds them;
//  - p = probs / sum in place, then the top_k candidates in (probability
//    desc, id asc) order by top_k rounds of a workgroup arg-max over the
//    threads' own best candidates;
//  - the top_p cut, the mass, one gen_range_f32(0, mass) draw from the lane's
//    SimpleRng and the running-sum match, in one thread.
// The surprise is the raw logits' logsumexp minus the chosen one, computed as
// greedy_kernel computes it.
constexpr int kMaxSampleTopK = 64;

struct SampleArgs {
  float temperature = 0.0f, top_p = 1.0f;
  int top_k = 1;
  unsigned long long* rng = nullptr;  // [lanes] SimpleRng states
  float* probs = nullptr;             // [lanes, V] scratch
  int* bad_mass = nullptr;            // raised on an invalid probability mass
};

// (pa, va) ranks before (pb, vb): higher probability, then lower id.
__device__ __forceinline__ bool ranks_before(float pa, int va, float pb, int vb) {
  return pa > pb || (pa == pb && va < vb);
}

// Vocabularies up to this size keep the lane's probability row in LDS, where
// the one-thread ordered sum reads it at LDS latency; larger ones use the
// global scratch row.
constexpr int kSampleLdsMaxV = 36 * 1024;
constexpr int kWinBloomWords = 64;  // 2048-bit filter of the penalty window ids

template <bool ROW_LDS>
__global__ __launch_bounds__(256) void sample_kernel(const float* __restrict__ logits, int V,
                                                     uint32_t* __restrict__ ids,
                                                     uint32_t* __restrict__ gen_ids,
                                                     const int* __restrict__ gen_pos, int n_lanes,
                                                     float* __restrict__ surprise, GreedyWindow gw, SampleArgs sa) {
  constexpr int H = pssa_hip_lanes::kHist;
  extern __shared__ __attribute__((aligned(16))) float s_row[];
  __shared__ uint32_t s_win[H];
  __shared__ float s_val[H];
  __shared__ uint32_t s_bloom[kWinBloomWords];
  __shared__ int s_n;
  __shared__ float smx[4], ssm[4], s_pm[4];
  __shared__ float s_bp[2][4];
  __shared__ int s_bv[2][4];
  __shared__ float s_max, s_sum;
  __shared__ float s_selp[kMaxSampleTopK];
  __shared__ int s_selv[kMaxSampleTopK];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* lg = logits + (size_t)row * V;
  float* pr = ROW_LDS ? s_row : sa.probs + (size_t)row * V;
  const bool pen = gw.penalty > 1.0f && gw.hist != nullptr;
  if (tid < kWinBloomWords) s_bloom[tid] = 0u;
  if (gw.hist && tid == 0) {
    int n = gw.hist_n[row], pos = gw.hist_pos[row];
    if (gw.append_row_id) {
      gw.hist[(size_t)row * H + pos] = ids[row];
      pos = (pos + 1) % H;
      n = n < H ? n + 1 : H;
      gw.hist_pos[row] = pos;
      gw.hist_n[row] = n;
    }
    s_n = pen ? n : 0;
    for (int j = 0; j < n && pen; ++j) s_win[j] = gw.hist[(size_t)row * H + (pos - n + j + H) % H];
  }
  __syncthreads();
  const int wn = s_n;
  // Penalised logits of the window ids: each distinct id divided (positive) or
  // multiplied by the penalty once per occurrence, kept at its first entry.
  if (wave == 0 && lane < wn) {
    const uint32_t id = s_win[lane];
    int c = 0;
    for (int j = 0; j < wn; ++j) c += s_win[j] == id;
    float l = id < (uint32_t)V ? lg[id] : 0.0f;
    for (int q = 0; q < c; ++q) l = l > 0.0f ? l / gw.penalty : l * gw.penalty;
    s_val[lane] = l;
    atomicOr(&s_bloom[(id >> 5) & (kWinBloomWords - 1)], 1u << (id & 31));
  }
  __syncthreads();
  // An id whose filter bit is clear is not in the window.
  auto plogit = [&](int v) {
    if (s_bloom[(v >> 5) & (kWinBloomWords - 1)] & (1u << (v & 31)))
      for (int j = 0; j < wn; ++j)
        if (s_win[j] == (uint32_t)v) return s_val[j];
    return lg[v];
  };

  // Maximum of the penalised logits over 1..V-1; logsumexp of the raw ones.
  float mx = -INFINITY, m = -INFINITY, sacc = 0.0f;
  int bad = 0;
  for (int v0 = 0; v0 < V; v0 += 256 * GR_CHUNK) {
    float x[GR_CHUNK];
#pragma unroll
    for (int k = 0; k < GR_CHUNK; ++k) {
      const int v = v0 + k * 256 + tid;
      x[k] = v < V ? lg[v] : -INFINITY;
    }
    float cm = -INFINITY;
#pragma unroll
    for (int k = 0; k < GR_CHUNK; ++k) {
      const int v = v0 + k * 256 + tid;
      if (v < V) bad |= !isfinite(x[k]);
      if (v >= 1 && v < V) mx = fmaxf(mx, wn ? plogit(v) : x[k]);
      cm = fmaxf(cm, x[k]);
    }
    float cs = 0.0f;
    if (cm != -INFINITY) {
#pragma unroll
      for (int k = 0; k < GR_CHUNK; ++k) cs += expf(x[k] - cm);
    }
    lse_merge(m, sacc, cm, cs);
  }
  bad = __syncthreads_or(bad);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    lse_merge(m, sacc, __shfl_xor(m, off, 64), __shfl_xor(sacc, off, 64));
  }
  if (lane == 0) {
    smx[wave] = m;
    ssm[wave] = sacc;
    s_pm[wave] = mx;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) lse_merge(m, sacc, smx[w], ssm[w]);
    s_max = fmaxf(fmaxf(s_pm[0], s_pm[1]), fmaxf(s_pm[2], s_pm[3]));
  }
  __syncthreads();
  const float top = s_max;
  const float temp = sa.temperature;
  // Subtract before dividing (src/inference.rs:139-142).
  for (int v = tid; v < V; v += 256)
    pr[v] = v == 0 ? 0.0f : (float)exp((double)((plogit(v) - top) / temp));
  __syncthreads();
  if (tid == 0) {
    // Adding probs[0] = 0 first leaves the sum +0, so the float4 reads can
    // start at id 0; the adds stay one at a time in id order.
    float sum = 0.0f;
    const int v4 = ROW_LDS ? V & ~3 : 0;
#pragma unroll 8
    for (int v = 0; v < v4; v += 4) {
      const float4 q = *reinterpret_cast<const float4*>(pr + v);
      sum += q.x;
      sum += q.y;
      sum += q.z;
      sum += q.w;
    }
    for (int v = v4 > 1 ? v4 : 1; v < V; ++v) sum += pr[v];
    s_sum = sum;
  }
  __syncthreads();
  const float sum = s_sum;
  const bool mass_ok = isfinite(sum) && sum > 0.0f;
  const int K = mass_ok ? min(V - 1, min(sa.top_k, kMaxSampleTopK)) : 0;
  if (K > 0) {
    for (int v = 1 + tid; v < V; v += 256) pr[v] = pr[v] / sum;
  }
  // Each thread keeps the best of its ids that rank after the last choice.
  // A choice ranks before every id not yet chosen, so only the thread that
  // owned it has to search again.
  float bp = -1.0f;
  int bv = INT32_MAX;
  auto own_best = [&](float lp, int lv) {
    bp = -1.0f;
    bv = INT32_MAX;
    for (int v = 1 + tid; v < V; v += 256) {
      const float p = pr[v];
      if (ranks_before(lp, lv, p, v) && ranks_before(p, v, bp, bv)) {
        bp = p;
        bv = v;
      }
    }
  };
  own_best(INFINITY, -1);
  for (int r = 0; r < K; ++r) {
    float wp = bp;
    int wv = bv;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float op = __shfl_xor(wp, off, 64);
      const int ov = __shfl_xor(wv, off, 64);
      if (ranks_before(op, ov, wp, wv)) {
        wp = op;
        wv = ov;
      }
    }
    // Two slots alternate by round, so one barrier per round suffices.
    if (lane == 0) {
      s_bp[r & 1][wave] = wp;
      s_bv[r & 1][wave] = wv;
    }
    __syncthreads();
    float gp = s_bp[r & 1][0];
    int gv = s_bv[r & 1][0];
    for (int w = 1; w < 4; ++w)
      if (ranks_before(s_bp[r & 1][w], s_bv[r & 1][w], gp, gv)) {
        gp = s_bp[r & 1][w];
        gv = s_bv[r & 1][w];
      }
    if (tid == 0) {
      s_selp[r] = gp;
      s_selv[r] = gv;
    }
    if (bv == gv) own_best(gp, gv);
  }
  __syncthreads();
  if (tid == 0) {
    int best = 0;
    if (!mass_ok) {
      if (sa.bad_mass) sa.bad_mass[0] = 1;
    } else {
      int cutoff = K;
      float cumulative = 0.0f;
      for (int i = 0; i < K; ++i) {
        cumulative += s_selp[i];
        if (cumulative >= sa.top_p) {
          cutoff = i + 1;
          break;
        }
      }
      const int nf = cutoff > 1 ? cutoff : 1;
      float mass = 0.0f;
      for (int i = 0; i < nf; ++i) mass += s_selp[i];
      // SimpleRng::next_u32 (xorshift64*) and gen_range_f32(0, mass)
      // (src/linalg.rs:13-27).
      unsigned long long x = sa.rng[row];
      x ^= x >> 12;
      x ^= x << 25;
      x ^= x >> 27;
      sa.rng[row] = x;
      const uint32_t u = (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
      const float norm = (float)u / (float)4294967295u;
      const float draw = norm * mass;  // low + norm * (high - low) with low = 0
      float running = 0.0f;
      best = s_selv[nf - 1];
      for (int i = 0; i < nf; ++i) {
        running += s_selp[i];
        if (draw <= running) {
          best = s_selv[i];
          break;
        }
      }
    }
    ids[row] = (uint32_t)best;
    if (gen_ids) gen_ids[(size_t)gen_pos[0] * n_lanes + row] = (uint32_t)best;
    if (surprise) surprise[row] = (m + logf(sacc)) - lg[best];
    if (bad && gw.nonfinite) gw.nonfinite[0] = 1;
  }
}

// The lanes' choice from L->logits: greedy at temperature 0, sampled above.
static Status launch_choice(pssa_hip_lanes* L, size_t n_lanes, const GreedyWindow& gw, uint32_t* gen_ids,
                            const int* gen_pos, float* surprise) {
  const hipStream_t st = L->ctx->stream;
  const int V = (int)L->model->cfg.d_vocab;
  if (L->temperature > 0.0f) {
    SampleArgs sa;
    sa.temperature = L->temperature;
    sa.top_p = L->top_p;
    sa.top_k = L->top_k;
    sa.rng = L->rng.as<unsigned long long>();
    sa.probs = L->probs.as<float>();
    sa.bad_mass = L->nonfinite.as<int>() + 2;
    if (V <= kSampleLdsMaxV)
      sample_kernel<true><<<(unsigned)n_lanes, 256, (size_t)V * 4, st>>>(
          L->logits.as<float>(), V, L->ids.as<uint32_t>(), gen_ids, gen_pos, (int)n_lanes, surprise, gw, sa);
    else
      sample_kernel<false><<<(unsigned)n_lanes, 256, 0, st>>>(L->logits.as<float>(), V, L->ids.as<uint32_t>(),
                                                              gen_ids, gen_pos, (int)n_lanes, surprise, gw, sa);
    PSSA_LAUNCH_CHECK("sample");
  } else {
    greedy_kernel<<<(unsigned)n_lanes, 256, 0, st>>>(L->logits.as<float>(), V, L->ids.as<uint32_t>(), gen_ids,
                                                     gen_pos, (int)n_lanes, surprise, gw);
    PSSA_LAUNCH_CHECK("greedy");
  }
  return Status::Ok();
}

// Per-layer operand pointers of the plastic write kernels (one launch covers
// every block).
static_assert(kMaxDepth <= 32, "ValueCaps holds one cap per block");

struct PlasticArgs {
  float* keys[kMaxDepth];
  float* norm_sq[kMaxDepth];
  float* values[kMaxDepth];
  void* values_t[kMaxDepth];
  float* conf[kMaxDepth];
  unsigned long long* last_seen[kMaxDepth];
  int* meta[kMaxDepth];
  float* up[kMaxDepth];
  const float* slow[kMaxDepth];
  void* u_eff[kMaxDepth];
  const float* tap_q;    // [depth, lanes, k]
  const float* tap_z;    // [depth, lanes, d]
  const float* vsrc;     // [depth, lanes, d] the values a bank write stores (tap_z, capped where a cap is set)
  const float* tap_a;    // [depth, lanes, d]
  const float* tap_act;  // [depth, lanes, r]
  const float* surprise; // [lanes]
  float* rate;           // [depth, lanes]
  int* writer;           // [depth, C]: the lane whose value a slot takes this step, or -1
  float* hgate[kMaxDepth];               // hybrid write gate per slot
  unsigned long long* hage[kMaxDepth];   // hybrid age per slot
  int hybrid[kMaxDepth];                 // block reads (and writes) through the hybrid path
  const float* gmean;    // [depth, lanes] mean memory-injection gate (hybrid blocks)
  const unsigned long long* step;
  int lanes, C, dk, d, r, wt_bf16;
};

__device__ __forceinline__ uint16_t to_bf16(float v) { return bf16_bits_dev(v); }

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// up[i,q] += rate_l * clamp(z_l[i] - a_l[i], -4, 4) * act_l[q] for lanes l in
// order (rounded as the reference: (rate * err) * act, then the add), then
// the GEMM operand u_eff = up + slow in the weight type.  blockIdx.y = block;
// a workgroup owns hb_i latent rows x r columns and first stages the clamped
// errors of its rows, every lane's activations and the rates in LDS, so each
// thread's lane-ordered chain runs out of LDS.
__global__ __launch_bounds__(256) void hebbian_kernel(PlasticArgs p, int hb_i) {
  extern __shared__ float hb_smem[];
  const int l = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
  const int i0 = blockIdx.x * hb_i, n = p.lanes, r = p.r, d = p.d;
  float* serr = hb_smem;          // [lanes][hb_i]
  float* sact = serr + n * hb_i;  // [lanes][r]
  float* srate = sact + n * r;    // [lanes]
  const float* z = p.tap_z + (size_t)l * n * d;
  const float* a = p.tap_a + (size_t)l * n * d;
  // Loads at a clamped in-range column, masked after: a load under the
  // column guard ended its block with a full wait, one round trip per element.
#pragma unroll 8
  for (int e = tid; e < n * hb_i; e += nt) {
    const int ln = e / hb_i, i = i0 + e % hb_i;
    const size_t o = (size_t)ln * d + min(i, d - 1);
    const float v = fminf(fmaxf(z[o] - a[o], -4.0f), 4.0f);
    serr[e] = i < d ? v : 0.0f;
  }
  const float* act = p.tap_act + (size_t)l * n * r;
#pragma unroll 8
  for (int e = tid; e < n * r; e += nt) sact[e] = act[e];
  for (int e = tid; e < n; e += nt) srate[e] = p.rate[(size_t)l * n + e];
  __syncthreads();
  const int ii = tid / r, q = tid % r, i = i0 + ii;
  if (ii >= hb_i || i >= d) return;
  const int e = i * r + q;
  float u = p.up[l][e];
#pragma unroll 8
  for (int ln = 0; ln < n; ++ln)
    u = __fadd_rn(u, __fmul_rn(__fmul_rn(srate[ln], serr[ln * hb_i + ii]), sact[ln * r + q]));
  p.up[l][e] = u;
  const float eff = u + p.slow[l][e];
  if (p.wt_bf16)
    static_cast<uint16_t*>(p.u_eff[l])[e] = to_bf16(eff);
  else
    static_cast<float*>(p.u_eff[l])[e] = eff;
}

// 0.02 / (1 + |z_final|) per (block, lane), the Hebbian rate of
// dream_replay_value, one wave per (block, lane).  The norm's square is a
// sequential f64 sum in the reference; here the wave sums it in any order,
// which is within RATE_SUM_REL (relative) of that sum, and the sequential sum
// runs only when the f32 rounding of the norm is not settled by that bound.
constexpr double RATE_SUM_REL = 4e-13;

__device__ __forceinline__ float rate_norm(double acc) { return (float)fmin(sqrt(acc), (double)FLT_MAX); }

__global__ __launch_bounds__(256) void hebbian_rate_kernel(PlasticArgs p) {
  const int l = blockIdx.y, lane = threadIdx.x & 63;
  const int ln = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (ln >= p.lanes) return;
  const float* zr = p.tap_z + ((size_t)l * p.lanes + ln) * p.d;
  double acc = 0.0;
  for (int i = lane; i < p.d; i += 64) acc = fma((double)zr[i], (double)zr[i], acc);
  acc = wave_sum_f64(acc);
  float tn = rate_norm(acc);
  if (rate_norm(acc * (1.0 - RATE_SUM_REL)) != rate_norm(acc * (1.0 + RATE_SUM_REL)) && lane == 0) {
    double seq = 0.0;
    {
#pragma clang fp contract(off)
      for (int i = 0; i < p.d; ++i) seq = seq + (double)zr[i] * (double)zr[i];
    }
    tn = rate_norm(seq);
  }
  if (lane == 0) p.rate[(size_t)l * p.lanes + ln] = 0.02f / (1.0f + tn);
}

// Protected writes of every block's bank (blockIdx.x = block) for all lanes,
// in lane order.  The accept/defend decisions depend only on the bank's
// counters, confidences and ages: those are staged in LDS, thread 0 makes
// the decisions sequentially, and the slot contents are then copied in
// parallel, each slot from the last lane in order that wrote it.
__global__ __launch_bounds__(256) void bank_write_kernel(PlasticArgs p) {
  extern __shared__ unsigned char bw_smem[];
  const int l = blockIdx.x, C = p.C, tid = threadIdx.x;
  unsigned long long* s_last = reinterpret_cast<unsigned long long*>(bw_smem);  // [C]
  float* s_conf = reinterpret_cast<float*>(s_last + C);                          // [C]
  int* writer = reinterpret_cast<int*>(s_conf + C);                              // [C]
  float* s_sp = reinterpret_cast<float*>(writer + C);                            // [lanes]
  float* conf = p.conf[l];
  unsigned long long* last_seen = p.last_seen[l];
  for (int c = tid; c < C; c += blockDim.x) {
    writer[c] = -1;
    s_conf[c] = conf[c];
    s_last[c] = last_seen[c];
  }
  for (int ln = tid; ln < p.lanes; ln += blockDim.x) s_sp[ln] = p.surprise[ln];
  __syncthreads();
  if (tid < 64) {
    // Wave 0 runs the decisions in lane order; every lane follows the same
    // (uniform) path, lane 0 stores.  Surprises come 64 at a time from
    // registers; the write-head slot's confidence, age and gate gain stay in
    // registers until the head moves.
    const int lane = tid;
    const unsigned long long cur = p.step[0] + 1;
    int* meta = p.meta[l];
    int count = meta[0], head = meta[1];
    float hconf = 0.0f, hgain = 0.0f;
    unsigned long long hlast = 0ull;
    // RateLimiterGate::apply_refractory_overwrite (src/defense.rs:45-67):
    // gain = max((1 - e^(-dt/60))^2, 0.005) with dt = cur - last_seen.
    auto load_head = [&]() {
      hconf = s_conf[head];
      hlast = s_last[head];
      const float dt = (float)(cur > hlast ? cur - hlast : 0ull);
      const float lin = 1.0f - expf(-dt / 60.0f);
      hgain = fmaxf(lin * lin, 0.005f);
    };
    if (count >= C) load_head();
    for (int base = 0; base < p.lanes; base += 64) {
      const float mysp = base + lane < p.lanes ? s_sp[base + lane] : 0.0f;
      const int nk = min(64, p.lanes - base);
      for (int k = 0; k < nk; ++k) {
        const float sp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mysp), k));
        if (!(sp > 3.5f)) continue;
        const int ln = base + k;
        if (count < C) {  // insert() into a free slot
          const int idx = count++;
          if (lane == 0) {
            s_conf[idx] = 1.0f;
            s_last[idx] = cur;
            writer[idx] = ln;
          }
          if (count == C) load_head();
          continue;
        }
        const float damage = 0.08f * sp * hgain;
        if (hconf > damage) {  // defended: the age resets, so dt = 0 next time
          hconf -= damage;
          hlast = cur;
          hgain = 0.005f;
          continue;
        }
        if (lane == 0) {
          s_conf[head] = 1.0f;
          s_last[head] = cur;
          writer[head] = ln;
        }
        head = (head + 1) % C;
        load_head();
      }
    }
    if (count >= C && lane == 0) {
      s_conf[head] = hconf;
      s_last[head] = hlast;
    }
    if (lane == 0) {
      meta[0] = count;
      meta[1] = head;
    }
  }
  __syncthreads();
  for (int c = tid; c < C; c += blockDim.x) {
    conf[c] = s_conf[c];
    last_seen[c] = s_last[c];
    p.writer[(size_t)l * C + c] = writer[c];
  }
}

// Slot contents of the writes bank_write_kernel decided: a workgroup covers
// 64 slots x 64 latent columns of one block; values are copied row-wise and
// the GEMM operand values_t [d, C] is written through an LDS transpose, both
// coalesced.  The workgroups of the first column tile also copy the keys and
// their squared norms (squared_norm, src/memory.rs:181-192: sequential f64).
__global__ __launch_bounds__(256) void bank_copy_kernel(PlasticArgs p) {
  __shared__ int w[64];
  __shared__ float tile[64][65];
  const int l = blockIdx.z, c0 = blockIdx.x * 64, j0 = blockIdx.y * 64, tid = threadIdx.x;
  const int C = p.C, d = p.d;
  const size_t n = p.lanes;
  if (tid < 64) w[tid] = c0 + tid < C ? p.writer[(size_t)l * C + c0 + tid] : -1;
  __syncthreads();
  for (int e = tid; e < 64 * 64; e += 256) {
    const int cc = e >> 6, jj = e & 63, c = c0 + cc, j = j0 + jj;
    if (w[cc] >= 0 && j < d) {
      const float v = p.vsrc[((size_t)l * n + w[cc]) * d + j];
      p.values[l][(size_t)c * d + j] = v;
      tile[cc][jj] = v;
    }
  }
  __syncthreads();
  for (int e = tid; e < 64 * 64; e += 256) {
    const int jj = e >> 6, cc = e & 63, c = c0 + cc, j = j0 + jj;
    if (w[cc] >= 0 && j < d) {
      if (p.wt_bf16)
        static_cast<uint16_t*>(p.values_t[l])[(size_t)j * C + c] = to_bf16(tile[cc][jj]);
      else
        static_cast<float*>(p.values_t[l])[(size_t)j * C + c] = tile[cc][jj];
    }
  }
  if (blockIdx.y == 0 && tid < 64 && w[tid] >= 0) {
    const int c = c0 + tid;
    // insert / insert_gated reset the slot's hybrid metadata (src/memory.rs:
    // 300-301, 497): gate 1.0, or the write gate on a hybrid block; age 0.
    p.hgate[l][c] = p.hybrid[l] ? p.gmean[(size_t)l * n + w[tid]] : 1.0f;
    p.hage[l][c] = 0ull;
    const float* kq = p.tap_q + ((size_t)l * n + w[tid]) * p.dk;
    double acc = 0.0;
    {
#pragma clang fp contract(off)
      for (int j = 0; j < p.dk; ++j) {
        const float kv = kq[j];
        p.keys[l][(size_t)c * p.dk + j] = kv;
        acc = acc + (double)kv * (double)kv;
      }
    }
    float v = (float)acc;
    if (acc < 1.0 && v == 1.0f) v = __uint_as_float(0x3f7fffffu);
    p.norm_sq[l][c] = v;
  }
}

__global__ void advance_kernel(unsigned long long* __restrict__ step, int* __restrict__ gen_pos) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    step[0] += 1;
    gen_pos[0] += 1;
  }
}

__global__ void advance_pos_kernel(int* __restrict__ gen_pos) {
  if (threadIdx.x == 0 && blockIdx.x == 0) gen_pos[0] += 1;
}

}  // namespace

size_t bank_write_lds(int capacity, int lanes) { return (size_t)capacity * (8 + 4 + 4) + (size_t)lanes * 4; }
int hebbian_rows(int rank) { return rank >= 256 ? 1 : 256 / rank; }
size_t hebbian_lds(int rank, int lanes) {
  return ((size_t)lanes * hebbian_rows(rank) + (size_t)lanes * rank + (size_t)lanes) * sizeof(float);
}

Status init_decode_attributes() {
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&bank_write_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&hebbian_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&sample_kernel<true>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, kSampleLdsMaxV * 4));
  return Status::Ok();
}

Status run_greedy_from_logits(pssa_hip_lanes* L, size_t n_lanes, bool record) {
  const hipStream_t st = L->ctx->stream;
  GreedyWindow gw;
  gw.hist = L->hist.as<uint32_t>();
  gw.hist_n = L->hist_n.as<int>();
  gw.hist_pos = L->hist_pos.as<int>();
  gw.penalty = L->rep_penalty;
  gw.nonfinite = L->nonfinite.as<int>();
  PSSA_RETURN_IF(launch_choice(L, n_lanes, gw, record ? L->gen_ids.as<uint32_t>() : nullptr,
                               record ? L->gen_pos.as<int>() : nullptr, nullptr));
  if (record) {
    advance_pos_kernel<<<1, 64, 0, st>>>(L->gen_pos.as<int>());
    PSSA_LAUNCH_CHECK("advance");
  }
  return Status::Ok();
}

Status run_decode_step(pssa_hip_lanes* L, size_t n_lanes, bool plastic) {
  const pssa_hip_model* M = L->model;
  const pssa_hip_config& c = M->cfg;
  const hipStream_t st = L->ctx->stream;
  const int d = (int)c.d_latent, k = (int)c.d_mem_key, r = (int)c.adapter_rank, C = (int)c.mem_capacity;
  const size_t n = n_lanes;
  PSSA_RETURN_IF(run_prefill(L, n_lanes, 1, plastic, false));
  // The Hebbian update (src/pssa.rs:1814-1832) reads only the forward's taps
  // and writes only the fast weights, which nothing else in the step reads:
  // it runs on an auxiliary stream beside the choice and the bank writes,
  // and the step counter's advance waits for both.
  const hipStream_t hs = L->aux_stream[0];
  if (plastic) {
    PSSA_HIP_TRY(hipEventRecord(L->ev_tail_fork, st));
    PSSA_HIP_TRY(hipStreamWaitEvent(hs, L->ev_tail_fork, 0));
  }
  GreedyWindow gw;
  gw.hist = L->hist.as<uint32_t>();
  gw.hist_n = L->hist_n.as<int>();
  gw.hist_pos = L->hist_pos.as<int>();
  gw.penalty = L->rep_penalty;
  gw.append_row_id = 1;  // the token this step consumed
  gw.nonfinite = L->nonfinite.as<int>();
  PSSA_RETURN_IF(launch_choice(L, n, gw, L->gen_ids.as<uint32_t>(), L->gen_pos.as<int>(), L->surprise.as<float>()));
  if (plastic) {
    L->tap_lanes = n;
    PlasticArgs p{};
    for (size_t l = 0; l < c.depth; ++l) {
      const DevBlock& B = M->blocks[l];
      p.keys[l] = B.keys.as<float>();
      p.norm_sq[l] = B.norm_sq.as<float>();
      p.values[l] = B.values.as<float>();
      p.values_t[l] = B.values_t.p;
      p.conf[l] = B.conf.as<float>();
      p.last_seen[l] = B.last_seen.as<unsigned long long>();
      p.hgate[l] = B.hgate.as<float>();
      p.hage[l] = B.hage.as<unsigned long long>();
      p.hybrid[l] = B.hybrid ? 1 : 0;
      p.meta[l] = B.meta.as<int>();
      p.up[l] = B.u_fast.as<float>();
      p.slow[l] = B.u_slow.as<float>();
      p.u_eff[l] = B.u_eff.p;
    }
    p.tap_q = L->tap_q.as<float>();
    p.tap_z = L->tap_z.as<float>();
    // Bank writes store capped copies of z_final where a block has a value
    // cap (insert's clamp, src/memory.rs:290-297); the Hebbian update keeps
    // the raw z_final.
    ValueCaps caps{};
    bool any_cap = false;
    for (size_t l = 0; l < c.depth; ++l) {
      caps.c[l] = M->blocks[l].value_cap;
      any_cap |= caps.c[l] > 0.0f;
    }
    p.vsrc = p.tap_z;
    if (any_cap) {
      PSSA_RETURN_IF(launch_clamp_rows(st, L->tap_z.as<float>(), L->tap_zcap.as<float>(), (int)(c.depth * n), d,
                                       (size_t)d, caps, (int)n, L->nonfinite.as<int>() + 1));
      p.vsrc = L->tap_zcap.as<float>();
    }
    p.tap_a = L->tap_a.as<float>();
    p.tap_act = L->tap_act.as<float>();
    p.surprise = L->surprise.as<float>();
    p.rate = L->hebb_rate.as<float>();
    p.writer = L->bank_writer.as<int>();
    p.gmean = L->tap_gmean.as<float>();
    p.step = M->step.as<unsigned long long>();
    p.lanes = (int)n;
    p.C = C;
    p.dk = k;
    p.d = d;
    p.r = r;
    p.wt_bf16 = M->dtype == PSSA_HIP_BF16 ? 1 : 0;
    const int depth = (int)c.depth;
    hebbian_rate_kernel<<<dim3((unsigned)((n + 3) / 4), depth), 256, 0, hs>>>(p);
    PSSA_LAUNCH_CHECK("hebbian_rate");
    const int hb_i = hebbian_rows(r);
    hebbian_kernel<<<dim3((unsigned)((d + hb_i - 1) / hb_i), depth), hb_i * r, hebbian_lds(r, (int)n), hs>>>(p,
                                                                                                         hb_i);
    PSSA_LAUNCH_CHECK("hebbian");
    PSSA_HIP_TRY(hipEventRecord(L->ev_tail_join, hs));
    bank_write_kernel<<<depth, 256, bank_write_lds(C, (int)n), st>>>(p);
    PSSA_LAUNCH_CHECK("bank_write");
    bank_copy_kernel<<<dim3((unsigned)((C + 63) / 64), (unsigned)((d + 63) / 64), depth), 256, 0, st>>>(p);
    PSSA_LAUNCH_CHECK("bank_copy");
    PSSA_HIP_TRY(hipStreamWaitEvent(st, L->ev_tail_join, 0));
    advance_kernel<<<1, 64, 0, st>>>(M->step.as<unsigned long long>(), L->gen_pos.as<int>());
  } else {
    advance_pos_kernel<<<1, 64, 0, st>>>(L->gen_pos.as<int>());
  }
  PSSA_LAUNCH_CHECK("advance");
  return Status::Ok();
}

}  // namespace pssa

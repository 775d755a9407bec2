// CPU oracle for the PSSA inference forward path -- TEST INFRASTRUCTURE ONLY.
//
// A plain restatement of the reference's scalar CPU path (Rust crate
// Sparticle62ops/pssa).  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg use it, as the checker and as the CPU baseline.  The
// product path never links it.
//
// Build: g++ -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).  Rust
// evaluates a*b+c as two rounded operations; so does this file.  The only
// fused multiply-adds are the explicit _mm256_fmadd_ps of the AVX2 dot tree,
// exactly where the reference uses them.
#include "pssa_oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <memory>
#include <thread>
#include <utility>
#include <vector>

namespace {

int g_dot_avx2 = 1;

// The bf16 mode of this build (weights and every GEMM's activation operand in
// bf16, fp32 accumulation, fp32 state path; the reference has no such mode,
// all its parameters are f32, src/pssa.rs:11-205).  When set, block_forward
// rounds each product's activation operand to bf16 where the device does;
// the weights are rounded by the caller.  Off: the reference's arithmetic.
int g_bf16_ops = 0;
// Recurrent depth loops (set_loops, src/pssa.rs:2171-2184): every block runs
// this many passes per token, each with its own carry; a lane's state is
// [depth, loops, d_latent * d_state] (loop 0 first, as
// copy_recurrent_state_to, src/pssa.rs:2263-2281).
size_t g_loops = 1;

// Round to the nearest bf16 (ties to even), widened back to f32.
inline float bf16r(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  u &= 0xFFFF0000u;
  std::memcpy(&f, &u, 4);
  return f;
}

// --- src/linalg.rs:1-28 SimpleRng (xorshift64*) --------------------------------
struct Rng {
  uint64_t state;
  explicit Rng(uint64_t seed) : state(seed == 0 ? 0x853c49e6748fea9bULL : seed) {}
  uint32_t next_u32() {
    uint64_t x = state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    state = x;
    return (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
  }
  // gen_range_f32: (u32 as f32) / (u32::MAX as f32), then low + norm*(high-low).
  float gen_range(float low, float high) {
    float norm = (float)next_u32() / (float)UINT32_MAX;
    return low + norm * (high - low);
  }
  // Standard normal for the baseline initialisation (Box-Muller in f64).
  double normal() {
    uint32_t a = next_u32();
    uint32_t b = next_u32();
    double u1 = ((double)a + 1.0) / 4294967296.0;
    double u2 = (double)b / 4294967296.0;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
};

// --- src/linalg.rs:282-298 dot_slice_portable ----------------------------------
float dot_portable(const float* a, const float* b, size_t n) {
  size_t i = 0;
  float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
  while (i + 4 <= n) {
    acc0 += a[i] * b[i];
    acc1 += a[i + 1] * b[i + 1];
    acc2 += a[i + 2] * b[i + 2];
    acc3 += a[i + 3] * b[i + 3];
    i += 4;
  }
  float sum = (acc0 + acc1) + (acc2 + acc3);
  while (i < n) {
    sum += a[i] * b[i];
    i++;
  }
  return sum;
}

// --- src/linalg.rs:210-280 dot_slice_avx2_fma ----------------------------------
__attribute__((target("avx2,fma"))) float dot_avx2(const float* a, const float* b, size_t n) {
  size_t i = 0;
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
  while (i + 32 <= n) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), acc1);
    acc2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), acc2);
    acc3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), acc3);
    i += 32;
  }
  while (i + 8 <= n) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
    i += 8;
  }
  __m256 lanes = _mm256_add_ps(_mm256_add_ps(acc0, acc1), _mm256_add_ps(acc2, acc3));
  __m128 folded = _mm_add_ps(_mm256_castps256_ps128(lanes), _mm256_extractf128_ps(lanes, 1));
  __m128 pair = _mm_hadd_ps(folded, folded);
  float sum = _mm_cvtss_f32(_mm_hadd_ps(pair, pair));
  while (i < n) {
    sum += a[i] * b[i];
    i++;
  }
  return sum;
}

// --- src/linalg.rs:184-199 dot_slice dispatch ---------------------------------
inline float dot(const float* a, const float* b, size_t n) {
  if (g_dot_avx2 && (n == 8 || n >= 16)) return dot_avx2(a, b, n);
  return dot_portable(a, b, n);
}

// --- src/linalg.rs:548-555 ------------------------------------------------------
inline float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
inline float softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// --- src/pssa.rs:109-116 ParamMatrix::matvec ------------------------------------
inline void matvec(const float* w, size_t rows, size_t cols, const float* x, float* out) {
  for (size_t r = 0; r < rows; r++) out[r] = dot(w + r * cols, x, cols);
}

// --- src/memory.rs:181-192 squared_norm (f64 accumulation) ---------------------
inline double squared_norm_f64(const float* p, size_t n) {
  double s = 0.0;
  for (size_t i = 0; i < n; i++) s += (double)p[i] * (double)p[i];
  return s;
}
inline float squared_norm(const float* p, size_t n) {
  double norm = squared_norm_f64(p, n);
  if (norm < 1.0 && (float)norm == 1.0f) {
    uint32_t bits;
    float one = 1.0f;
    std::memcpy(&bits, &one, 4);
    bits -= 1;
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
  }
  return (float)norm;
}

// --- src/memory.rs:173 MAX_PROJECTED_RADIUS; 194-211 diffeomorphic_project -----
const double kMaxProjectedRadius = 1.0 - 8.0 * (double)FLT_EPSILON;
inline float project(const float* q, float* out, size_t n) {
  double r = std::sqrt(squared_norm_f64(q, n));
  double scale = (r == 0.0) ? 1.0 : std::min(r / (1.0 + r), kMaxProjectedRadius) / r;
  for (size_t i = 0; i < n; i++) out[i] = (float)((double)q[i] * scale);
  return (float)std::min(r, (double)FLT_MAX);
}

// Rust std f64::asinh: ln_1p(ax + ax / (hypot(1, 1/ax) + 1/ax)) with the sign
// of x restored (library/std/src/f64.rs; hypot and ln_1p are the platform libm).
inline double rust_asinh(double x) {
  double ax = std::fabs(x);
  double ix = 1.0 / ax;
  return std::copysign(std::log1p(ax + (ax / (std::hypot(1.0, ix) + ix))), x);
}

// --- src/memory.rs:242-262 poincare_distance ------------------------------------
inline float poincare_distance(const float* u, float u_sq, const float* v, float v_sq, size_t n) {
  double sq = 0.0;
  for (size_t i = 0; i < n; i++) {
    double d = (double)u[i] - (double)v[i];
    sq += d * d;
  }
  double denom = (1.0 - (double)u_sq) * (1.0 - (double)v_sq);
  return (float)(2.0 * rust_asinh(std::sqrt(sq / denom)));
}

inline uint32_t f2u(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
inline float u2f(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// --- src/memory.rs:344-426 retrieve_soft_into (with optional exact top-k) -----
float retrieve(const float* keys, const float* norm_sq, const float* values, size_t count,
               size_t capacity, size_t dk, size_t dv, const float* q, float tau, size_t top_k,
               float* out_val, float* w, uint32_t* out_idx) {
  float q_sq = squared_norm(q, dk);
  if (count == 0) {
    std::fill(out_val, out_val + dv, 0.0f);
    std::fill(w, w + capacity, 0.0f);
    return 0.0f;
  }
  float min_dist = FLT_MAX;
  for (size_t idx = 0; idx < count; idx++) {
    float dist = poincare_distance(q, q_sq, keys + idx * dk, norm_sq[idx], dk);
    min_dist = std::fmin(min_dist, dist);
    w[idx] = dist;
  }
  if (top_k != 0 && top_k < count) {
    // Keep the k smallest (distance bits, slot) pairs, then mix them in slot order.
    std::vector<std::pair<uint32_t, uint32_t>> all(count);
    for (size_t idx = 0; idx < count; idx++) all[idx] = {f2u(w[idx]), (uint32_t)idx};
    std::partial_sort(all.begin(), all.begin() + top_k, all.end());
    std::vector<std::pair<uint32_t, uint32_t>> sel(all.begin(), all.begin() + top_k);
    std::sort(sel.begin(), sel.end(),
              [](const std::pair<uint32_t, uint32_t>& a, const std::pair<uint32_t, uint32_t>& b) {
                return a.second < b.second;
              });
    std::fill(w, w + capacity, 0.0f);
    float sum = 0.0f;
    for (auto& s : sel) sum += expf((min_dist - u2f(s.first)) / tau);
    std::fill(out_val, out_val + dv, 0.0f);
    size_t n = 0;
    for (auto& s : sel) {
      float weight = expf((min_dist - u2f(s.first)) / tau) / sum;
      w[s.second] = weight;
      const float* v = values + (size_t)s.second * dv;
      if (g_bf16_ops)
        for (size_t j = 0; j < dv; j++) out_val[j] += bf16r(weight) * bf16r(v[j]);
      else
        for (size_t j = 0; j < dv; j++) out_val[j] += weight * v[j];
      if (out_idx) out_idx[n++] = s.second;
    }
    if (g_bf16_ops)
      for (size_t j = 0; j < dv; j++) out_val[j] = bf16r(out_val[j]);
    return min_dist;
  }
  float sum = 0.0f;
  for (size_t idx = 0; idx < count; idx++) {
    w[idx] = expf((min_dist - w[idx]) / tau);
    sum += w[idx];
  }
  std::fill(out_val, out_val + dv, 0.0f);
  for (size_t idx = 0; idx < count; idx++) {
    float wi = w[idx] / sum;
    w[idx] = wi;
    const float* v = values + idx * dv;
    if (g_bf16_ops)
      for (size_t j = 0; j < dv; j++) out_val[j] += bf16r(wi) * bf16r(v[j]);
    else
      for (size_t j = 0; j < dv; j++) out_val[j] += wi * v[j];
  }
  if (g_bf16_ops)
    for (size_t j = 0; j < dv; j++) out_val[j] = bf16r(out_val[j]);
  if (out_idx)
    for (size_t i = 0; i < top_k; i++) out_idx[i] = i < count ? (uint32_t)i : 0xFFFFFFFFu;
  return min_dist;
}

inline uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }

// --- src/memory.rs:568-660 retrieve_hybrid_into ----------------------------------
// Slot i's age is age[i] + age_add (the bumps of this pass not yet stored).
float retrieve_hybrid(const float* keys, const float* norm_sq, const float* values, size_t count,
                      size_t capacity, size_t dk, size_t dv, const float* q, float tau, size_t top_k,
                      const float* gate, const uint64_t* age, uint64_t age_add, float lam,
                      float* out_val, float* w, uint32_t* out_idx) {
  if (count == 0) {
    std::fill(out_val, out_val + dv, 0.0f);
    std::fill(w, w + capacity, 0.0f);
    return 0.0f;
  }
  const double log_lam = std::log((double)lam);
  float q_sq = squared_norm(q, dk);
  float min_dist = FLT_MAX;
  std::vector<float> dists(count);
  for (size_t idx = 0; idx < count; idx++) {
    dists[idx] = poincare_distance(q, q_sq, keys + idx * dk, norm_sq[idx], dk);
    min_dist = std::fmin(min_dist, dists[idx]);
  }
  std::vector<char> live(count, 1);
  if (top_k != 0 && top_k < count) {
    std::vector<std::pair<uint32_t, uint32_t>> all(count);
    for (size_t idx = 0; idx < count; idx++) all[idx] = {f2u(dists[idx]), (uint32_t)idx};
    std::partial_sort(all.begin(), all.begin() + top_k, all.end());
    std::fill(live.begin(), live.end(), 0);
    for (size_t i = 0; i < top_k; i++) live[all[i].second] = 1;
    if (out_idx) {
      size_t n = 0;
      for (size_t idx = 0; idx < count; idx++)
        if (live[idx]) out_idx[n++] = (uint32_t)idx;
    }
  }
  std::fill(w, w + capacity, 0.0f);
  float sum = 0.0f;
  for (size_t idx = 0; idx < count; idx++) {
    if (!live[idx]) continue;
    const uint64_t a = sat_add(age ? age[idx] : 0, age_add);
    const float decay = (float)std::exp((double)a * log_lam);
    const float wi = expf((min_dist - dists[idx]) / tau) * (gate ? gate[idx] : 1.0f) * decay;
    w[idx] = wi;
    sum += wi;
  }
  if (sum == 0.0f) {  // fully gated out: the unweighted softmax over the live slots
    for (size_t idx = 0; idx < count; idx++) {
      if (!live[idx]) continue;
      w[idx] = expf((min_dist - dists[idx]) / tau);
      sum += w[idx];
    }
  }
  std::fill(out_val, out_val + dv, 0.0f);
  for (size_t idx = 0; idx < count; idx++) {
    if (!live[idx]) continue;
    const float wi = w[idx] / sum;
    w[idx] = wi;
    const float* v = values + idx * dv;
    if (g_bf16_ops)
      for (size_t j = 0; j < dv; j++) out_val[j] += bf16r(wi) * bf16r(v[j]);
    else
      for (size_t j = 0; j < dv; j++) out_val[j] += wi * v[j];
  }
  if (g_bf16_ops)
    for (size_t j = 0; j < dv; j++) out_val[j] = bf16r(out_val[j]);
  return min_dist;
}

// --- src/defense.rs:18-22, 45-67 --------------------------------------------------
float refractory_gain(uint64_t delta_tokens, float tau) {
  float dt = (float)delta_tokens;
  float linear = 1.0f - expf(-dt / tau);
  return std::fmax(linear * linear, 0.005f);
}

// Scratch for one block's token step (src/pssa.rs:506-620 inference buffers).
struct Scratch {
  std::vector<float> xn, delta, bb, cc, y, qe, qp, mw, mval, g, mp, act, adout, zraw, h1, u, zf;
  std::vector<float> xb, yb, zb;  // bf16-rounded GEMM operands (bf16 mode)
  uint64_t age_add = 1;  // hybrid read: bumps of the current pass not yet stored
  std::vector<float> rates;  // -softplus(a_raw), src/pssa.rs:787-796
  void resize(const oracle_config& c) {
    size_t d = c.d_latent, s = c.d_state, k = c.d_mem_key, C = c.mem_capacity, r = c.adapter_rank;
    xn.assign(d, 0);
    xb.assign(d, 0);
    yb.assign(d, 0);
    zb.assign(d, 0);
    delta.assign(d, 0);
    bb.assign(s, 0);
    cc.assign(s, 0);
    y.assign(d, 0);
    qe.assign(k, 0);
    qp.assign(k, 0);
    mw.assign(C, 0);
    mval.assign(d, 0);
    g.assign(d, 0);
    mp.assign(d, 0);
    act.assign(r, 0);
    adout.assign(d, 0);
    zraw.assign(d, 0);
    h1.assign(2 * d, 0);
    u.assign(d, 0);
    zf.assign(d, 0);
    rates.assign(d * s, 0);
  }
};

void refresh_rates(const oracle_block& b, const oracle_config& c, Scratch& sc) {
  size_t n = c.d_latent * c.d_state;
  for (size_t i = 0; i < n; i++) sc.rates[i] = -softplus(b.a_raw[i]);
}

// --- src/pssa.rs:1072-1116 forward_continuous_inference (norm + projections) ---
// --- src/pssa.rs:1122-1209 forward_continuous_inference_projected -------------
void block_forward(const oracle_block& b, const oracle_config& c, Scratch& sc, float* h,
                   const float* e, float* z_out) {
  const size_t d = c.d_latent, s = c.d_state, k = c.d_mem_key, r = c.adapter_rank;
  const size_t dmlp = 2 * d;
  // 1. affine RMSNorm with a scalar left-to-right sum of squares.
  float sum_sq = 0.0f;
  for (size_t i = 0; i < d; i++) sum_sq += e[i] * e[i];
  float inv_rms = 1.0f / sqrtf(sum_sq / (float)d + 1e-5f);
  for (size_t i = 0; i < d; i++) sc.xn[i] = b.norm_gamma[i] * (e[i] * inv_rms) + b.norm_beta[i];
  // The products' activation operand: x-hat itself, or its bf16 rounding in
  // the bf16 mode (the SSM below always reads the f32 x-hat).
  const float* xg = sc.xn.data();
  if (g_bf16_ops) {
    for (size_t i = 0; i < d; i++) sc.xb[i] = bf16r(sc.xn[i]);
    xg = sc.xb.data();
  }
  // 2. data-dependent projections
  matvec(b.w_delta, d, d, xg, sc.delta.data());
  for (size_t i = 0; i < d; i++) sc.delta[i] = softplus(sc.delta[i]);
  matvec(b.w_b, s, d, xg, sc.bb.data());
  matvec(b.w_c, s, d, xg, sc.cc.data());
  // 3. SSM state update, i outer / j inner
  const float ssm_scale = 1.0f / sqrtf((float)s);
  for (size_t i = 0; i < d; i++) {
    float di = sc.delta[i];
    float yi = 0.0f;
    for (size_t j = 0; j < s; j++) {
      size_t idx = i * s + j;
      float bar_a = expf(di * sc.rates[idx]);
      float bar_b = di * sc.bb[j];
      float hv = bar_a * h[idx] + bar_b * sc.xn[i];
      h[idx] = hv;
      yi += hv * sc.cc[j];
    }
    sc.y[i] = yi;
  }
  // 4. retrieval query, projection, soft read
  const float* yg = sc.y.data();
  if (g_bf16_ops) {
    for (size_t i = 0; i < d; i++) sc.yb[i] = bf16r(sc.y[i]);
    yg = sc.yb.data();
  }
  for (size_t q = 0; q < k; q++) sc.qe[q] = dot(b.w_qx + q * d, xg, d) + dot(b.w_qh + q * d, yg, d);
  project(sc.qe.data(), sc.qp.data(), k);
  if (b.mem_hybrid_enabled)  // src/pssa.rs:1153-1162 (the ages are bumped by the caller)
    retrieve_hybrid(b.mem_keys, b.mem_norm_sq, b.mem_values, b.mem_count, c.mem_capacity, k, d,
                    sc.qp.data(), c.tau_mem, b.mem_top_k, b.mem_hybrid_gate, b.mem_hybrid_age, sc.age_add,
                    b.mem_hybrid_lam, sc.mval.data(), sc.mw.data(), nullptr);
  else
    retrieve(b.mem_keys, b.mem_norm_sq, b.mem_values, b.mem_count, c.mem_capacity, k, d,
             sc.qp.data(), c.tau_mem, b.mem_top_k, sc.mval.data(), sc.mw.data(), nullptr);
  matvec(b.w_gate, d, d, xg, sc.g.data());
  for (size_t i = 0; i < d; i++) sc.g[i] = sigmoid(sc.g[i]);
  matvec(b.w_proj, d, d, sc.mval.data(), sc.mp.data());  // bf16 mode: the readout is already rounded
  // 5. plastic adapter (src/adapter.rs:37-48)
  matvec(b.adapter_down, r, d, xg, sc.act.data());
  for (size_t q = 0; q < r; q++) {
    float hv = sc.act[q];
    sc.act[q] = hv * sigmoid(hv);
  }
  for (size_t i = 0; i < d; i++) {
    float total = 0.0f;
    if (g_bf16_ops)  // the device's operand: bf16(fast + slow) times bf16(act)
      for (size_t q = 0; q < r; q++)
        total += bf16r(b.adapter_up[i * r + q] + b.adapter_slow[i * r + q]) * bf16r(sc.act[q]);
    else
      for (size_t q = 0; q < r; q++) total += (b.adapter_up[i * r + q] + b.adapter_slow[i * r + q]) * sc.act[q];
    sc.adout[i] = total;
  }
  // 6. aggregation and SiLU MLP
  for (size_t i = 0; i < d; i++) sc.zraw[i] = (sc.y[i] * ssm_scale) + (sc.g[i] * sc.mp[i]) + sc.adout[i];
  const float* zg = sc.zraw.data();
  if (g_bf16_ops) {
    for (size_t i = 0; i < d; i++) sc.zb[i] = bf16r(sc.zraw[i]);
    zg = sc.zb.data();
  }
  matvec(b.mlp_w1, dmlp, d, zg, sc.h1.data());
  for (size_t i = 0; i < dmlp; i++) {
    float hv = sc.h1[i];
    sc.h1[i] = g_bf16_ops ? bf16r(hv * sigmoid(hv)) : hv * sigmoid(hv);
  }
  matvec(b.mlp_w2, d, dmlp, sc.h1.data(), sc.u.data());
  for (size_t i = 0; i < d; i++) z_out[i] = sc.zraw[i] + sc.u[i];
}

struct Runner {
  const oracle_model* m;
  std::vector<Scratch> sc;
  std::vector<float> feat, out;
  explicit Runner(const oracle_model* mm) : m(mm) {
    const oracle_config& c = m->cfg;
    sc.resize(c.depth);
    for (size_t l = 0; l < c.depth; l++) {
      sc[l].resize(c);
      refresh_rates(m->blocks[l], c, sc[l]);
    }
    feat.assign(c.d_latent, 0);
    out.assign(c.d_latent, 0);
  }
  // --- src/pssa.rs:2312-2337 forward_inference_features (single loop) ----------
  void set_age_add(uint64_t a) {
    for (auto& x : sc) x.age_add = a;
  }
  void features(float* state, uint32_t id) {
    const oracle_config& c = m->cfg;
    const size_t d = c.d_latent, ds = c.d_latent * c.d_state;
    const float scale = 1.0f / sqrtf((float)c.depth);
    const size_t loops = g_loops;
    if (loops == 1) {
      block_forward(m->blocks[0], c, sc[0], state, m->embed + (size_t)id * d, feat.data());
      for (size_t l = 1; l < c.depth; l++) {
        block_forward(m->blocks[l], c, sc[l], state + l * ds, feat.data(), out.data());
        for (size_t i = 0; i < d; i++) feat[i] += scale * out[i];
      }
      return;
    }
    // --- src/pssa.rs:2338-2373: each block's passes add out / loops to the
    // features they read; every block after the first then returns
    // input + residual_scale * features.
    const float loop_scale = 1.0f / (float)loops;
    std::memcpy(feat.data(), m->embed + (size_t)id * d, d * 4);
    std::vector<float> inputs(d);
    for (size_t l = 0; l < c.depth; l++) {
      if (l > 0) inputs = feat;
      for (size_t k = 0; k < loops; k++) {
        block_forward(m->blocks[l], c, sc[l], state + (l * loops + k) * ds, feat.data(), out.data());
        for (size_t i = 0; i < d; i++) feat[i] += loop_scale * out[i];
      }
      if (l > 0)
        for (size_t i = 0; i < d; i++) feat[i] = inputs[i] + scale * feat[i];
    }
  }
  // --- src/pssa.rs:2379-2385 inference_logits ------------------------------------
  void logits(float* lg) {
    const oracle_config& c = m->cfg;
    const size_t d = c.d_latent;
    if (g_bf16_ops) {
      std::vector<float> fb(d);
      for (size_t i = 0; i < d; i++) fb[i] = bf16r(feat[i]);
      matvec(m->unembed, c.d_vocab, d, fb.data(), lg);
    } else {
      matvec(m->unembed, c.d_vocab, d, feat.data(), lg);
    }
    const float logit_scale = 1.0f / sqrtf((float)d);
    for (size_t v = 0; v < c.d_vocab; v++) lg[v] *= logit_scale;
  }
};

// bump_hybrid_ages (src/memory.rs:501-507) `times` times on every hybrid block.
static void bump_hybrid(const oracle_model* m, uint64_t times) {
  for (size_t l = 0; l < m->cfg.depth; l++) {
    const oracle_block& b = m->blocks[l];
    if (!b.mem_hybrid_enabled || !b.mem_hybrid_age) continue;
    for (size_t i = 0; i < b.mem_count; i++) b.mem_hybrid_age[i] = sat_add(b.mem_hybrid_age[i], times);
  }
}

template <class F>
void parallel_for(size_t n, int threads, F f) {
  if (threads <= 1 || n <= 1) {
    for (size_t i = 0; i < n; i++) f(i);
    return;
  }
  std::atomic<size_t> next(0);
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; t++)
    pool.emplace_back([&]() {
      for (;;) {
        size_t i = next.fetch_add(1);
        if (i >= n) break;
        f(i);
      }
    });
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

void oracle_set_dot_avx2(int enabled) { g_dot_avx2 = enabled ? 1 : 0; }
void oracle_set_bf16_operands(int enabled) { g_bf16_ops = enabled ? 1 : 0; }
void oracle_set_loops(size_t loops) { g_loops = loops < 1 ? 1 : loops; }
size_t oracle_get_loops(void) { return g_loops; }
float oracle_bf16_round(float x) { return bf16r(x); }
int oracle_get_bf16_operands(void) { return g_bf16_ops; }
int oracle_get_dot_avx2(void) { return g_dot_avx2; }

uint64_t oracle_rng_new(uint64_t seed) { return Rng(seed).state; }
uint32_t oracle_rng_next_u32(uint64_t* state) {
  Rng r(*state);
  r.state = *state;
  uint32_t v = r.next_u32();
  *state = r.state;
  return v;
}
float oracle_dot(const float* a, const float* b, size_t n) { return dot(a, b, n); }
float oracle_softplus(float x) { return softplus(x); }
float oracle_sigmoid(float x) { return sigmoid(x); }

// --- src/pssa.rs:86-101 random_xavier; 630-700 block constructor; 2019-2072 ---
static void xavier(Rng& rng, float* w, size_t rows, size_t cols) {
  float limit = sqrtf(6.0f / (float)(rows + cols));
  for (size_t i = 0; i < rows * cols; i++) w[i] = rng.gen_range(-limit, limit);
}

// HiPPO log-spaced timescales, src/pssa.rs:649-665.
// tau_max = 200 is the reference's range (src/pssa.rs:649-665); the baseline
// initialisation uses 13, so that the slowest mode's transition at the
// initial step size softplus(0) = ln 2 is exp(-ln 2 / 13) = 0.948 < 0.95.
static void hippo_rates(float* a_raw, size_t d, size_t s, float tau_max) {
  const float ln_min = logf(1.5f);
  const float ln_max = logf(tau_max);
  for (size_t i = 0; i < d; i++)
    for (size_t j = 0; j < s; j++) {
      float ratio = s > 1 ? (float)j / (float)(s - 1) : 0.0f;
      float tau = expf(ln_min + ratio * (ln_max - ln_min));
      float rate = 1.0f / tau;
      a_raw[i * s + j] = logf(expm1f(rate));
    }
}

static void reset_block_common(const oracle_block& b, const oracle_config& c, float tau_max) {
  const size_t d = c.d_latent, C = c.mem_capacity, k = c.d_mem_key;
  for (size_t i = 0; i < d; i++) {
    b.norm_gamma[i] = 1.0f;
    b.norm_beta[i] = 0.0f;
  }
  hippo_rates(b.a_raw, d, c.d_state, tau_max);
  std::fill(b.mem_keys, b.mem_keys + C * k, 0.0f);
  std::fill(b.mem_values, b.mem_values + C * d, 0.0f);
  std::fill(b.mem_norm_sq, b.mem_norm_sq + C, 0.0f);
  std::fill(b.mem_confidence, b.mem_confidence + C, 1.0f);
  std::fill(b.mem_last_seen, b.mem_last_seen + C, (uint64_t)0);
}

uint64_t oracle_init_reference(const oracle_model* m, uint64_t seed) {
  const oracle_config& c = m->cfg;
  const size_t v = c.d_vocab, d = c.d_latent, s = c.d_state, k = c.d_mem_key, r = c.adapter_rank;
  Rng rng(seed);
  auto block = [&](oracle_block& b) {
    reset_block_common(b, c, 200.0f);
    xavier(rng, b.w_delta, d, d);
    xavier(rng, b.w_b, s, d);
    xavier(rng, b.w_c, s, d);
    xavier(rng, b.w_qx, k, d);
    xavier(rng, b.w_qh, k, d);
    xavier(rng, b.w_gate, d, d);
    xavier(rng, b.w_proj, d, d);
    xavier(rng, b.adapter_down, r, d);  // src/adapter.rs:16-24
    std::fill(b.adapter_up, b.adapter_up + d * r, 0.0f);
    std::fill(b.adapter_slow, b.adapter_slow + d * r, 0.0f);
    xavier(rng, b.mlp_w1, 2 * d, d);
    std::fill(b.mlp_w2, b.mlp_w2 + d * 2 * d, 0.0f);
    b.mem_count = 0;
    b.mem_write_head = 0;
  };
  xavier(rng, m->embed, v, d);
  block(m->blocks[0]);
  xavier(rng, m->unembed, v, d);
  for (size_t l = 1; l < c.depth; l++) block(m->blocks[l]);
  return rng.state;
}

static void normal_fill(Rng& rng, float* w, size_t n, double std_dev) {
  for (size_t i = 0; i < n; i++) w[i] = (float)(std_dev * rng.normal());
}

uint64_t oracle_init_baseline(const oracle_model* m, uint64_t seed) {
  const oracle_config& c = m->cfg;
  const size_t v = c.d_vocab, d = c.d_latent, s = c.d_state, k = c.d_mem_key, r = c.adapter_rank;
  Rng rng(seed);
  const double sd = 0.02;
  auto block = [&](oracle_block& b) {
    reset_block_common(b, c, 13.0f);
    normal_fill(rng, b.w_delta, d * d, sd);
    normal_fill(rng, b.w_b, s * d, sd);
    normal_fill(rng, b.w_c, s * d, sd);
    normal_fill(rng, b.w_qx, k * d, sd);
    normal_fill(rng, b.w_qh, k * d, sd);
    normal_fill(rng, b.w_gate, d * d, sd);
    normal_fill(rng, b.w_proj, d * d, sd);
    normal_fill(rng, b.adapter_down, r * d, sd);
    normal_fill(rng, b.adapter_up, d * r, sd);
    normal_fill(rng, b.adapter_slow, d * r, sd);
    normal_fill(rng, b.mlp_w1, 2 * d * d, sd);
    normal_fill(rng, b.mlp_w2, d * 2 * d, sd);
    b.mem_count = 0;
    b.mem_write_head = 0;
  };
  normal_fill(rng, m->embed, v * d, sd);
  block(m->blocks[0]);
  normal_fill(rng, m->unembed, v * d, sd);
  for (size_t l = 1; l < c.depth; l++) block(m->blocks[l]);
  return rng.state;
}

static void ball_vector(Rng& rng, float* out, size_t n, float max_radius) {
  std::vector<float> dir(n);
  for (size_t i = 0; i < n; i++) dir[i] = (float)rng.normal();
  double norm = std::sqrt(squared_norm_f64(dir.data(), n));
  double rad = (double)rng.next_u32() / 4294967296.0 * (double)max_radius;
  for (size_t i = 0; i < n; i++) out[i] = norm > 0.0 ? (float)((double)dir[i] / norm * rad) : 0.0f;
}

// --- src/memory.rs:264-303 insert ------------------------------------------------
// --- src/memory.rs:150-170 clamp_value ------------------------------------------
// Iterator::sum over (x as f64)^2, left to right (src/memory.rs:190-192).
static double value_norm_sq(const float* v, size_t n) {
  double s = 0.0;
  for (size_t i = 0; i < n; i++) s += (double)v[i] * (double)v[i];
  return s;
}

int oracle_clamp_value(float* value, size_t n, float cap) {
  const double cap_sq = (double)cap * (double)cap;
  const double norm_sq = value_norm_sq(value, n);
  // assert!(norm_sq.is_finite(), "capped memory value must be finite")
  if (!std::isfinite(norm_sq)) return -1;
  if (norm_sq <= cap_sq) return 0;
  const double scale = (double)cap / std::sqrt(norm_sq);
  for (size_t i = 0; i < n; i++) value[i] = (float)((double)value[i] * scale);
  // One ulp toward zero per pass until the rounded vector fits.
  while (value_norm_sq(value, n) > cap_sq)
    for (size_t i = 0; i < n; i++)
      if (value[i] != 0.0f) {
        uint32_t u;
        std::memcpy(&u, &value[i], 4);
        u -= 1;
        std::memcpy(&value[i], &u, 4);
      }
  return 0;
}

int oracle_bank_set_value_cap(oracle_block* b, size_t capacity, size_t dv, float cap) {
  if (cap > 0.0f) {
    // The reference panics at the first non-finite slot; here nothing changes.
    for (size_t s = 0; s < capacity; s++)
      if (!std::isfinite(value_norm_sq(b->mem_values + s * dv, dv))) return -1;
    for (size_t s = 0; s < capacity; s++) oracle_clamp_value(b->mem_values + s * dv, dv, cap);
  }
  b->mem_value_cap = cap;
  return 0;
}

int64_t oracle_bank_insert(oracle_block* b, size_t capacity, size_t dk, size_t dv,
                           const float* key, const float* val) {
  float key_sq = squared_norm(key, dk);
  if (!(std::isfinite(key_sq) && key_sq < 1.0f)) return -1;
  if (b->mem_value_cap > 0.0f && !std::isfinite(value_norm_sq(val, dv))) return -2;  // clamp_value's assertion
  size_t idx;
  if (b->mem_count < capacity) {
    idx = b->mem_count;
    b->mem_count += 1;
  } else {
    idx = b->mem_write_head;
    b->mem_write_head = (b->mem_write_head + 1) % capacity;
  }
  std::memcpy(b->mem_keys + idx * dk, key, dk * 4);
  b->mem_norm_sq[idx] = key_sq;
  std::memcpy(b->mem_values + idx * dv, val, dv * 4);
  if (b->mem_value_cap > 0.0f) (void)oracle_clamp_value(b->mem_values + idx * dv, dv, b->mem_value_cap);
  b->mem_confidence[idx] = 1.0f;
  b->mem_last_seen[idx] = 0;
  if (b->mem_hybrid_gate) b->mem_hybrid_gate[idx] = 1.0f;  // src/memory.rs:300-301
  if (b->mem_hybrid_age) b->mem_hybrid_age[idx] = 0;
  return (int64_t)idx;
}

// --- src/memory.rs:305-342 insert_protected + src/defense.rs:45-67 -------------
int64_t oracle_bank_insert_protected(oracle_block* b, size_t capacity, size_t dk, size_t dv,
                                     const float* key, const float* val, float surprise,
                                     uint64_t step) {
  if (b->mem_count < capacity) {
    int64_t idx = oracle_bank_insert(b, capacity, dk, dv, key, val);
    if (idx >= 0) b->mem_last_seen[idx] = step;
    return idx;
  }
  size_t idx = b->mem_write_head;
  float* conf = &b->mem_confidence[idx];
  uint64_t last = b->mem_last_seen[idx];
  uint64_t delta_t = step > last ? step - last : 0;
  float gain = refractory_gain(delta_t, 60.0f);
  float damage = 0.08f * surprise * gain;
  if (*conf > damage) {
    *conf -= damage;
    b->mem_last_seen[idx] = step;
    return -1;
  }
  *conf = 1.0f;
  b->mem_last_seen[idx] = step;
  int64_t ins = oracle_bank_insert(b, capacity, dk, dv, key, val);
  if (ins >= 0) b->mem_last_seen[ins] = step;
  return ins;
}

// --- src/memory.rs:488-499 insert_gated ----------------------------------------
int64_t oracle_bank_insert_gated(oracle_block* b, size_t capacity, size_t dk, size_t dv,
                                 const float* key, const float* val, float gate) {
  if (!(std::isfinite(gate) && gate >= 0.0f)) return -1;
  int64_t idx = oracle_bank_insert(b, capacity, dk, dv, key, val);
  if (idx >= 0 && b->mem_hybrid_gate) b->mem_hybrid_gate[idx] = gate;
  return idx;
}

// --- src/memory.rs:520-556 insert_gated_protected ------------------------------
int64_t oracle_bank_insert_gated_protected(oracle_block* b, size_t capacity, size_t dk, size_t dv,
                                           const float* key, const float* val, float gate,
                                           float surprise, uint64_t step) {
  if (!(std::isfinite(gate) && gate >= 0.0f)) return -1;
  if (b->mem_count < capacity) {
    int64_t idx = oracle_bank_insert_gated(b, capacity, dk, dv, key, val, gate);
    if (idx >= 0) b->mem_last_seen[idx] = step;
    return idx;
  }
  size_t idx = b->mem_write_head;
  float* conf = &b->mem_confidence[idx];
  uint64_t last = b->mem_last_seen[idx];
  uint64_t delta_t = step > last ? step - last : 0;
  float gain = refractory_gain(delta_t, 60.0f);
  float damage = 0.08f * surprise * gain;
  if (*conf > damage) {
    *conf -= damage;
    b->mem_last_seen[idx] = step;
    return -1;
  }
  *conf = 1.0f;
  b->mem_last_seen[idx] = step;
  int64_t ins = oracle_bank_insert_gated(b, capacity, dk, dv, key, val, gate);
  if (ins >= 0) b->mem_last_seen[ins] = step;
  return ins;
}

// --- src/memory.rs:501-507 bump_hybrid_ages ------------------------------------
void oracle_bank_bump_hybrid_ages(oracle_block* b, uint64_t times) {
  if (!b->mem_hybrid_age) return;
  for (size_t i = 0; i < b->mem_count; i++) b->mem_hybrid_age[i] = sat_add(b->mem_hybrid_age[i], times);
}

void oracle_retrieve_hybrid_batch(const float* keys, const float* norm_sq, const float* values,
                                  size_t count, size_t capacity, size_t d_key, size_t d_val,
                                  const float* q_pnc, size_t n_q, float tau, size_t top_k,
                                  const float* gate, const uint64_t* age, float lam,
                                  float* out_val, float* out_min, uint32_t* out_idx,
                                  float* out_weights, int threads) {
  parallel_for(n_q, threads, [&](size_t q) {
    std::vector<float> w(capacity > 0 ? capacity : 1);
    float mn = retrieve_hybrid(keys, norm_sq, values, count, capacity, d_key, d_val,
                               q_pnc + q * d_key, tau, top_k, gate, age, 0, lam, out_val + q * d_val,
                               w.data(), out_idx ? out_idx + q * top_k : nullptr);
    if (out_min) out_min[q] = mn;
    if (out_weights) std::memcpy(out_weights + q * capacity, w.data(), capacity * 4);
  });
}

float oracle_refractory_gain(uint64_t delta_tokens, float tau) {
  return refractory_gain(delta_tokens, tau);
}

void oracle_populate_banks(const oracle_model* m, uint64_t seed, uint64_t count, float max_radius) {
  const oracle_config& c = m->cfg;
  const size_t d = c.d_latent, k = c.d_mem_key;
  Rng rng(seed);
  std::vector<float> key(k), val(d);
  for (size_t l = 0; l < c.depth; l++) {
    oracle_block* b = &m->blocks[l];
    for (uint64_t n = 0; n < count; n++) {
      ball_vector(rng, key.data(), k, max_radius);
      ball_vector(rng, val.data(), d, max_radius);
      oracle_bank_insert(b, c.mem_capacity, k, d, key.data(), val.data());
    }
  }
}

float oracle_squared_norm(const float* p, size_t n) { return squared_norm(p, n); }
float oracle_project(const float* q, float* out, size_t n) { return project(q, out, n); }
float oracle_poincare_distance(const float* u, float u_sq, const float* v, float v_sq, size_t n) {
  return poincare_distance(u, u_sq, v, v_sq, n);
}
double oracle_rust_asinh(double x) { return rust_asinh(x); }

float oracle_retrieve(const float* keys, const float* norm_sq, const float* values, size_t count,
                      size_t capacity, size_t d_key, size_t d_val, const float* q_pnc, float tau,
                      size_t top_k, float* out_val, float* out_weights) {
  return retrieve(keys, norm_sq, values, count, capacity, d_key, d_val, q_pnc, tau, top_k, out_val,
                  out_weights, nullptr);
}

void oracle_retrieve_batch(const float* keys, const float* norm_sq, const float* values,
                           size_t count, size_t capacity, size_t d_key, size_t d_val,
                           const float* q_pnc, size_t n_q, float tau, size_t top_k,
                           float* out_val, float* out_min, uint32_t* out_idx, int threads) {
  parallel_for(n_q, threads, [&](size_t q) {
    std::vector<float> w(capacity > 0 ? capacity : 1);
    float mn = retrieve(keys, norm_sq, values, count, capacity, d_key, d_val, q_pnc + q * d_key,
                        tau, top_k, out_val + q * d_val, w.data(),
                        out_idx ? out_idx + q * top_k : nullptr);
    if (out_min) out_min[q] = mn;
  });
}

// --- src/backend.rs:801-830 gemm_cpu_reference: Y = X W^T with dot_slice -------
void oracle_gemm_xwt(const float* x, const float* w, size_t m, size_t n, size_t k, float* y) {
  for (size_t i = 0; i < m; i++)
    for (size_t j = 0; j < n; j++) y[i * n + j] = dot(x + i * k, w + j * k, k);
}

// --- src/gpu_batch.rs:392-437 materialize + tests/backend_cuda.rs:126-140 twin --
void oracle_ssm_forward(const float* delta, const float* b_proj, const float* x_norm,
                        const float* rates, const float* c_proj, const float* initial,
                        size_t L, size_t dm, size_t ds, float* bar_a, float* bar_b,
                        float* states, float* y) {
  size_t stride = dm * ds;
  std::vector<float> h(initial, initial + stride);
  if (states) std::memcpy(states, initial, stride * 4);
  for (size_t t = 0; t < L; t++) {
    for (size_t i = 0; i < dm; i++) {
      float di = delta[t * dm + i];
      float yi = 0.0f;
      for (size_t j = 0; j < ds; j++) {
        size_t c = i * ds + j;
        float a = expf(di * rates[c]);
        float b = di * b_proj[t * ds + j];
        if (bar_a) bar_a[t * stride + c] = a;
        if (bar_b) bar_b[t * stride + c] = b;
        float hv = a * h[c] + b * x_norm[t * dm + i];
        h[c] = hv;
        if (states) states[(t + 1) * stride + c] = hv;
        yi += hv * c_proj[t * ds + j];
      }
      y[t * dm + i] = yi;
    }
  }
}

void oracle_forward_inference(const oracle_model* m, float* state, uint32_t id, float* logits) {
  Runner run(m);
  run.features(state, id);
  bump_hybrid(m, 1);
  if (logits) run.logits(logits);
}

void oracle_forward_features(const oracle_model* m, float* state, uint32_t id, float* features) {
  Runner run(m);
  run.features(state, id);
  bump_hybrid(m, 1);
  std::memcpy(features, run.feat.data(), m->cfg.d_latent * 4);
}

// --- src/pssa.rs:2393-2442 prefill_inference (tiles are bit-identical to the
// token loop, src/pssa.rs:1885-1906; head on the last token only) ------------
// Prefill of one lane without storing the hybrid ages (lanes advance
// together).  An invalid id stops it after the tokens before it
// (src/pssa.rs:2411-2418): *done is the count processed, logits untouched.
static int prefill_lane(const oracle_model* m, float* state, const uint32_t* ids, size_t n, float* logits,
                        size_t* done) {
  *done = 0;
  if (n == 0) return -1;
  Runner run(m);
  for (size_t t = 0; t < n; t++) {
    if (ids[t] >= m->cfg.d_vocab) return -2;
    run.set_age_add(t + 1);
    run.features(state, ids[t]);
    *done = t + 1;
  }
  if (logits) run.logits(logits);
  return 0;
}

int oracle_prefill(const oracle_model* m, float* state, const uint32_t* ids, size_t n, float* logits) {
  size_t done = 0;
  const int rc = prefill_lane(m, state, ids, n, logits, &done);
  bump_hybrid(m, done);
  return rc;
}

int oracle_prefill_lanes(const oracle_model* m, float* states, const uint32_t* ids, size_t lanes,
                         size_t n, float* logits, int threads) {
  const oracle_config& c = m->cfg;
  size_t per = c.depth * g_loops * c.d_latent * c.d_state;
  std::atomic<int> rc(0);
  std::vector<size_t> done(lanes, 0);
  parallel_for(lanes, threads, [&](size_t l) {
    int r = prefill_lane(m, states + l * per, ids + l * n, n, logits ? logits + l * c.d_vocab : nullptr, &done[l]);
    if (r) rc = r;
  });
  // The lanes' tokens t read ages + t + 1; the ages end the longest prefix higher.
  size_t most = 0;
  for (size_t d : done) most = d > most ? d : most;
  bump_hybrid(m, most);
  return rc.load();
}

// --- src/pssa.rs:2597-2752 forward_train_chunk (depth one, single loop) ---------
float oracle_train_chunk_forward(const oracle_model* m, float* state, const uint32_t* ids,
                                 const uint32_t* targets, size_t n, float* logits) {
  const oracle_config& c = m->cfg;
  const size_t v = c.d_vocab;
  Runner run(m);
  float total = 0.0f;
  std::vector<float> probs(v);
  for (size_t t = 0; t < n; t++) {
    run.set_age_add(t + 1);  // src/pssa.rs:1334-1345 bumps per token too
    run.features(state, ids[t]);
    float* lg = logits + t * v;
    run.logits(lg);
    float max_l = -INFINITY;
    for (size_t i = 0; i < v; i++)
      if (lg[i] > max_l) max_l = lg[i];
    float sum_exp = 0.0f;
    for (size_t i = 0; i < v; i++) {
      float e = expf(lg[i] - max_l);
      probs[i] = e;
      sum_exp += e;
    }
    float loss = (max_l - lg[targets[t]]) + logf(sum_exp);
    total += loss;
  }
  bump_hybrid(m, n);
  return total / (float)n;
}

// f32::total_cmp order key: larger key = larger in IEEE total order.
static int32_t total_order_key(float f) {
  int32_t b;
  std::memcpy(&b, &f, 4);
  return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

// sample() with temperature 0 (src/inference.rs:123-127): max_by over ids
// 1..V-1 of total_cmp, ties broken toward the lower id.
uint32_t oracle_greedy(const float* logits, size_t v) {
  uint32_t best = 1;
  for (uint32_t i = 2; i < v; i++)
    if (total_order_key(logits[i]) > total_order_key(logits[best])) best = i;
  return best;
}

// --- src/inference.rs:104-127 sample() at temperature 0 -------------------------
int64_t oracle_sample_greedy(float* logits, size_t v, const uint32_t* hist, size_t n_hist, float penalty) {
  for (size_t i = 0; i < v; i++)
    if (!std::isfinite(logits[i])) return -1;
  if (penalty > 1.0f) {
    // Each of the last 64 ids, once per occurrence, in history order.
    for (size_t j = n_hist > 64 ? n_hist - 64 : 0; j < n_hist; j++) {
      float& l = logits[hist[j]];
      if (l > 0.0f)
        l /= penalty;
      else
        l *= penalty;
    }
  }
  return (int64_t)oracle_greedy(logits, v);
}

// --- src/inference.rs:102-178 sample() at any temperature -----------------------
// The repetition penalty over the last 64 ids, then greedy at temperature 0;
// otherwise probs over ids 1..V-1 (the maximum over 1..V-1 subtracted before
// dividing by the temperature, f32 exp, a sequential f32 sum), candidates in
// (probability descending, id ascending) order, the first top_k of them cut
// where the running f32 sum first reaches top_p, and one draw of
// gen_range_f32(0, mass) from the caller's generator matched against the
// running sum.  Returns the id, -1 for non-finite logits, -2 for an invalid
// probability mass, -3 without candidates.
int64_t oracle_sample(float* logits, size_t v, const uint32_t* hist, size_t n_hist, float penalty,
                      float temperature, float top_p, size_t top_k, uint64_t* rng_state) {
  if (temperature == 0.0f) return oracle_sample_greedy(logits, v, hist, n_hist, penalty);
  for (size_t i = 0; i < v; i++)
    if (!std::isfinite(logits[i])) return -1;
  if (penalty > 1.0f) {
    for (size_t j = n_hist > 64 ? n_hist - 64 : 0; j < n_hist; j++) {
      float& l = logits[hist[j]];
      if (l > 0.0f)
        l /= penalty;
      else
        l *= penalty;
    }
  }
  float mx = -INFINITY;
  for (size_t i = 1; i < v; i++) mx = std::max(mx, logits[i]);
  std::vector<float> probs(v, 0.0f);
  float sum = 0.0f;
  for (size_t i = 1; i < v; i++) {
    probs[i] = std::exp((logits[i] - mx) / temperature);
    sum += probs[i];
  }
  if (!std::isfinite(sum) || sum <= 0.0f) return -2;
  std::vector<std::pair<uint32_t, float>> cand;
  for (size_t i = 1; i < v; i++)
    if (std::isfinite(probs[i])) cand.emplace_back((uint32_t)i, probs[i] / sum);
  if (cand.empty()) return -3;
  // total_cmp on non-negative finite probabilities is the numeric order.
  std::sort(cand.begin(), cand.end(), [](const std::pair<uint32_t, float>& a, const std::pair<uint32_t, float>& b) {
    return a.second != b.second ? a.second > b.second : a.first < b.first;
  });
  const size_t k = std::min(cand.size(), top_k);
  size_t cutoff = k;
  float cumulative = 0.0f;
  for (size_t i = 0; i < k; i++) {
    cumulative += cand[i].second;
    if (cumulative >= top_p) {
      cutoff = i + 1;
      break;
    }
  }
  const size_t nf = std::max<size_t>(cutoff, 1);
  float mass = 0.0f;
  for (size_t i = 0; i < nf; i++) mass += cand[i].second;
  Rng rng(1);
  rng.state = *rng_state;
  const float draw = rng.gen_range(0.0f, mass);
  *rng_state = rng.state;
  float running = 0.0f;
  uint32_t id = cand[nf - 1].first;
  for (size_t i = 0; i < nf; i++) {
    running += cand[i].second;
    if (draw <= running) {
      id = cand[i].first;
      break;
    }
  }
  return (int64_t)id;
}

void oracle_dense_scan(const float* a, const float* b, const float* h0, size_t batch, size_t L,
                       size_t s, float* h, int threads) {
  parallel_for(batch, threads, [&](size_t bi) {
    std::vector<float> cur(h0 + bi * s, h0 + (bi + 1) * s), nxt(s);
    for (size_t t = 0; t < L; t++) {
      const float* A = a + ((bi * L + t) * s) * s;
      const float* bt = b + (bi * L + t) * s;
      for (size_t r = 0; r < s; r++) {
        double acc = 0.0;
        for (size_t q = 0; q < s; q++) acc += (double)A[r * s + q] * (double)cur[q];
        nxt[r] = (float)(acc + (double)bt[r]);
      }
      std::memcpy(h + (bi * L + t) * s, nxt.data(), s * 4);
      std::swap(cur, nxt);
    }
  });
}

// --- src/pssa.rs:1814-1832 dream_replay_value fast-weight rule ---------------
void oracle_hebbian_update(float* up, const float* target, const float* current, const float* act,
                           size_t d, size_t r) {
  double tn = std::sqrt(squared_norm_f64(target, d));
  float rate = 0.02f / (1.0f + (float)std::min(tn, (double)FLT_MAX));
  for (size_t i = 0; i < d; i++) {
    float err = std::min(std::max(target[i] - current[i], -4.0f), 4.0f);
    for (size_t q = 0; q < r; q++) up[i * r + q] += rate * err * act[q];
  }
}

// forward_inference (src/pssa.rs:2387-2391) that also returns, per block,
// the projected query, the block output z_final, the adapter output and the
// adapter activations: the operands of the plastic decode rules.
void oracle_forward_taps(const oracle_model* m, float* state, uint32_t id, float* q_pnc,
                         float* z_final, float* ad_out, float* act, float* logits) {
  const oracle_config& c = m->cfg;
  const size_t d = c.d_latent, ds = c.d_latent * c.d_state, k = c.d_mem_key, r = c.adapter_rank;
  Runner run(m);
  const float scale = 1.0f / sqrtf((float)c.depth);
  for (size_t l = 0; l < c.depth; l++) {
    float* z = l == 0 ? run.feat.data() : run.out.data();
    const float* in = l == 0 ? m->embed + (size_t)id * d : run.feat.data();
    block_forward(m->blocks[l], c, run.sc[l], state + l * ds, in, z);
    std::memcpy(q_pnc + l * k, run.sc[l].qp.data(), k * 4);
    std::memcpy(z_final + l * d, z, d * 4);
    std::memcpy(ad_out + l * d, run.sc[l].adout.data(), d * 4);
    std::memcpy(act + l * r, run.sc[l].act.data(), r * 4);
    if (l > 0)
      for (size_t i = 0; i < d; i++) run.feat[i] += scale * run.out[i];
  }
  bump_hybrid(m, 1);
  if (logits) run.logits(logits);
}

// Greedy decode over `lanes` independent streams sharing one model
// (forward_inference per stream, src/pssa.rs:2387-2391; greedy sample,
// src/inference.rs:123-127).  With `plastic` set, every step then applies,
// block by block and in lane order, (a) the refractory-protected bank write of
// the stream's projected query and block output when its surprise
// -log softmax(logits)[chosen] exceeds 3.5 (insert_protected,
// src/memory.rs:305-342; the write rule of insert_training_memory_at,
// src/pssa.rs:3705-3736), and (b) the Hebbian fast-weight rule of
// dream_replay_value (src/pssa.rs:1814-1832) with the block output as the
// target and the adapter output as the prediction.  The step counter that the
// refractory gate reads advances by one per step; step k uses step_base + k.
int oracle_decode(oracle_model* m, float* states, uint32_t* ids, size_t lanes, size_t steps,
                  int plastic, uint64_t step_base, uint32_t* out_ids, float* logits_last,
                  float* surprise_last, int threads) {
  if (g_loops != 1) return -9;  // the composed decode step is single-loop
  const oracle_config& c = m->cfg;
  const size_t d = c.d_latent, ds = c.d_latent * c.d_state, V = c.d_vocab, k = c.d_mem_key,
               r = c.adapter_rank, depth = c.depth;
  for (size_t i = 0; i < lanes; i++)
    if (ids[i] >= V) return -1;
  std::vector<float> lg(lanes * V), surprise(lanes);
  std::vector<float> tq(lanes * depth * k), tz(lanes * depth * d), ta(lanes * depth * d),
      tact(lanes * depth * r), tgate(lanes * depth);
  // The rate cache does not change during decode (only banks and the fast
  // adapter do), so each stream keeps one runner.
  std::vector<std::unique_ptr<Runner>> runners(lanes);
  parallel_for(lanes, threads, [&](size_t ln) { runners[ln].reset(new Runner(m)); });
  for (size_t step = 0; step < steps; step++) {
    parallel_for(lanes, threads, [&](size_t ln) {
      Runner& run = *runners[ln];
      float* st = states + ln * depth * ds;
      const float scale = 1.0f / sqrtf((float)depth);
      for (size_t l = 0; l < depth; l++) {
        float* z = l == 0 ? run.feat.data() : run.out.data();
        const float* in = l == 0 ? m->embed + (size_t)ids[ln] * d : run.feat.data();
        block_forward(m->blocks[l], c, run.sc[l], st + l * ds, in, z);
        std::memcpy(&tq[(ln * depth + l) * k], run.sc[l].qp.data(), k * 4);
        std::memcpy(&tz[(ln * depth + l) * d], z, d * 4);
        std::memcpy(&ta[(ln * depth + l) * d], run.sc[l].adout.data(), d * 4);
        std::memcpy(&tact[(ln * depth + l) * r], run.sc[l].act.data(), r * 4);
        // Hybrid write gate: mean memory-injection gate (src/pssa.rs:3719-3726).
        float gs = 0.0f;
        for (size_t i = 0; i < d; i++) gs += run.sc[l].g[i];
        tgate[ln * depth + l] = gs / (float)d;
        if (l > 0)
          for (size_t i = 0; i < d; i++) run.feat[i] += scale * run.out[i];
      }
      float* lgl = &lg[ln * V];
      run.logits(lgl);
      const uint32_t next = oracle_greedy(lgl, V);
      float mx = -INFINITY;
      for (size_t v = 0; v < V; v++) mx = std::fmax(mx, lgl[v]);
      float sum = 0.0f;
      for (size_t v = 0; v < V; v++) sum += expf(lgl[v] - mx);
      surprise[ln] = (mx + logf(sum)) - lgl[next];
      out_ids[step * lanes + ln] = next;
    });
    bump_hybrid(m, 1);  // the lanes' reads of this step saw one more bump
    if (plastic) {
      const uint64_t cur = step_base + step + 1;
      for (size_t l = 0; l < depth; l++) {
        oracle_block* b = &m->blocks[l];
        for (size_t ln = 0; ln < lanes; ln++)
          if (surprise[ln] > 3.5f) {
            if (b->mem_hybrid_enabled)
              oracle_bank_insert_gated_protected(b, c.mem_capacity, k, d, &tq[(ln * depth + l) * k],
                                                 &tz[(ln * depth + l) * d], tgate[ln * depth + l],
                                                 surprise[ln], cur);
            else
              oracle_bank_insert_protected(b, c.mem_capacity, k, d, &tq[(ln * depth + l) * k],
                                           &tz[(ln * depth + l) * d], surprise[ln], cur);
          }
        for (size_t ln = 0; ln < lanes; ln++)
          oracle_hebbian_update(b->adapter_up, &tz[(ln * depth + l) * d], &ta[(ln * depth + l) * d],
                                &tact[(ln * depth + l) * r], d, r);
      }
    }
    for (size_t ln = 0; ln < lanes; ln++) ids[ln] = out_ids[step * lanes + ln];
  }
  if (logits_last) std::memcpy(logits_last, lg.data(), lanes * V * 4);
  if (surprise_last) std::memcpy(surprise_last, surprise.data(), lanes * 4);
  return 0;
}

}  // extern "C"

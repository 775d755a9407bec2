// Host-side weight construction for the HIP path: the reference's model
// initialisation and the bank population used by the benchmarks.
//
// Built with -ffp-contract=off: the reference (Rust) evaluates a*b+c as two
// rounded operations, and the initial weights must be bit-identical to
// PSSALayerV2::new for the same seed.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/pssa_hip.h"

namespace {

// xorshift64* generator, src/linalg.rs:1-28 (seed 0 remapped as in SimpleRng::new).
class XorShift64Star {
 public:
  explicit XorShift64Star(uint64_t seed) : s_(seed ? seed : 0x853c49e6748fea9bULL) {}
  uint32_t u32() {
    s_ ^= s_ >> 12;
    s_ ^= s_ << 25;
    s_ ^= s_ >> 27;
    return (uint32_t)((s_ * 0x2545F4914F6CDD1DULL) >> 32);
  }
  // SimpleRng::gen_range_f32.
  float uniform(float lo, float hi) {
    const float t = (float)u32() / (float)UINT32_MAX;
    return lo + t * (hi - lo);
  }
  // Box-Muller standard normal (baseline initialisation).
  double gauss() {
    const double u1 = ((double)u32() + 1.0) / 4294967296.0;
    const double u2 = (double)u32() / 4294967296.0;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
  uint64_t state() const { return s_; }

 private:
  uint64_t s_;
};

void fill_xavier(XorShift64Star& g, float* w, size_t rows, size_t cols) {
  const float lim = sqrtf(6.0f / (float)(rows + cols));  // src/pssa.rs:86-101
  const size_t n = rows * cols;
  for (size_t i = 0; i < n; ++i) w[i] = g.uniform(-lim, lim);
}

void fill_gauss(XorShift64Star& g, float* w, size_t n, double sd) {
  for (size_t i = 0; i < n; ++i) w[i] = (float)(sd * g.gauss());
}

// Log-spaced decay timescales tau in [1.5, tau_max] stored as raw rates
// ln(expm1(1/tau)) so that -softplus(raw) = -1/tau (src/pssa.rs:649-665,
// where tau_max = 200).  The baseline initialisation takes tau_max = 13: its
// slowest mode's transition at the initial step size softplus(0) = ln 2 is
// exp(-ln 2 / 13) = 0.948, a spectral radius below 0.95.
constexpr float kTauMaxReference = 200.0f, kTauMaxBaseline = 13.0f;
void fill_hippo(float* a_raw, size_t d, size_t s, float tau_max) {
  const float lo = logf(1.5f), hi = logf(tau_max);
  for (size_t j = 0; j < s; ++j) {
    const float frac = s > 1 ? (float)j / (float)(s - 1) : 0.0f;
    const float raw = logf(expm1f(1.0f / expf(lo + frac * (hi - lo))));
    for (size_t i = 0; i < d; ++i) a_raw[i * s + j] = raw;
  }
}

double norm2_f64(const float* p, size_t n) {
  double acc = 0.0;
  for (size_t i = 0; i < n; ++i) acc += (double)p[i] * (double)p[i];
  return acc;
}

// HyperbolicEpisodicBankV2::squared_norm (src/memory.rs:181-192).
float bank_norm_sq(const float* p, size_t n) {
  const double v = norm2_f64(p, n);
  if (v < 1.0 && (float)v == 1.0f) return std::nextafter(1.0f, 0.0f);
  return (float)v;
}

void set_err(char* err, size_t n, const std::string& m) {
  if (err && n) std::snprintf(err, n, "%s", m.c_str());
}

bool check_weights(const pssa_hip_weights* w, char* err, size_t n) {
  if (!w || !w->blocks || !w->embed || !w->unembed) {
    set_err(err, n, "weights: null pointer");
    return false;
  }
  const pssa_hip_config& c = w->cfg;
  if (c.depth < 1 || c.depth > 32 || !c.d_vocab || !c.d_latent || !c.d_state || !c.d_mem_key ||
      !c.mem_capacity || !c.adapter_rank) {
    set_err(err, n, "weights: dimensions must be positive and depth in 1..=32");
    return false;
  }
  for (uint64_t l = 0; l < c.depth; ++l) {
    const pssa_hip_block& b = w->blocks[l];
    const void* ptrs[] = {b.norm_gamma, b.norm_beta,  b.a_raw,        b.w_delta,   b.w_b,
                          b.w_c,        b.w_qx,       b.w_qh,         b.w_gate,    b.w_proj,
                          b.adapter_down, b.adapter_up, b.adapter_slow, b.mlp_w1,  b.mlp_w2,
                          b.mem_keys,   b.mem_values, b.mem_norm_sq,  b.mem_confidence,
                          b.mem_last_seen};
    for (const void* p : ptrs)
      if (!p) {
        set_err(err, n, "weights: null block tensor");
        return false;
      }
  }
  return true;
}

void clear_block(const pssa_hip_config& c, pssa_hip_block& b, float tau_max) {
  const size_t d = c.d_latent, s = c.d_state, k = c.d_mem_key, C = c.mem_capacity;
  std::fill(b.norm_gamma, b.norm_gamma + d, 1.0f);
  std::fill(b.norm_beta, b.norm_beta + d, 0.0f);
  fill_hippo(b.a_raw, d, s, tau_max);
  std::fill(b.mem_keys, b.mem_keys + C * k, 0.0f);
  std::fill(b.mem_values, b.mem_values + C * d, 0.0f);
  std::fill(b.mem_norm_sq, b.mem_norm_sq + C, 0.0f);
  std::fill(b.mem_confidence, b.mem_confidence + C, 1.0f);
  std::fill(b.mem_last_seen, b.mem_last_seen + C, (uint64_t)0);
  b.mem_count = 0;
  b.mem_write_head = 0;
}

}  // namespace

extern "C" int pssa_hip_weights_init(const pssa_hip_weights* w, uint64_t seed, int mode,
                                     uint64_t* rng_state, char* err, size_t err_len) {
  if (!check_weights(w, err, err_len)) return PSSA_HIP_EINVAL;
  if (mode != PSSA_HIP_INIT_REFERENCE && mode != PSSA_HIP_INIT_BASELINE) {
    set_err(err, err_len, "weights_init: unknown mode");
    return PSSA_HIP_EINVAL;
  }
  const pssa_hip_config& c = w->cfg;
  const size_t V = c.d_vocab, d = c.d_latent, s = c.d_state, k = c.d_mem_key, r = c.adapter_rank;
  XorShift64Star g(seed);
  const bool ref = mode == PSSA_HIP_INIT_REFERENCE;
  auto mat = [&](float* p, size_t rows, size_t cols) {
    if (ref)
      fill_xavier(g, p, rows, cols);
    else
      fill_gauss(g, p, rows * cols, 0.02);
  };
  // Draw order of PSSAContinuousBlockV2::new_with_rng_and_loops
  // (src/pssa.rs:630-700) and PlasticAdapterV2::new (src/adapter.rs:16-24).
  auto block = [&](pssa_hip_block& b) {
    clear_block(c, b, ref ? kTauMaxReference : kTauMaxBaseline);
    mat(b.w_delta, d, d);
    mat(b.w_b, s, d);
    mat(b.w_c, s, d);
    mat(b.w_qx, k, d);
    mat(b.w_qh, k, d);
    mat(b.w_gate, d, d);
    mat(b.w_proj, d, d);
    mat(b.adapter_down, r, d);
    if (ref) {
      std::fill(b.adapter_up, b.adapter_up + d * r, 0.0f);
      std::fill(b.adapter_slow, b.adapter_slow + d * r, 0.0f);
    } else {
      fill_gauss(g, b.adapter_up, d * r, 0.02);
      fill_gauss(g, b.adapter_slow, d * r, 0.02);
    }
    mat(b.mlp_w1, 2 * d, d);
    if (ref)
      std::fill(b.mlp_w2, b.mlp_w2 + d * 2 * d, 0.0f);
    else
      fill_gauss(g, b.mlp_w2, d * 2 * d, 0.02);
  };
  // PSSALayerV2::new_with_device_and_loops (src/pssa.rs:2036-2050): embedding,
  // first block, unembedding, then the extra blocks.
  mat(w->embed, V, d);
  block(w->blocks[0]);
  mat(w->unembed, V, d);
  for (uint64_t l = 1; l < c.depth; ++l) block(w->blocks[l]);
  if (rng_state) *rng_state = g.state();
  return PSSA_HIP_OK;
}

extern "C" int pssa_hip_weights_populate_banks(const pssa_hip_weights* w, uint64_t seed,
                                               uint64_t count, float max_radius, char* err,
                                               size_t err_len) {
  if (!check_weights(w, err, err_len)) return PSSA_HIP_EINVAL;
  if (!(max_radius >= 0.0f && max_radius < 1.0f)) {
    set_err(err, err_len, "populate_banks: radius must be in [0, 1)");
    return PSSA_HIP_EINVAL;
  }
  const pssa_hip_config& c = w->cfg;
  const size_t d = c.d_latent, k = c.d_mem_key, C = c.mem_capacity;
  XorShift64Star g(seed);
  std::vector<float> key(k), val(d);
  auto ball = [&](float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)g.gauss();
    const double len = std::sqrt(norm2_f64(out, n));
    const double rad = (double)g.u32() / 4294967296.0 * (double)max_radius;
    for (size_t i = 0; i < n; ++i) out[i] = len > 0.0 ? (float)((double)out[i] / len * rad) : 0.0f;
  };
  for (uint64_t l = 0; l < c.depth; ++l) {
    pssa_hip_block& b = w->blocks[l];
    for (uint64_t m = 0; m < count; ++m) {
      ball(key.data(), k);
      ball(val.data(), d);
      // HyperbolicEpisodicBankV2::insert (src/memory.rs:264-303).
      const float key_sq = bank_norm_sq(key.data(), k);
      size_t slot;
      if (b.mem_count < C) {
        slot = b.mem_count++;
      } else {
        slot = b.mem_write_head;
        b.mem_write_head = (b.mem_write_head + 1) % C;
      }
      std::memcpy(b.mem_keys + slot * k, key.data(), k * sizeof(float));
      b.mem_norm_sq[slot] = key_sq;
      std::memcpy(b.mem_values + slot * d, val.data(), d * sizeof(float));
      b.mem_confidence[slot] = 1.0f;
      b.mem_last_seen[slot] = 0;
      if (b.mem_hybrid_gate) b.mem_hybrid_gate[slot] = 1.0f;  // src/memory.rs:300-301
      if (b.mem_hybrid_age) b.mem_hybrid_age[slot] = 0;
    }
  }
  return PSSA_HIP_OK;
}

// clamp_value (src/memory.rs:150-170): the reference's left-to-right f64
// squared norm, f64 scale with f32 rounding, then one ulp toward zero per
// pass until the rounded value fits.
static double value_norm_sq(const float* v, size_t n) {
  double s = 0.0;
  for (size_t i = 0; i < n; i++) s += (double)v[i] * (double)v[i];
  return s;
}

// The caller has checked that the squared norm is finite (the reference
// asserts it, src/memory.rs:151-152).
static void clamp_value(float* v, size_t n, float cap) {
  const double cap_sq = (double)cap * (double)cap;
  const double nsq = value_norm_sq(v, n);
  if (!(nsq > cap_sq)) return;
  const double scale = (double)cap / std::sqrt(nsq);
  for (size_t i = 0; i < n; i++) v[i] = (float)((double)v[i] * scale);
  for (int pass = 0; pass < 1024 && value_norm_sq(v, n) > cap_sq; ++pass)
    for (size_t i = 0; i < n; i++)
      if (v[i] != 0.0f) {
        uint32_t u;
        std::memcpy(&u, &v[i], 4);
        u -= 1;
        std::memcpy(&v[i], &u, 4);
      }
}

extern "C" int pssa_hip_weights_set_value_cap(const pssa_hip_weights* w, float cap, char* err, size_t err_len) {
  if (!check_weights(w, err, err_len)) return PSSA_HIP_EINVAL;
  if (!(std::isfinite(cap) && cap >= 0.0f)) {
    set_err(err, err_len, "memory value cap must be positive and finite");
    return PSSA_HIP_EINVAL;
  }
  const pssa_hip_config& c = w->cfg;
  // Every capacity slot is clamped, so every one must have a finite norm;
  // checked for all blocks before any value changes.
  if (cap > 0.0f)
    for (size_t l = 0; l < c.depth; l++)
      for (size_t s = 0; s < c.mem_capacity; s++)
        if (!std::isfinite(value_norm_sq(w->blocks[l].mem_values + s * c.d_latent, c.d_latent))) {
          set_err(err, err_len, "capped memory value must be finite");
          return PSSA_HIP_EINVAL;
        }
  for (size_t l = 0; l < c.depth; l++) {
    pssa_hip_block& b = w->blocks[l];
    if (cap > 0.0f)
      for (size_t s = 0; s < c.mem_capacity; s++) clamp_value(b.mem_values + s * c.d_latent, c.d_latent, cap);
    b.mem_value_cap = cap;
  }
  return PSSA_HIP_OK;
}

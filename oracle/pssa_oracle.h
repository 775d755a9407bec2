/*
 * CPU oracle for the PSSA inference forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (pssa_amd/, include/)
 * links, loads or calls this code.  It is a plain C++ restatement of the
 * reference's scalar CPU path (Sparticle62ops/pssa, Rust) and is used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker and CPU baseline.
 *
 * Every function cites the reference file:line it restates.  Evaluation
 * order follows the reference exactly (Rust does not contract a*b+c into an
 * FMA, so this file is compiled with -ffp-contract=off), which makes the
 * small-shape results bit-identical to the reference's golden fixtures
 * (tests/fixtures/depth_one_*_observed.bin, words 0..22).
 *
 * Parity status per function (details in the tests that pin them):
 *   rng / xavier / hippo init ........ pinned: INITIAL fixture bytes
 *   dot (portable, avx2) ............. pinned: observed words 0..22 (both files)
 *   block forward (norm, ssm, query,
 *     projection, soft read, gate,
 *     adapter, mlp), logits, loss .... pinned: observed words 0..22
 *   top-k read ........................ pinned: reference closed-form tests
 *                                        (memory_expansion.rs:53-93) + brute sort
 *   depth>1 residual .................. pinned: closed form (depth-2 model whose
 *                                        second block is zeroed reduces to depth 1)
 *   dense scan ........................ pinned: closed form (orthogonal-scaled
 *                                        transitions, diagonal case == diagonal scan)
 *   refractory gate ................... pinned: closed form (feature_benchmark.rs:446-500)
 *   greedy sample ..................... pinned: total_cmp order and tie rule, closed
 *                                        cases (src/inference.rs:123-127)
 *   hybrid read ....................... pinned: reference tests (memory.rs:893-1010:
 *                                        neutral == soft bitwise, recency rebinding,
 *                                        gate-zero dropout, fully gated fallback,
 *                                        metadata reset on overwrite)
 *   decode composition (oracle_decode)  parity unpinned as a whole: it composes the
 *                                        pinned forward, greedy, insert_protected and
 *                                        Hebbian rules; the reference has no such step
 */
#ifndef PSSA_ORACLE_H
#define PSSA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same layout as pssa_hip_config / pssa_hip_block / pssa_hip_model in
 * include/pssa_hip.h (declared separately so the oracle never includes
 * product headers). */
typedef struct {
  uint64_t depth;
  uint64_t d_vocab;
  uint64_t d_latent;
  uint64_t d_state;
  uint64_t d_mem_key;
  uint64_t mem_capacity;
  uint64_t adapter_rank;
  float tau_mem;
  uint32_t _pad;
} oracle_config;

typedef struct {
  float* norm_gamma;     /* [d] */
  float* norm_beta;      /* [d] */
  float* a_raw;          /* [d*s] */
  float* w_delta;        /* [d,d] */
  float* w_b;            /* [s,d] */
  float* w_c;            /* [s,d] */
  float* w_qx;           /* [k,d] */
  float* w_qh;           /* [k,d] */
  float* w_gate;         /* [d,d] */
  float* w_proj;         /* [d,d] */
  float* adapter_down;   /* [r,d] */
  float* adapter_up;     /* [d,r] */
  float* adapter_slow;   /* [d,r] */
  float* mlp_w1;         /* [2d,d] */
  float* mlp_w2;         /* [d,2d] */
  float* mem_keys;       /* [C,k] */
  float* mem_values;     /* [C,d] */
  float* mem_norm_sq;    /* [C] */
  float* mem_confidence; /* [C] */
  uint64_t* mem_last_seen; /* [C] */
  uint64_t mem_count;
  uint64_t mem_write_head;
  float* mem_hybrid_gate;    /* [C] or NULL (reads as 1.0) */
  uint64_t* mem_hybrid_age;  /* [C] or NULL (reads as 0) */
  uint32_t mem_hybrid_enabled;
  float mem_hybrid_lam;
  uint64_t mem_top_k; /* memory.top_k, 0 = full read (src/memory.rs:102-108) */
  float mem_value_cap; /* memory.value_cap (src/memory.rs:13-14): > 0 caps written values, 0 = none */
  uint32_t _pad;
} oracle_block;

typedef struct {
  oracle_config cfg;
  float* embed;   /* [V,d] */
  float* unembed; /* [V,d] */
  oracle_block* blocks; /* [depth] */
} oracle_model;

/* Reduction tree used by dot_slice: 1 = AVX2/FMA tree, 0 = portable tree. */
void oracle_set_dot_avx2(int enabled);
/* The bf16 mode of the device path (not a reference mode): every product's
 * activation operand rounded to bf16 (nearest even) where the device rounds
 * it, fp32 accumulation, the fp32 state path unchanged.  The caller rounds
 * the weights.  Process-wide; 0 (the default) is the reference arithmetic. */
void oracle_set_bf16_operands(int enabled);
int oracle_get_bf16_operands(void);
/* The rounding of that mode: nearest bf16, ties to even, as f32. */
float oracle_bf16_round(float x);
int oracle_get_dot_avx2(void);

/* linalg primitives */
/* Recurrent depth loops for the forward paths (1: the original model); a
 * lane's state is then [depth, loops, d_latent * d_state]. */
void oracle_set_loops(size_t loops);
size_t oracle_get_loops(void);
uint64_t oracle_rng_new(uint64_t seed);
uint32_t oracle_rng_next_u32(uint64_t* state);
float oracle_dot(const float* a, const float* b, size_t n);
float oracle_softplus(float x);
float oracle_sigmoid(float x);

/* Fill every tensor of the model with the reference initialisation
 * (SimpleRng draw order of PSSALayerV2::new).  Returns the final RNG state. */
uint64_t oracle_init_reference(const oracle_model* m, uint64_t seed);
/* Fill with the seeded N(0, 0.02) "baseline" initialisation. */
uint64_t oracle_init_baseline(const oracle_model* m, uint64_t seed);
/* Fill every block's bank with `count` slots: keys/values uniform in
 * direction with radius U[0, max_radius), inserted through insert(). */
void oracle_populate_banks(const oracle_model* m, uint64_t seed, uint64_t count, float max_radius);

/* Bank primitives (src/memory.rs). */
float oracle_squared_norm(const float* p, size_t n);
float oracle_project(const float* q, float* out, size_t n);
float oracle_poincare_distance(const float* u, float u_sq, const float* v, float v_sq, size_t n);
double oracle_rust_asinh(double x);
/* retrieve_soft_into for one query; top_k == 0 means full soft read.
 * Returns min distance.  weights has `capacity` entries. */
float oracle_retrieve(const float* keys, const float* norm_sq, const float* values,
                      size_t count, size_t capacity, size_t d_key, size_t d_val,
                      const float* q_pnc, float tau, size_t top_k,
                      float* out_val, float* out_weights);
/* Batched retrieval over many queries on `threads` threads. out_idx may be
 * NULL; when given it holds the top_k selected slot indices per query in
 * ascending slot order. */
void oracle_retrieve_batch(const float* keys, const float* norm_sq, const float* values,
                           size_t count, size_t capacity, size_t d_key, size_t d_val,
                           const float* q_pnc, size_t n_q, float tau, size_t top_k,
                           float* out_val, float* out_min, uint32_t* out_idx, int threads);
/* insert / insert_protected (src/memory.rs:264-342).  Returns slot or -1. */
int64_t oracle_bank_insert(oracle_block* b, size_t capacity, size_t d_key, size_t d_val,
                           const float* key, const float* val);
int64_t oracle_bank_insert_protected(oracle_block* b, size_t capacity, size_t d_key,
                                     size_t d_val, const float* key, const float* val,
                                     float surprise, uint64_t step);
float oracle_refractory_gain(uint64_t delta_tokens, float tau);
/* Hybrid read state (src/memory.rs:488-556): insert_gated,
 * insert_gated_protected, bump_hybrid_ages. */
int64_t oracle_bank_insert_gated(oracle_block* b, size_t capacity, size_t d_key, size_t d_val,
                                 const float* key, const float* val, float gate);
int64_t oracle_bank_insert_gated_protected(oracle_block* b, size_t capacity, size_t d_key,
                                           size_t d_val, const float* key, const float* val,
                                           float gate, float surprise, uint64_t step);
void oracle_bank_bump_hybrid_ages(oracle_block* b, uint64_t times);
/* set_value_cap (src/memory.rs:121-134): cap > 0 clamps every capacity slot's
 * value to Euclidean norm <= cap and caps later writes; 0 disables it and
 * keeps the values.  clamp_value's rule (src/memory.rs:150-170).  Where the
 * reference asserts a finite squared norm (src/memory.rs:151-152) these
 * return -1 and change nothing; an insert into a capped bank returns -2 for
 * such a value. */
int oracle_bank_set_value_cap(oracle_block* b, size_t capacity, size_t d_val, float cap);
int oracle_clamp_value(float* value, size_t n, float cap);
/* retrieve_hybrid_into (src/memory.rs:568-660) for n_q queries against one
 * bank state (gate [count], age [count]); outputs as oracle_retrieve_batch,
 * plus weights [n_q, capacity] (may be NULL).  out_idx lists the live slots
 * in ascending order when top_k selects. */
void oracle_retrieve_hybrid_batch(const float* keys, const float* norm_sq, const float* values,
                                  size_t count, size_t capacity, size_t d_key, size_t d_val,
                                  const float* q_pnc, size_t n_q, float tau, size_t top_k,
                                  const float* gate, const uint64_t* age, float lam,
                                  float* out_val, float* out_min, uint32_t* out_idx,
                                  float* out_weights, int threads);

/* Stage twins. */
void oracle_gemm_xwt(const float* x, const float* w, size_t m, size_t n, size_t k, float* y);
void oracle_ssm_forward(const float* delta, const float* b_proj, const float* x_norm,
                        const float* rates, const float* c_proj, const float* initial,
                        size_t seq_len, size_t d_m, size_t d_s, float* bar_a,
                        float* bar_b, float* states, float* y);

/* Model paths.  `state` is the per-block carry [depth, d*s], updated. */
void oracle_forward_inference(const oracle_model* m, float* state, uint32_t id,
                              float* logits /* [V] or NULL */);
int oracle_prefill(const oracle_model* m, float* state, const uint32_t* ids, size_t n,
                   float* logits /* [V] or NULL */);
/* Independent lanes, each with its own carry, on `threads` threads. */
int oracle_prefill_lanes(const oracle_model* m, float* states /* [lanes, depth, d*s] */,
                         const uint32_t* ids /* [lanes, n] */, size_t lanes, size_t n,
                         float* logits /* [lanes, V] or NULL */, int threads);
/* Depth-one training forward of one chunk: scaled logits [n,V] and mean loss
 * (PSSALayerV2::forward_train_chunk, src/pssa.rs:2597-2752). */
float oracle_train_chunk_forward(const oracle_model* m, float* state, const uint32_t* ids,
                                 const uint32_t* targets, size_t n, float* logits);
/* Per-token features of the last block (z after residual), for tests. */
void oracle_forward_features(const oracle_model* m, float* state, uint32_t id, float* features);
/* Greedy argmax over ids 1..V-1 in f32::total_cmp order, ties to the lower
 * id (src/inference.rs:123-127). */
uint32_t oracle_greedy(const float* logits, size_t v);
// sample() at temperature 0 (src/inference.rs:104-127) with the repetition
// penalty over the last 64 history ids; logits are penalised in place.
// Returns the id, or -1 for non-finite logits.
int64_t oracle_sample_greedy(float* logits, size_t v, const uint32_t* hist, size_t n_hist, float penalty);
// sample() at any temperature (src/inference.rs:102-178); rng_state is the
// caller's SimpleRng state, advanced by one draw when temperature > 0.
int64_t oracle_sample(float* logits, size_t v, const uint32_t* hist, size_t n_hist, float penalty,
                      float temperature, float top_p, size_t top_k, uint64_t* rng_state);


/* Dense-transition scan h_t = A_t h_{t-1} + b_t, sequential. */
void oracle_dense_scan(const float* a, const float* b, const float* h0, size_t batch,
                       size_t seq_len, size_t s, float* h, int threads);

/* Hebbian fast-weight rule of dream replay (src/pssa.rs:1814-1832). */
void oracle_hebbian_update(float* up_fast, const float* target, const float* current,
                           const float* act, size_t d, size_t r);

/* forward_inference plus per-block taps: q_pnc [depth,k], z_final [depth,d],
 * ad_out [depth,d] (adapter output), act [depth,r] (adapter activations). */
void oracle_forward_taps(const oracle_model* m, float* state, uint32_t id, float* q_pnc,
                         float* z_final, float* ad_out, float* act, float* logits);

/* Greedy decode of `lanes` streams for `steps` steps from ids[lanes] (updated
 * to the last generated ids); out_ids [steps, lanes].  plastic != 0 adds the
 * per-step lane-ordered protected bank write and Hebbian adapter update;
 * the model's banks and adapter_up are modified in place.  logits_last and
 * surprise_last (may be NULL) receive the last step's [lanes, V] logits and
 * [lanes] surprise.  Returns -1 on an id outside the vocabulary. */
int oracle_decode(oracle_model* m, float* states, uint32_t* ids, size_t lanes, size_t steps,
                  int plastic, uint64_t step_base, uint32_t* out_ids, float* logits_last,
                  float* surprise_last, int threads);

#ifdef __cplusplus
}
#endif
#endif

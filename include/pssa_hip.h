/*
 * pssa_hip.h -- C ABI of the MI355X (gfx950) PSSA inference forward path.
 *
 * This is the drop-in boundary a Rust FFI crate binds to add a `Hip` variant
 * next to the reference's CPU / WebGPU / CUDA backends.  It mirrors the
 * reference's backend surface (Sparticle62ops/pssa):
 *
 *   enum Device / enum GpuDispatch ........ src/backend.rs:1013-1446
 *   CudaContext::init / fatal policy ...... src/cuda.rs:169-192, 592-602
 *   PSSALayerV2::{forward_inference,
 *                 prefill_inference} ...... src/pssa.rs:2387-2442
 *
 * Conventions (same as the reference's contract, src/backend.rs:11-48,
 * src/cuda.rs:520-589):
 *   - All matrices are row-major.  Y = X * W^T with X [batch*M, K], W [N, K].
 *   - Every pointer comes with its element count; counts and shapes are
 *     validated before any allocation or launch.  On a validation error the
 *     return is PSSA_HIP_EINVAL, `err` holds the reason, outputs are untouched.
 *   - Calls taking host buffers are synchronous: they return after the results
 *     are copied back and the stream is synchronised.
 *   - Errors raised by the device after a launch are fatal
 *     (pssa_hip_is_fatal() != 0): the caller must not fall back silently,
 *     matching panic_if_fatal_cuda_error (src/cuda.rs:592-602).
 *   - A context may be used from one thread at a time (the reference
 *     serialises its CUDA context behind a Mutex, src/cuda.rs:155-166); this
 *     library locks internally.
 *   - `err`/`err_len` may be NULL/0.
 */
#ifndef PSSA_HIP_H
#define PSSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PSSA_HIP_ABI_VERSION 1

/* Status codes. */
#define PSSA_HIP_OK 0
#define PSSA_HIP_EINVAL (-1)      /* argument/shape validation failed, nothing ran */
#define PSSA_HIP_ENODEV (-2)      /* no usable gfx950 device */
#define PSSA_HIP_ENOMEM (-3)      /* device allocation failed, nothing ran */
#define PSSA_HIP_EDEVICE (-4)     /* HIP runtime or kernel failure: fatal */
#define PSSA_HIP_EUNSUPPORTED (-5)
#define PSSA_HIP_CANCELLED 1          /* pssa_hip_prefill_cancellable stopped early (not an error) */

/* Weight storage types. */
#define PSSA_HIP_F32 0
#define PSSA_HIP_BF16 1

/* Weight initialisation modes (pssa_hip_weights_init). */
#define PSSA_HIP_INIT_REFERENCE 0 /* PSSALayerV2::new draw order, src/pssa.rs:2019-2072 */
#define PSSA_HIP_INIT_BASELINE 1  /* seeded N(0, 0.02) for every matrix; log-spaced rates with
                                     timescales 1.5..13, so exp(ln 2 * A) < 0.95 */

typedef struct pssa_hip_ctx pssa_hip_ctx;       /* device context (CudaContext peer) */
typedef struct pssa_hip_model pssa_hip_model;   /* device-resident weights + banks   */
typedef struct pssa_hip_lanes pssa_hip_lanes;   /* per-lane carries + workspaces     */

/* Model dimensions: PSSAConfigV2 (src/pssa.rs:254-331) fields used by the
 * forward path.  adapter_rank is the adapter's fixed rank (16 in the
 * reference, src/pssa.rs:644). */
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
} pssa_hip_config;

/* Host view of one PSSAContinuousBlockV2 (src/pssa.rs:506-620).  d=d_latent,
 * s=d_state, k=d_mem_key, C=mem_capacity, r=adapter_rank. */
typedef struct {
  float* norm_gamma;       /* [d]            norm_gamma.data                 */
  float* norm_beta;        /* [d]            norm_beta.data                  */
  float* a_raw;            /* [d*s]          a_mat.data (A = -softplus(raw)) */
  float* w_delta;          /* [d,d]                                          */
  float* w_b;              /* [s,d]                                          */
  float* w_c;              /* [s,d]                                          */
  float* w_qx;             /* [k,d]                                          */
  float* w_qh;             /* [k,d]                                          */
  float* w_gate;           /* [d,d]                                          */
  float* w_proj;           /* [d,d]                                          */
  float* adapter_down;     /* [r,d]          adapters[0].down_proj           */
  float* adapter_up;       /* [d,r]          adapters[0].up_proj (fast)      */
  float* adapter_slow;     /* [d,r]          adapters[0].consolidated_up     */
  float* mlp_w1;           /* [2d,d]                                         */
  float* mlp_w2;           /* [d,2d]                                         */
  float* mem_keys;         /* [C,k]          memory.keys                     */
  float* mem_values;       /* [C,d]          memory.values                   */
  float* mem_norm_sq;      /* [C]            memory.norm_sq                  */
  float* mem_confidence;   /* [C]            memory.confidence               */
  uint64_t* mem_last_seen; /* [C]            memory.last_seen_step           */
  uint64_t mem_count;      /*                memory.count                    */
  uint64_t mem_write_head; /*                memory.write_head               */
  /* Hybrid read (src/memory.rs:19-33, runtime-only, never checkpointed). */
  float* mem_hybrid_gate;     /* [C] memory.hybrid_gate; NULL reads as 1.0  */
  uint64_t* mem_hybrid_age;   /* [C] memory.hybrid_age; NULL reads as 0     */
  uint32_t mem_hybrid_enabled; /*    memory.hybrid_enabled                  */
  float mem_hybrid_lam;        /*    memory.hybrid_lam, in (0, 1]           */
  uint64_t mem_top_k;          /*    memory.top_k (runtime-only), 0 = full read */
  float mem_value_cap;         /*    memory.value_cap (runtime-only), 0 = none  */
  uint32_t _pad;
} pssa_hip_block;

/* Host view of PSSALayerV2's inference parameters (src/pssa.rs:1920-1960). */
typedef struct {
  pssa_hip_config cfg;
  float* embed;            /* [V,d] embed_w.data   */
  float* unembed;          /* [V,d] unembed_w.data */
  pssa_hip_block* blocks;  /* [depth]: block, extra_blocks... */
} pssa_hip_weights;

/* ---------------------------------------------------------------- context */

int pssa_hip_abi_version(void);

/* Device::try_gpu / CudaContext::init (src/backend.rs:1467-1482,
 * src/cuda.rs:169-192).  Fails with PSSA_HIP_ENODEV unless `device` is a
 * gfx950 agent. */
int pssa_hip_init(int device, pssa_hip_ctx** out, char* err, size_t err_len);
void pssa_hip_destroy(pssa_hip_ctx* ctx);
/* GpuDispatch::backend_label (src/backend.rs:1439). */
int pssa_hip_device_name(const pssa_hip_ctx* ctx, char* out, size_t out_len);
/* panic_if_fatal_cuda_error classification (src/cuda.rs:592-602). */
int pssa_hip_is_fatal(int code);
int pssa_hip_synchronize(pssa_hip_ctx* ctx, char* err, size_t err_len);

/* Device buffers for the *_resident entry points, for callers without a HIP
 * allocator of their own.  Copies are synchronous on the context stream. */
#define PSSA_HIP_H2D 0
#define PSSA_HIP_D2H 1
#define PSSA_HIP_D2D 2
int pssa_hip_device_alloc(pssa_hip_ctx* ctx, size_t bytes, void** out, char* err, size_t err_len);
void pssa_hip_device_free(pssa_hip_ctx* ctx, void* ptr);
int pssa_hip_memcpy(pssa_hip_ctx* ctx, void* dst, const void* src, size_t bytes, int kind, char* err,
                    size_t err_len);

/* ------------------------------------------------- host-side weight set-up
 * These run on the host only (no device needed). */

/* PSSALayerV2::new (src/pssa.rs:2019-2072) when mode == PSSA_HIP_INIT_REFERENCE:
 * SimpleRng xorshift64* (src/linalg.rs:1-28), Xavier-uniform matrices
 * (src/pssa.rs:86-101) in the reference draw order, HiPPO log-spaced rates
 * (src/pssa.rs:649-665), zero mlp_w2 / adapter up (src/pssa.rs:683,
 * src/adapter.rs:19), empty banks.  Returns the final RNG state in *rng_state. */
int pssa_hip_weights_init(const pssa_hip_weights* w, uint64_t seed, int mode,
                          uint64_t* rng_state, char* err, size_t err_len);
/* Inserts `count` slots into every block's bank through insert()
 * (src/memory.rs:264-303): keys and values uniform in direction with radius
 * U[0, max_radius). */
int pssa_hip_weights_populate_banks(const pssa_hip_weights* w, uint64_t seed, uint64_t count,
                                    float max_radius, char* err, size_t err_len);

/* set_value_cap (src/memory.rs:121-134) on every block of a host model:
 * cap > 0 clamps every capacity slot's value to Euclidean norm <= cap with
 * clamp_value's rule (src/memory.rs:150-170) and records the cap, so later
 * bank writes on the device are capped too; 0 removes the cap and keeps the
 * values.  A negative or non-finite cap is an error. */
int pssa_hip_weights_set_value_cap(const pssa_hip_weights* w, float cap, char* err, size_t err_len);

/* ---------------------------------------------- stage dispatch (GpuDispatch)
 * Host buffers in, host buffers out, synchronous. */

/* GpuDispatch::try_dispatch_gemm_into (src/backend.rs:1049-1085):
 * y[batch*m, n] = x[batch*m, k] * w[n, k]^T.  w_dtype selects the storage of
 * `w` (F32, or BF16 as uint16 bit patterns); accumulation is fp32.  `w` goes
 * through the weight cache below. */
int pssa_hip_gemm_xwt(pssa_hip_ctx* ctx, const float* x, size_t x_len, const void* w,
                      size_t w_len, int w_dtype, size_t m, size_t n, size_t k, size_t batch,
                      float* y, size_t y_len, char* err, size_t err_len);

/* GpuDispatch::gemm_nn_into (src/backend.rs:1152-1168): row-major
 * out[m, n] = a[m, k] * b[k, n], fp32. */
int pssa_hip_gemm_nn(pssa_hip_ctx* ctx, const float* a, size_t a_len, const float* b, size_t b_len, size_t m,
                     size_t k, size_t n, float* out, size_t out_len, char* err, size_t err_len);

/* GpuDispatch::gemm_tn_accumulate_into (src/backend.rs:1170-1184): row-major
 * out[k, n] += a[m, k]^T * b[m, n], fp32. */
int pssa_hip_gemm_tn_accumulate(pssa_hip_ctx* ctx, const float* a, size_t a_len, const float* b, size_t b_len,
                                size_t m, size_t k, size_t n, float* out, size_t out_len, char* err,
                                size_t err_len);

/* GEMM weights stay on the device between calls, keyed by (host address,
 * element count) like the reference's CUDA weight cache (CudaContext::
 * weight_buffer, src/cuda.rs:198-227): pssa_hip_gemm_xwt reuses the copy of
 * a weight it has seen, so a caller that changes a weight's host data in
 * place must invalidate it.  Stale copies are uploaded again on next use. */
typedef struct pssa_hip_weight_key {
  const void* ptr; /* host address of the weight passed to pssa_hip_gemm_xwt */
  size_t len;      /* its element count (w_len) */
} pssa_hip_weight_key;

/* GpuDispatch::invalidate_weights (src/backend.rs:1113-1120, src/cuda.rs:229-240):
 * every cached weight is stale. */
void pssa_hip_invalidate_weights(pssa_hip_ctx* ctx);

/* GpuDispatch::invalidate_weights_only (src/backend.rs:1122-1134,
 * src/cuda.rs:242-252): only the weights with these keys are stale. */
int pssa_hip_invalidate_weights_only(pssa_hip_ctx* ctx, const pssa_hip_weight_key* keys, size_t n_keys,
                                     char* err, size_t err_len);

/* Cached weights: entries, how many are current, device bytes (no reference
 * counterpart; for tests and tools). */
int pssa_hip_weight_cache_stats(pssa_hip_ctx* ctx, size_t* entries, size_t* current, size_t* bytes);

/* GpuDispatch::softplus_in_place (src/backend.rs:1419-1428). */
int pssa_hip_softplus_in_place(pssa_hip_ctx* ctx, float* values, size_t len, char* err,
                               size_t err_len);

/* GpuDispatch::ssm_forward (src/backend.rs:1213-1244):
 *   bar_a = exp(delta_i * rate_ij), bar_b = delta_i * b_j,
 *   h_t = bar_a * h_{t-1} + bar_b * x_i,  y_ti = sum_j h_tij * c_tj.
 * delta/x_norm [L,d], b_proj/c_proj [L,s], rates [d*s] (already -softplus),
 * initial [d*s].  bar_a/bar_b [L*d*s], states [(L+1)*d*s] and final_state
 * [d*s] are optional (NULL = not materialised); y_ssm [L,d] is required.
 * delta_raw / rate_deriv are the reference's backward inputs; they are
 * accepted for signature parity and may be NULL. */
int pssa_hip_ssm_forward(pssa_hip_ctx* ctx, const float* delta, size_t delta_len,
                         const float* delta_raw, const float* b_proj, size_t b_len,
                         const float* x_norm, size_t x_len, const float* rates, size_t rates_len,
                         const float* rate_deriv, const float* c_proj, size_t c_len,
                         const float* initial, size_t initial_len, size_t seq_len, size_t d_m,
                         size_t d_s, float* bar_a, float* bar_b, float* states, float* y_ssm,
                         size_t y_len, float* final_state, char* err, size_t err_len);

/* GpuDispatch::ssm_forward_resident (src/backend.rs:1186-1211): the scan of
 * pssa_hip_ssm_forward with its tape (bar_a, bar_b, states, y_ssm) kept on
 * the device for the next pssa_hip_memory_forward_after_ssm on this context,
 * which consumes it.  A later call replaces an unconsumed tape. */
int pssa_hip_ssm_forward_resident(pssa_hip_ctx* ctx, const float* delta, size_t delta_len,
                                  const float* delta_raw, const float* b_proj, size_t b_len,
                                  const float* x_norm, size_t x_len, const float* rates, size_t rates_len,
                                  const float* c_proj, size_t c_len, const float* initial, size_t initial_len,
                                  size_t seq_len, size_t d_m, size_t d_s, char* err, size_t err_len);

/* GpuDispatch::memory_forward (src/backend.rs:1345-1385) for seq_len rows:
 *   q_euc = x_norm W_qx^T + y_ssm W_qh^T; q_pnc = project(q_euc);
 *   soft read over `count` slots (retrieve_soft_into, src/memory.rs:344-426)
 *   or exact top_k (top_k = 0: full soft read);
 *   g_mem = sigmoid(x_norm W_gate^T); m_proj = m_val W_proj^T; m_inj = g_mem*m_proj.
 * Outputs: q_euc/q_pnc [L,k], q_norm [L], weights [L,capacity], m_val/g_mem/
 * m_proj/m_inj [L,d_val].  Any output except m_inj may be NULL. */
int pssa_hip_memory_forward(pssa_hip_ctx* ctx, const float* x_norm, const float* y_ssm,
                            const float* w_qx, const float* w_qh, const float* w_gate,
                            const float* w_proj, const float* keys, const float* norm_sq,
                            const float* values, size_t seq_len, size_t d_m, size_t d_k,
                            size_t d_val, size_t capacity, size_t count, float tau, size_t top_k,
                            float* q_euc, float* q_pnc, float* q_norm, float* weights,
                            float* m_val, float* g_mem, float* m_proj, float* m_inj, char* err,
                            size_t err_len);

/* GpuDispatch::memory_forward_after_ssm (src/backend.rs:1246-1289): the
 * memory stage on the resident y_ssm of the last pssa_hip_ssm_forward_resident
 * (same seq_len and d_m, else PSSA_HIP_EINVAL), plus copies of that tape:
 * bar_a, bar_b [L*d*s], states [(L+1)*d*s], y_ssm [L,d] (each may be NULL).
 * Other arguments and outputs as pssa_hip_memory_forward. */
int pssa_hip_memory_forward_after_ssm(pssa_hip_ctx* ctx, const float* x_norm, const float* w_qx,
                                      const float* w_qh, const float* w_gate, const float* w_proj,
                                      const float* keys, const float* norm_sq, const float* values,
                                      size_t seq_len, size_t d_m, size_t d_k, size_t d_val, size_t capacity,
                                      size_t count, float tau, size_t top_k, float* bar_a, float* bar_b,
                                      float* states, float* y_ssm, float* q_euc, float* q_pnc, float* q_norm,
                                      float* weights, float* m_val, float* g_mem, float* m_proj, float* m_inj,
                                      char* err, size_t err_len);

/* Batched retrieve_soft_into (src/memory.rs:344-426; the reference's parallel
 * per-query read, src/gpu_batch.rs:700-740) for n_q projected queries
 * q_pnc [n_q, d_key] over `count` occupied slots.  top_k = 0: full soft
 * read; otherwise exact top-k by (distance bits, slot).  out_val
 * [n_q, d_val] required; out_min [n_q], out_idx [n_q, top_k] (ascending slot
 * order) and out_weights [n_q, capacity] optional. */
int pssa_hip_retrieve(pssa_hip_ctx* ctx, const float* q_pnc, size_t n_q, const float* keys,
                      const float* norm_sq, const float* values, size_t capacity, size_t count,
                      size_t d_key, size_t d_val, float tau, size_t top_k, float* out_val,
                      float* out_min, uint32_t* out_idx, float* out_weights, char* err,
                      size_t err_len);

/* pssa_hip_retrieve on device-resident buffers (plain device pointers from
 * any allocator); asynchronous on the context stream. */
int pssa_hip_retrieve_resident(pssa_hip_ctx* ctx, const float* d_q_pnc, size_t n_q,
                               const float* d_keys, const float* d_norm_sq, const float* d_values,
                               size_t capacity, size_t count, size_t d_key, size_t d_val, float tau,
                               size_t top_k, float* d_out_val, float* d_out_min,
                               uint32_t* d_out_idx, char* err, size_t err_len);

/* pssa_hip_retrieve_resident without any device allocation.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Results equal pssa_hip_retrieve_resident's bit for bit.  The
 * exact top-k path runs 8192 queries per pass in a static scratch array of
 * 19 MiB that each GPU the library runs on holds until the process ends;
 * a shape needing more scratch fails with PSSA_HIP_EINVAL.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (from two
 * contexts, or two streams) race and must be serialised by the caller. */
int pssa_hip_retrieve_resident_noalloc(pssa_hip_ctx* ctx, const float* d_q_pnc, size_t n_q,
                                       const float* d_keys, const float* d_norm_sq, const float* d_values,
                                       size_t capacity, size_t count, size_t d_key, size_t d_val, float tau,
                                       size_t top_k, float* d_out_val, float* d_out_min,
                                       uint32_t* d_out_idx, char* err, size_t err_len);

/* retrieve_hybrid_into (src/memory.rs:568-660) for n_q queries against one
 * bank state: over the live slots (the top_k nearest by (distance bits, slot),
 * or all when top_k is 0 or >= count) w_i = exp((min_dist - d_i)/tau) *
 * gate[i] * (float)exp(age[i] * ln(lam)), renormalised; a read whose live
 * weights are all zero falls back to the unweighted softmax.  gate and age
 * [count] are the bank's hybrid_gate / hybrid_age (the caller bumps ages
 * before the read, as forward_inference does).  Outputs as pssa_hip_retrieve;
 * out_idx [n_q, top_k] lists the live slots in ascending order. */
int pssa_hip_retrieve_hybrid(pssa_hip_ctx* ctx, const float* q_pnc, size_t n_q, const float* keys,
                             const float* norm_sq, const float* values, size_t capacity, size_t count,
                             size_t d_key, size_t d_val, float tau, size_t top_k, const float* gate,
                             const uint64_t* age, float lam, float* out_val, float* out_min,
                             uint32_t* out_idx, float* out_weights, char* err, size_t err_len);

/* Dense-transition scan h_t = A_t h_{t-1} + b_t (no reference counterpart:
 * the reference's SSM is diagonal; this is the standalone dense kernel).
 * a [batch, L, s, s] row-major (h_t[r] = sum_c A_t[r][c] h_{t-1}[c] + b_t[r]),
 * b [batch, L, s], h0 [batch, s] (NULL = zeros), h [batch, L, s].
 * Accuracy: every h_t is an exact fp32 step (fused multiply-adds) from the
 * state before it.  With s = 64 and L >= 256 (16-byte aligned a and b) the
 * state entering each 32-step sub-chunk is carried through the composed
 * maps of the sub-chunks before it in its 128-step window, products of
 * bf16 hi/lo splits (about 2^-17 relative per factor); a composed map that
 * is not finite or does not contract (Frobenius norm above 1) is not used,
 * and those sub-chunks are replayed step by step in fp32 instead, so
 * orthogonal or growing transitions get the exact recurrence's accuracy. */
int pssa_hip_dense_scan(pssa_hip_ctx* ctx, const float* a, const float* b, const float* h0,
                        size_t batch, size_t seq_len, size_t d_state, float* h, char* err,
                        size_t err_len);

/* Same recurrence on device-resident buffers (plain device pointers from any
 * allocator); asynchronous on the context stream once the context's scratch
 * holds the two-level schedule's maps for this shape.  A first call with a
 * larger shape grows that scratch (stream synchronise, free, allocate):
 * call pssa_hip_dense_scan_reserve beforehand to keep every call
 * asynchronous and allocation-free. */
int pssa_hip_dense_scan_resident(pssa_hip_ctx* ctx, const float* d_a, const float* d_b,
                                 const float* d_h0, size_t batch, size_t seq_len, size_t d_state,
                                 float* d_h, char* err, size_t err_len);

/* Grows the context's scratch (synchronously) to what a dense scan of this
 * shape needs; later pssa_hip_dense_scan_resident calls of this or a
 * smaller shape allocate nothing. */
int pssa_hip_dense_scan_reserve(pssa_hip_ctx* ctx, size_t batch, size_t seq_len, size_t d_state, char* err,
                                size_t err_len);

/* ------------------------------------------------------------ model paths */

/* Upload the weights (converted to `weight_dtype`), banks and the cached
 * rates -softplus(a_raw) (refresh_ssm_rates, src/pssa.rs:787-796). */
int pssa_hip_model_load(pssa_hip_ctx* ctx, const pssa_hip_weights* w, int weight_dtype,
                        pssa_hip_model** out, char* err, size_t err_len);
void pssa_hip_model_free(pssa_hip_model* model);

/* Independent lanes (SequenceBatch, src/sequence_batch.rs:21-78) sharing one
 * model: each lane owns a carry [depth, d*s] (h_persistent per block).
 * max_tokens bounds lanes*seq_len of a prefill call.  Carries start at zero. */
int pssa_hip_lanes_create(pssa_hip_ctx* ctx, const pssa_hip_model* model, size_t lanes,
                          size_t max_tokens, pssa_hip_lanes** out, char* err, size_t err_len);
void pssa_hip_lanes_free(pssa_hip_lanes* lanes);
/* reset_recurrent_state (src/pssa.rs:2245-2250) for every lane. */
int pssa_hip_lanes_reset(pssa_hip_lanes* lanes, char* err, size_t err_len);
/* carry layout [lanes, depth, loops, d*s] (loops = 1 unless
 * pssa_hip_lanes_set_loops; the SSM part of copy_recurrent_state_to,
 * src/pssa.rs:2263-2281). */
int pssa_hip_lanes_get_carry(pssa_hip_lanes* lanes, float* out, size_t len, char* err,
                             size_t err_len);
int pssa_hip_lanes_set_carry(pssa_hip_lanes* lanes, const float* in, size_t len, char* err,
                             size_t err_len);

/* prefill_inference (src/pssa.rs:2399-2442) on every lane: ids [lanes, seq_len]
 * continue each lane's carry; logits_last [lanes, V] receives the last
 * token's logits (may be NULL for a zero generation budget).  An id >= V
 * follows the reference (src/pssa.rs:2411-2418): each lane first consumes
 * the ids before its first invalid one, then the call fails with "prompt ID
 * <id> outside model vocabulary" (the first lane's) and leaves logits_last
 * alone.  Shape errors fail before anything runs. */
int pssa_hip_prefill(pssa_hip_lanes* lanes, const uint32_t* ids, size_t n_lanes, size_t seq_len,
                     float* logits_last, size_t logits_len, char* err, size_t err_len);

/* prefill_inference on lanes 0..n_lanes-1 with their own prompt lengths
 * (the ragged form of the stage API's inference row, lens[B]): lane i
 * consumes lens[i] >= 1 ids, packed in lane order in `ids`, from its carry;
 * logits_last [n_lanes, V] (may be NULL) receives each lane's last-token
 * logits.  Lanes run together as in pssa_hip_prefill: a hybrid read sees
 * token t of every lane with the ages bumped t + 1 times, and the ages end
 * max(lens) higher. */
int pssa_hip_prefill_ragged(pssa_hip_lanes* lanes, const uint32_t* ids, const uint64_t* lens, size_t n_lanes,
                            float* logits_last, size_t logits_len, char* err, size_t err_len);

/* prefill_inference with its cancellation callback (src/pssa.rs:2399-2418):
 * `cancelled(user)` is asked before every `chunk` tokens (chunk = 1 asks
 * before every token, as the reference does); a nonzero answer stops the
 * prefill with PSSA_HIP_CANCELLED, the carries advanced through the
 * *processed tokens and logits_last untouched.  Invalid ids as in
 * pssa_hip_prefill, within the chunk they fall in.  n_lanes * min(chunk,
 * seq_len) must fit max_tokens.  Results equal pssa_hip_prefill bit for bit. */
typedef int (*pssa_hip_cancel_fn)(void* user);
int pssa_hip_prefill_cancellable(pssa_hip_lanes* lanes, const uint32_t* ids, size_t n_lanes, size_t seq_len,
                                 size_t chunk, pssa_hip_cancel_fn cancelled, void* user, float* logits_last,
                                 size_t logits_len, size_t* processed, char* err, size_t err_len);

/* forward_inference (src/pssa.rs:2387-2391): one token per lane. */
int pssa_hip_forward_inference(pssa_hip_lanes* lanes, const uint32_t* ids, size_t n_lanes,
                               float* logits, size_t logits_len, char* err, size_t err_len);

/* ------------------------------------------------- batch training forward */

/* One training sequence of a batch (Sequence, src/sequence_batch.rs:21-28). */
typedef struct pssa_hip_sequence {
  uint64_t lane;            /* stable lane index; omitted lanes keep their carry */
  const uint32_t* inputs;   /* [len] input ids */
  const uint32_t* targets;  /* [len] target ids */
  uint64_t len;             /* 1..=max_tokens */
  uint32_t reset;           /* nonzero: zero this lane's carry first */
  uint32_t _pad;
} pssa_hip_sequence;

/* SequenceBatch::forward (src/sequence_batch.rs:233-384; the stages of
 * forward_train_chunk_batched, src/gpu_batch.rs:1699-1755, per lane of
 * stacked depth, src/sequence_batch.rs:560-609): each sequence runs from its
 * lane's carry, every token row gets its scaled logits and cross-entropy
 * loss, and *out_loss is the token mean over the packed batch (sequences in
 * the given order, summed left to right in f32).  The logits of every row
 * stay on the device; token_losses [tokens] and logits [tokens, V] (packed
 * order, either may be NULL) receive copies.  Errors, before anything runs:
 * a sequence count outside 1..=lanes, repeated or out-of-range lanes, an
 * empty or over-long sequence, more than max_tokens tokens in all, an id >=
 * V, a model with the hybrid read on (the reference's batched stages reject
 * it).  A non-finite loss is reported after the carries have advanced, as in
 * the reference. */
int pssa_hip_batch_forward(pssa_hip_lanes* lanes, const pssa_hip_sequence* seqs, size_t n_seqs,
                           float* out_loss, float* token_losses, size_t token_losses_len, float* logits,
                           size_t logits_len, char* err, size_t err_len);

/* Device-resident prefill for measurement: stage ids on the device once,
 * then run prefill with no host traffic (asynchronous on the context stream;
 * pssa_hip_synchronize or a read completes it).  read_logits copies the last
 * prefill's last-token logits [lanes of that prefill, V]. */
int pssa_hip_lanes_stage_ids(pssa_hip_lanes* lanes, const uint32_t* ids, size_t n_lanes,
                             size_t seq_len, char* err, size_t err_len);
int pssa_hip_lanes_prefill_staged(pssa_hip_lanes* lanes, char* err, size_t err_len);
int pssa_hip_lanes_read_logits(pssa_hip_lanes* lanes, float* out, size_t len, char* err,
                               size_t err_len);

/* ----------------------------------------------------------------- decode */

#define PSSA_HIP_DECODE_PLASTIC 1 /* apply the plastic write rules after every step */
#define PSSA_HIP_DECODE_GRAPH 2   /* replay one hipGraph-captured step */

/* Greedy decode of `steps` tokens on lanes 0..n_lanes-1, each continuing its
 * carry: every step is forward_inference (src/pssa.rs:2387-2391) on the
 * lane's current token followed by the greedy choice over ids 1..V-1 in
 * f32::total_cmp order, ties to the lower id (sample() at temperature 0,
 * src/inference.rs:123-127).  out_ids [steps, n_lanes] receives the
 * generated ids.  first_ids NULL continues the last prefill (which must have
 * covered the same n_lanes lanes, with no reset, carry change or decode since)
 * as the reference's generate loop does (src/inference.rs:367-379): row 0 is
 * the greedy choice from the prefill's logits and each later row costs one
 * step on the row before it (steps - 1 steps).  first_ids [n_lanes] instead
 * are fed to a first step, and every row costs a step; a decode continues
 * with its last row as first_ids, since that token is not yet consumed.
 * logits_last [n_lanes, V] (may be NULL) receives the logits of the last
 * choice.  The choice applies the lanes' repetition penalty (see
 * pssa_hip_lanes_set_repetition_penalty); non-finite logits fail the call
 * with "model emitted non-finite logits" once its steps have run, as
 * sample() refuses them (src/inference.rs:110-112).
 *
 * PSSA_HIP_DECODE_PLASTIC adds, after each step and block by block in lane
 * order, the refractory-protected bank write of the lane's projected query and
 * block output when the surprise -log softmax(logits)[chosen] exceeds 3.5
 * (insert_protected, src/memory.rs:305-342; write rule of
 * insert_training_memory_at, src/pssa.rs:3705-3736), and the Hebbian update of
 * the adapter's fast weights toward the block output (dream_replay_value,
 * src/pssa.rs:1814-1832).  The reference applies neither during inference;
 * this composition is an extension of its decode step.  The model's banks and
 * fast weights change; its step counter advances by one per step.
 * PSSA_HIP_DECODE_GRAPH captures one step into a hipGraph (once per lane
 * count and flag set) and replays it; results equal the eager steps. */
/* The per-block taps of the last plastic decode step, for lanes 0..n_lanes-1
 * (n_lanes must be that step's lane count): the projected query q_pnc
 * [n_lanes, d_mem_key], the block output z_final [n_lanes, d_latent]
 * (memory value and Hebbian target), the adapter output [n_lanes, d_latent]
 * and the adapter activations [n_lanes, adapter_rank] of block `layer`, the
 * quantities the reference's write rule and dream_replay_value read
 * (src/pssa.rs:1814-1832, 3705-3736).  Any output may be NULL. */
int pssa_hip_lanes_get_taps(pssa_hip_lanes* lanes, size_t layer, size_t n_lanes, float* q_pnc, float* z_final,
                            float* ad_out, float* act, char* err, size_t err_len);

/* InferenceConfig::repetition_penalty for the lanes' greedy choice
 * (sample(), src/inference.rs:113-121): before each choice the logits of the
 * lane's last 64 consumed ids (prompt and generated, since the last
 * pssa_hip_lanes_reset) are divided by `penalty` when positive and
 * multiplied otherwise, once per occurrence.  1 (the default) turns it off,
 * the benchmark's pure argmax; the reference's default is 1.25.  Must be
 * finite and >= 1 (src/inference.rs:97-99). */
int pssa_hip_lanes_set_repetition_penalty(pssa_hip_lanes* lanes, float penalty, char* err, size_t err_len);

/* set_loops (src/pssa.rs:2171-2184; forward_inference_features,
 * src/pssa.rs:2338-2373): every block runs `loops` passes per token, each with
 * its own carry and adding output / loops to the features it read; every
 * block after the first returns input + features / sqrt(depth).  1..=32; 1 is
 * the original model.  Loop 0 keeps each block's carry, the others start at
 * zero; pssa_hip_lanes_reset zeroes all.  Prefill, forward_inference and the
 * greedy or sampled decode run looped; the batched training forward, plastic
 * decode and the hybrid read are PSSA_HIP_EUNSUPPORTED with loops > 1 here. */
int pssa_hip_lanes_set_loops(pssa_hip_lanes* lanes, size_t loops, char* err, size_t err_len);

/* InferenceConfig::{temperature, top_p, top_k} for the lanes' choice
 * (sample(), src/inference.rs:128-178; validation :87-100).  temperature 0 (the
 * default) is the greedy choice.  Above 0 each choice draws one value from the
 * lane's SimpleRng (src/linalg.rs:5-28), which this call seeds with `seed` for
 * every lane (the reference's engine uses SimpleRng::new(1337),
 * src/inference.rs:73); the states then persist across decode calls and
 * resets.  Probabilities are exp((logit - max) / temperature) over ids
 * 1..V-1 after the repetition penalty, summed in id order; the first top_k
 * in (probability desc, id asc) order, cut where their running sum reaches
 * top_p, are drawn from.  Must satisfy temperature finite >= 0, top_p finite
 * in (0, 1], top_k >= 1; top_k above 64 with temperature > 0 is
 * PSSA_HIP_EUNSUPPORTED here.  An invalid probability mass fails the decode
 * with "invalid sampling probability mass". */
int pssa_hip_lanes_set_sampling(pssa_hip_lanes* lanes, float temperature, float top_p, size_t top_k,
                                uint64_t seed, char* err, size_t err_len);

int pssa_hip_decode(pssa_hip_lanes* lanes, const uint32_t* first_ids, size_t n_lanes,
                    size_t steps, int flags, uint32_t* out_ids, size_t out_len,
                    float* logits_last, size_t logits_len, char* err, size_t err_len);

/* Reads one block's plastic state back from the device: adapter fast
 * weights [d,r], bank keys [C,k], values [C,d], norm_sq [C], confidence [C],
 * last_seen [C], count, write_head, and the model's step counter.  Any
 * pointer may be NULL. */
int pssa_hip_model_get_plastic(pssa_hip_model* model, size_t layer, float* adapter_up, float* keys,
                               float* values, float* norm_sq, float* confidence,
                               uint64_t* last_seen, uint64_t* count, uint64_t* write_head,
                               uint64_t* step, char* err, size_t err_len);

/* set_hybrid_read (src/pssa.rs:2232-2243, src/memory.rs:510-518) on every
 * block: lam must be finite and in (0, 1].  With the hybrid read on, every
 * forward step first ages each live slot by one (bump_hybrid_ages,
 * src/memory.rs:501-507) and then reads with retrieve_hybrid_into
 * (src/pssa.rs:1153-1162); all lanes of a call advance together, so token t
 * of a prefill reads with the ages bumped t + 1 times and the ages end T
 * higher (one lane: exactly the reference's token loop).  The plastic decode
 * write becomes insert_gated_protected (src/memory.rs:524-556) with the gate
 * the mean of the block's memory-injection gate at the written token
 * (src/pssa.rs:3719-3726).  Every bank write resets the slot's gate to 1.0
 * (gated writes: to that gate) and its age to 0 (src/memory.rs:300-301). */
int pssa_hip_model_set_hybrid_read(pssa_hip_model* model, int enabled, float lam, char* err,
                                   size_t err_len);

/* set_memory_top_k (src/pssa.rs:2215-2226) on every block: each read keeps
 * the top_k nearest slots by (distance bits, slot) and renormalises over
 * them (retrieve_soft_into, src/memory.rs:380-407); 0 = the full read (the
 * reference's None).  At most 64 here. */
int pssa_hip_model_set_memory_top_k(pssa_hip_model* model, size_t top_k, char* err, size_t err_len);

/* set_value_cap (src/memory.rs:121-134) on every block of a loaded model:
 * cap > 0 clamps every slot's value to Euclidean norm <= cap (clamp_value,
 * src/memory.rs:150-170, bit for bit) and caps the plastic decode's bank
 * writes; 0 removes the cap and keeps the values. */
int pssa_hip_model_set_value_cap(pssa_hip_model* model, float cap, char* err, size_t err_len);

/* Reads one block's hybrid-read state back from the device: gate [C] and
 * age [C] (either may be NULL). */
int pssa_hip_model_get_hybrid(pssa_hip_model* model, size_t layer, float* gate, uint64_t* age,
                              char* err, size_t err_len);

/* Per-stage kernel time (ms, summed over layers) of the most recent prefill,
 * recorded with HIP events on the stream the kernels run on.  enable = 1 turns
 * recording on for later calls, 0 off, -1 leaves it unchanged.  names/ms
 * arrays of `cap` entries (either may be NULL); returns the number of stages. */
int pssa_hip_lanes_stage_times(pssa_hip_lanes* lanes, int enable, const char** names, float* ms,
                               size_t cap);

#ifdef __cplusplus
}
#endif
#endif /* PSSA_HIP_H */

// Poincare-ball episodic memory read (HyperbolicEpisodicBankV2, src/memory.rs).
#pragma once
#include "common.h"

namespace pssa {

struct RetrieveArgs {
  const float* q = nullptr;     // queries [n, ld_q]: Euclidean (project=1) or already in the ball
  int ld_q = 0;
  int project = 1;
  float* q_pnc = nullptr;       // optional [n, dk] projected queries
  float* q_norm = nullptr;      // optional [n] ||q_euc|| (diffeomorphic_project's return)
  const float* keys = nullptr;  // [capacity, dk]
  const float* norm_sq = nullptr;  // [capacity]
  const float* values = nullptr;   // [capacity, dv] (needed when top_k > 0)
  int n = 0, dk = 0, dv = 0, capacity = 0, count = 0;
  const int* count_dev = nullptr;  // when set, the occupied-slot count is read from device memory
  float tau = 0.1f;
  int top_k = 0;                // 0: full soft read -> weights only (readout is a GEMM)
  float* weights = nullptr;     // [n, capacity]; optional
  uint16_t* weights16 = nullptr;  // [n, capacity] bf16 bits; optional (operand of a bf16 readout)
  float* out_val = nullptr;     // [n, dv] (top-k readout)
  float* out_min = nullptr;     // optional [n]
  uint32_t* out_idx = nullptr;  // optional [n, top_k], ascending slot order
  // Device scratch for the ranked top-k path (retrieve_scratch_bytes); when
  // absent or too small the general kernel runs instead.
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  int chunk = 0;  // queries per ranked dot/pick pass (0: the default, 32768)
  // Hybrid read (retrieve_hybrid_into, src/memory.rs:568-660): with hgate
  // set, live slot s weighs exp((min - d_s)/tau) * hgate[s] * decay_s,
  // decay_s = (float)exp(age_s * log_lam), age_s = hage[s] + age_base
  // (+ row % age_T + 1 when age_T > 0, the bumps of a T-token prefill's
  // earlier tokens), saturating; a read whose live weights sum to zero falls
  // back to the unweighted softmax.  hage may be null (ages 0).
  const float* hgate = nullptr;
  const unsigned long long* hage = nullptr;
  double log_lam = 0.0;
  unsigned long long age_base = 0;
  int age_T = 0;
  // Fused query product (a decode step's few-query soft read, see
  // retrieve_fuses_query): with qw set the Euclidean query of row r is
  // qa[r] . qw^T + qaux[r], qa [n, ld_qa] bf16 rows, qw [dk, qk] bf16
  // (K-contiguous), qaux [n, ld_qaux] fp32, formed on the matrix cores in the
  // tiled GEMMs' K order and summed with qaux as their ADD_AUX epilogue does,
  // so it is the q a separate product writes; q is not read.
  const uint16_t* qa = nullptr;
  int ld_qa = 0;
  const uint16_t* qw = nullptr;
  int qk = 0;
  const float* qaux = nullptr;
  int ld_qaux = 0;
};

// Whether launch_retrieve forms the query product itself for these
// arguments (qa, qw and qaux set): the few-query soft read with one query
// per wave, d_key <= 32, qk % 128 == 0 and the panels within LDS.
bool retrieve_fuses_query(const RetrieveArgs& a);

// Scratch the ranked top-k path needs for these arguments (0: not taken).
size_t retrieve_scratch_bytes(const RetrieveArgs& a);

// The allocation-free retrieval (pssa_hip_retrieve_resident_noalloc) runs
// the ranked path kNoallocChunk queries per pass in a static per-device
// scratch array of kNoallocScratchBytes.
constexpr int kNoallocChunk = 8192;
constexpr size_t kNoallocScratchBytes = (size_t)19 << 20;  // 19 MiB
// The device address of the current device's scratch array (resolved once
// per device with hipGetSymbolAddress; call with the device current).
Status noalloc_scratch_address(void** out);

Status launch_retrieve(hipStream_t stream, const RetrieveArgs& a);
// One-time per-device set-up a later launch_retrieve with these arguments
// needs (call it outside graph capture).
Status prepare_retrieve(const RetrieveArgs& a);
// Per-device kernel attributes (large dynamic LDS), set at context creation
// so that no attribute call happens during graph capture.
Status init_retrieve_attributes();

constexpr int kMaxTopK = 64;

// Per-row Euclidean norm caps of clamp_rows: c[r / rows_per_cap] (<= 0: none).
struct ValueCaps {
  float c[32];
};
// clamp_value (src/memory.rs:150-170) on rows [n_rows, d], src -> dst.  A
// capped row with a non-finite norm is copied and sets *bad = 1 (may be null).
Status launch_clamp_rows(hipStream_t stream, const float* src, float* dst, int n_rows, int d, size_t ld,
                         const ValueCaps& caps, int rows_per_cap, int* bad);

}  // namespace pssa

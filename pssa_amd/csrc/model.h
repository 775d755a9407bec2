// Device-resident PSSA model and per-lane prefill/decode state.
#pragma once
#include <array>

#include "common.h"

namespace pssa {

constexpr int kMaxDepth = 32;  // PSSAConfigV2 depth limit enforced by check_config

struct DevBlock {
  DevBuf w_in;     // [n_in, d]: W_delta; W_B; W_C; W_qx; W_gate; adapter D  (weight dtype)
  DevBuf w_qh;     // [k, d]
  DevBuf w_proj;   // [d, d]
  DevBuf mlp_w1;   // [2d, d]
  DevBuf mlp_w2;   // [d, 2d]
  DevBuf u_eff;    // [d, r] weight dtype: adapter fast + consolidated weights (the GEMM operand)
  DevBuf u_fast;   // [d, r] f32: adapters[0].up_proj, updated by plastic decode
  DevBuf u_slow;   // [d, r] f32: adapters[0].consolidated_up
  DevBuf gamma;    // [d] f32
  DevBuf beta;     // [d] f32
  DevBuf rates2;   // [d*s] f32: -softplus(a_raw) * log2(e)
  DevBuf keys;     // [C, k] f32
  DevBuf norm_sq;  // [C] f32
  DevBuf values;   // [C, d] f32 (top-k readout)
  DevBuf values_t; // [d, C] weight dtype (soft-read readout GEMM operand)
  DevBuf conf;     // [C] f32 memory.confidence
  DevBuf last_seen;  // [C] u64 memory.last_seen_step
  DevBuf meta;     // int32 [2]: memory.count, memory.write_head
  // Hybrid read (src/memory.rs:19-33): per-slot write gate and age on the
  // device, the toggle and ln(lam) on the host.
  DevBuf hgate;    // [C] f32 memory.hybrid_gate
  DevBuf hage;     // [C] u64 memory.hybrid_age
  bool hybrid = false;
  float lam = 1.0f;
  int top_k = 0;  // memory.top_k (src/memory.rs:102-108), 0 = full read
  float value_cap = 0.0f;  // memory.value_cap (src/memory.rs:13-14), 0 = none
};

// Stage ids used for per-kernel timing.
enum Stage : int {
  ST_EMBED = 0,
  ST_NORM,
  ST_GEMM_IN,
  ST_SSM,
  ST_SSM_AUX,
  ST_GEMM_QH,
  ST_RETRIEVE,
  ST_GEMM_READ,
  ST_GEMM_PROJ,
  ST_GEMM_MLP1,
  ST_GEMM_MLP2,
  ST_HEAD,
  ST_COUNT
};
extern const char* const kStageNames[ST_COUNT];

}  // namespace pssa

struct pssa_hip_model {
  pssa_hip_ctx* ctx = nullptr;
  pssa_hip_config cfg{};
  int dtype = PSSA_HIP_F32;
  size_t n_in = 0;  // width of the fused input projection
  pssa::DevBuf embed;    // [V, d] f32 (row gather)
  pssa::DevBuf unembed;  // [V, d] weight dtype
  std::vector<pssa::DevBlock> blocks;
  pssa::DevBuf step;     // u64: step counter read by the refractory gate in plastic decode
  // Advances on every set_hybrid_read / set_memory_top_k, so that a captured
  // decode step built for other read settings is captured again.
  uint64_t hybrid_epoch = 0;
};

struct pssa_hip_lanes {
  pssa_hip_ctx* ctx = nullptr;
  const pssa_hip_model* model = nullptr;
  size_t lanes = 0, max_tokens = 0;
  pssa::DevBuf carry;  // [lanes, depth, d*s]
  pssa::DevBuf ids;    // [max_tokens] u32
  // Activations for max_tokens rows.  fp32: X residual stream [n,d], XN norm
  // output [n,d], P fused input projection [n,n_in], Y SSM readout [n,d],
  // Q memory query [n,k], Zraw [n,d].  Operand type of the model (bf16 or
  // fp32): XNh, Yh, Zrawh (bf16 copies, aliases of the fp32 buffers in an
  // fp32 model), Wm soft-read weights [n,C], Mval read values [n,d],
  // H1 MLP hidden [n,2d].
  pssa::DevBuf X, XN, XNh, P, Y, Yh, Q, Wm, Mval, Zraw, Zrawh, H1, logits;
  pssa::DevBuf Ypart;  // SSM partial readouts when d_state needs more than two state blocks
  // Decode state (allocated on the first decode call): per-block taps of the
  // last step [depth, lanes, *], the surprise of each lane's greedy choice
  // [lanes], the Hebbian rates 0.02/(1+|z_final|) [depth, lanes], the
  // generated ids [gen_cap, lanes] and the generation position.
  pssa::DevBuf tap_q, tap_z, tap_a, tap_act, surprise, hebb_rate, gen_ids, gen_pos;
  pssa::DevBuf tap_gmean;    // [depth, lanes] mean memory-injection gate (hybrid write gate)
  pssa::DevBuf tap_zcap;     // [depth, lanes, d] z_final rows clamped to the value caps (bank writes)
  pssa::DevBuf bank_writer;  // [depth, capacity] writing lane of each slot in the current step
  size_t tap_lanes = 0;      // lanes of the last plastic step whose taps the buffers hold
  // Batch training forward (allocated on its first call): the fp32 scaled
  // logits of every token row [max_tokens, V], each row's target id and
  // packed token index [2, max_tokens], the per-token losses in packed order
  // [max_tokens], and a carry workspace [lanes, depth, d*s] for sequences
  // whose lanes are not 0..n-1 in length order.
  pssa::DevBuf tok_logits, tok_meta, tok_loss, carry_work;
  // Repetition-penalty window (sample(), src/inference.rs:113-121): per lane
  // a ring of the last kHist consumed ids (prompt and generated), its fill
  // count and next position; the penalty (1 = off) and a flag the greedy
  // choice raises on non-finite logits.
  static constexpr int kHist = 64;
  pssa::DevBuf hist, hist_n, hist_pos, nonfinite;
  float rep_penalty = 1.0f;
  float graph_penalty = 1.0f;
  // Sampling at temperature > 0 (sample(), src/inference.rs:128-178): the
  // settings (temperature 0: the greedy choice), each lane's SimpleRng state
  // and the per-lane probability scratch [lanes, V]; the captured step
  // records the settings it was built with.
  // Recurrent depth loops (set_loops, src/pssa.rs:2171-2184): passes per
  // block and token, each with its own carry ([lanes, depth, loops] matrices of d*s);
  // Xin keeps a looped layer's input rows.
  size_t loops = 1;
  pssa::DevBuf Xin;
  float temperature = 0.0f, top_p = 1.0f;
  int top_k = 1;
  pssa::DevBuf rng, probs;
  float graph_temperature = 0.0f, graph_top_p = 1.0f;
  int graph_top_k = 1;
  size_t dec_lanes = 0, gen_cap = 0;
  // Captured decode step (one per lane count and plasticity setting).
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  size_t graph_lanes = 0;
  int graph_plastic = -1;
  uint64_t graph_hybrid_epoch = 0;
  // Ids staged on the device by stage_ids (lanes x len; 0 once `ids` holds
  // anything else) and the lanes whose last-token logits from a prefill are
  // in `logits` (0 when none are: a decode without first ids continues from
  // them).
  size_t staged_lanes = 0, staged_len = 0;
  size_t logit_lanes = 0;
  bool timing = false;
  std::array<float, pssa::ST_COUNT> stage_ms{};
  std::array<int, pssa::ST_COUNT> stage_calls{};
  std::vector<hipEvent_t> events;
  std::vector<int> event_stage;
  // Extra streams (default priority) for the concurrent lane groups of a
  // prefill, and the events that fork, stagger and join them.
  static constexpr int kMaxGroups = 4;
  hipStream_t aux_stream[kMaxGroups - 1] = {};
  hipEvent_t ev_fork = nullptr;
  hipEvent_t ev_first[kMaxGroups - 1] = {}, ev_join[kMaxGroups - 1] = {};
  // Fork and join of a plastic decode step's Hebbian update (aux_stream[0]).
  hipEvent_t ev_tail_fork = nullptr, ev_tail_join = nullptr;
  ~pssa_hip_lanes() {
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
    if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (ev_fork) (void)hipEventDestroy(ev_fork);
    if (ev_tail_fork) (void)hipEventDestroy(ev_tail_fork);
    if (ev_tail_join) (void)hipEventDestroy(ev_tail_join);
    for (int g = 0; g < kMaxGroups - 1; ++g) {
      if (ev_first[g]) (void)hipEventDestroy(ev_first[g]);
      if (ev_join[g]) (void)hipEventDestroy(ev_join[g]);
      if (aux_stream[g]) (void)hipStreamDestroy(aux_stream[g]);
    }
  }
};

namespace pssa {
// Runs prefill for `n_lanes` lanes of `T` tokens whose ids are already in
// lanes->ids (row-major [n_lanes, T]); last-token logits land in lanes->logits.
// With `taps` set (single-token decode) every block also records its
// projected query, adapter output, z_final and adapter activations into the
// lanes' tap buffers.
// `append` adds each lane's consumed ids to its repetition-penalty window
// (a decode step leaves that to the greedy choice, which appends the token
// it consumed).
Status run_prefill(pssa_hip_lanes* L, size_t n_lanes, size_t T, bool taps = false, bool append = true);
// Rows of one segment of a ragged prefill or training forward: n_lanes
// lanes of T tokens.  Every pointer addresses the segment's first row
// (lane).  With `logits` null only each lane's last-token logits are
// computed, into lanes->logits rows 0..n_lanes-1.
struct TrainRows {
  const uint32_t* ids = nullptr;      // [n_lanes * T] input ids
  const uint32_t* targets = nullptr;  // [n_lanes * T] target ids
  const uint32_t* index = nullptr;    // [n_lanes * T] packed token index of each row
  float* logits = nullptr;            // [n_lanes * T, V] scaled logits
  float* loss = nullptr;              // per-token losses, indexed by `index`
  float* carry = nullptr;             // [n_lanes, depth, d*s] carries, advanced in place
};
// The forward of stage_embed_norm .. stage_logits_loss (src/gpu_batch.rs:
// 445-1250) over one segment: every row gets its scaled logits and its
// cross-entropy loss.  The hybrid read is not supported here (the
// reference's batched stages reject it).
Status run_train_segment(pssa_hip_lanes* L, size_t n_lanes, size_t T, const TrainRows& tr);
// One segment of a ragged prefill (last-token logits only; hybrid ages
// advance T as in run_prefill).
Status run_prefill_segment(pssa_hip_lanes* L, size_t n_lanes, size_t T, const TrainRows& rows,
                           const int* lane_map);
// Appends each row's last min(T, kHist) ids of ids [n_lanes, T] to the
// window of lane lane_map[row] (lane_map null: lane = row).
Status launch_hist_append(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t T, const int* lane_map);
// One greedy decode step for n_lanes lanes (ids in lanes->ids, replaced by
// the chosen ids); plastic adds the lane-ordered protected bank writes and
// the Hebbian adapter update.  Only kernel launches: safe to capture.
Status run_decode_step(pssa_hip_lanes* L, size_t n_lanes, bool plastic);
// Greedy choice from lanes->logits without a forward step (first decode
// token after a prefill); with `record` it is also the generated row at
// gen_pos, which then advances.
Status run_greedy_from_logits(pssa_hip_lanes* L, size_t n_lanes, bool record);
// Dynamic LDS of the bank-write kernel and its per-device attribute set-up.
size_t bank_write_lds(int capacity, int lanes);
// LDS of the Hebbian update for adapter rank `rank` and `lanes` lanes.
size_t hebbian_lds(int rank, int lanes);
Status init_decode_attributes();
Status launch_fill_zero(hipStream_t stream, float* p, size_t n);
Status launch_copy_cols(hipStream_t stream, const float* in, int ld_in, float* out, int ld_out,
                        size_t rows, int cols);
Status launch_mul(hipStream_t stream, const float* a, const float* b, float* out, size_t n);
Status launch_softplus(hipStream_t stream, float* p, size_t n);
Status launch_sigmoid(hipStream_t stream, float* p, size_t n);
Status launch_check_ids(hipStream_t stream, const uint32_t* ids, size_t n, uint32_t vocab, int* bad);
}  // namespace pssa

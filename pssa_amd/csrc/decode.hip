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

#include "model.h"

namespace pssa {

namespace {

// f32::total_cmp order: a larger key is a larger value in IEEE total order.
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t b = __float_as_int(f);
  return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

// One workgroup per lane: greedy id over 1..V-1 (ties to the lower id) and
// the surprise logsumexp(logits) - logits[chosen].
__global__ __launch_bounds__(256) void greedy_kernel(const float* __restrict__ logits, int V,
                                                     uint32_t* __restrict__ ids,
                                                     uint32_t* __restrict__ gen_ids,
                                                     const int* __restrict__ gen_pos, int n_lanes,
                                                     float* __restrict__ surprise) {
  __shared__ int32_t sk[256];
  __shared__ int sid[256];
  __shared__ float sm[256];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* lg = logits + (size_t)row * V;
  int32_t bk = INT32_MIN;
  int bi = V;
  float mx = -INFINITY;
  for (int v = tid; v < V; v += 256) {
    const float x = lg[v];
    mx = fmaxf(mx, x);
    if (v >= 1) {
      const int32_t k = total_key(x);
      if (k > bk || (k == bk && v < bi)) {
        bk = k;
        bi = v;
      }
    }
  }
  sk[tid] = bk;
  sid[tid] = bi;
  sm[tid] = mx;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (tid < off) {
      const int32_t k2 = sk[tid + off];
      const int i2 = sid[tid + off];
      if (k2 > sk[tid] || (k2 == sk[tid] && i2 < sid[tid])) {
        sk[tid] = k2;
        sid[tid] = i2;
      }
      sm[tid] = fmaxf(sm[tid], sm[tid + off]);
    }
    __syncthreads();
  }
  const int best = sid[0];
  const float gmax = sm[0];
  __syncthreads();
  float part = 0.0f;
  for (int v = tid; v < V; v += 256) part += expf(lg[v] - gmax);
  sm[tid] = part;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (tid < off) sm[tid] += sm[tid + off];
    __syncthreads();
  }
  if (tid == 0) {
    ids[row] = (uint32_t)best;
    if (gen_ids) gen_ids[(size_t)gen_pos[0] * n_lanes + row] = (uint32_t)best;
    if (surprise) surprise[row] = (gmax + logf(sm[0])) - lg[best];
  }
}

// Per-layer operand pointers of the plastic write kernels (one launch covers
// every block).
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
  const float* tap_a;    // [depth, lanes, d]
  const float* tap_act;  // [depth, lanes, r]
  const float* surprise; // [lanes]
  float* rate;           // [depth, lanes]
  const unsigned long long* step;
  int lanes, C, dk, d, r, wt_bf16;
};

__device__ __forceinline__ uint16_t to_bf16(float v) {
  uint32_t b = __float_as_uint(v);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

// up[i,q] += rate_l * clamp(z_l[i] - a_l[i], -4, 4) * act_l[q] for lanes l in
// order (rounded as the reference: (rate * err) * act, then the add), then
// the GEMM operand u_eff = up + slow in the weight type.  blockIdx.y = block.
__global__ void hebbian_kernel(PlasticArgs p) {
  const int l = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= p.d * p.r) return;
  const int i = e / p.r, q = e % p.r;
  const size_t n = p.lanes;
  const float* z = p.tap_z + (size_t)l * n * p.d;
  const float* a = p.tap_a + (size_t)l * n * p.d;
  const float* act = p.tap_act + (size_t)l * n * p.r;
  const float* rate = p.rate + (size_t)l * n;
  float u = p.up[l][e];
  for (int ln = 0; ln < p.lanes; ++ln) {
    const float err = fminf(fmaxf(z[(size_t)ln * p.d + i] - a[(size_t)ln * p.d + i], -4.0f), 4.0f);
    u = __fadd_rn(u, __fmul_rn(__fmul_rn(rate[ln], err), act[(size_t)ln * p.r + q]));
  }
  p.up[l][e] = u;
  const float eff = u + p.slow[l][e];
  if (p.wt_bf16)
    static_cast<uint16_t*>(p.u_eff[l])[e] = to_bf16(eff);
  else
    static_cast<float*>(p.u_eff[l])[e] = eff;
}

// 0.02 / (1 + |z_final|) per (block, lane): the Hebbian rate of
// dream_replay_value, with the norm as a sequential f64 sum.
__global__ void hebbian_rate_kernel(PlasticArgs p) {
  const int l = blockIdx.y;
  const int ln = blockIdx.x * blockDim.x + threadIdx.x;
  if (ln >= p.lanes) return;
  const float* zr = p.tap_z + ((size_t)l * p.lanes + ln) * p.d;
  double acc = 0.0;
  {
#pragma clang fp contract(off)
    for (int i = 0; i < p.d; ++i) acc = acc + (double)zr[i] * (double)zr[i];
  }
  const double tn = sqrt(acc);
  p.rate[(size_t)l * p.lanes + ln] = 0.02f / (1.0f + (float)fmin(tn, (double)FLT_MAX));
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
  if (tid == 0) {
    const unsigned long long cur = p.step[0] + 1;
    int* meta = p.meta[l];
    int count = meta[0], head = meta[1];
    for (int ln = 0; ln < p.lanes; ++ln) {
      const float sp = s_sp[ln];
      if (!(sp > 3.5f)) continue;
      int idx;
      if (count < C) {  // insert() into a free slot
        idx = count++;
      } else {
        idx = head;
        // RateLimiterGate::apply_refractory_overwrite (src/defense.rs:45-67).
        const unsigned long long last = s_last[idx];
        const float dt = (float)(cur > last ? cur - last : 0ull);
        const float lin = 1.0f - expf(-dt / 60.0f);
        const float gain = fmaxf(lin * lin, 0.005f);
        const float damage = 0.08f * sp * gain;
        if (s_conf[idx] > damage) {
          s_conf[idx] -= damage;
          s_last[idx] = cur;
          continue;
        }
        head = (head + 1) % C;
      }
      s_conf[idx] = 1.0f;
      s_last[idx] = cur;
      writer[idx] = ln;
    }
    meta[0] = count;
    meta[1] = head;
  }
  __syncthreads();
  for (int c = tid; c < C; c += blockDim.x) {
    conf[c] = s_conf[c];
    last_seen[c] = s_last[c];
  }
  const int wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
  const size_t n = p.lanes;
  for (int c = wave; c < C; c += nw) {
    const int ln = writer[c];
    if (ln < 0) continue;
    const float* kq = p.tap_q + ((size_t)l * n + ln) * p.dk;
    const float* vz = p.tap_z + ((size_t)l * n + ln) * p.d;
    for (int j = lane; j < p.dk; j += 64) p.keys[l][(size_t)c * p.dk + j] = kq[j];
    for (int j = lane; j < p.d; j += 64) {
      const float v = vz[j];
      p.values[l][(size_t)c * p.d + j] = v;
      if (p.wt_bf16)
        static_cast<uint16_t*>(p.values_t[l])[(size_t)j * C + c] = to_bf16(v);
      else
        static_cast<float*>(p.values_t[l])[(size_t)j * C + c] = v;
    }
    if (lane == 0) {
      // squared_norm (src/memory.rs:181-192): sequential f64 sum.
      double acc = 0.0;
      {
#pragma clang fp contract(off)
        for (int j = 0; j < p.dk; ++j) acc = acc + (double)kq[j] * (double)kq[j];
      }
      float v = (float)acc;
      if (acc < 1.0 && v == 1.0f) v = __uint_as_float(0x3f7fffffu);
      p.norm_sq[l][c] = v;
    }
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

Status init_decode_attributes() {
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&bank_write_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  return Status::Ok();
}

Status run_greedy_from_logits(pssa_hip_lanes* L, size_t n_lanes) {
  const hipStream_t st = L->ctx->stream;
  const int V = (int)L->model->cfg.d_vocab;
  greedy_kernel<<<(unsigned)n_lanes, 256, 0, st>>>(L->logits.as<float>(), V, L->ids.as<uint32_t>(),
                                                   nullptr, nullptr, (int)n_lanes, nullptr);
  PSSA_LAUNCH_CHECK("greedy");
  return Status::Ok();
}

Status run_decode_step(pssa_hip_lanes* L, size_t n_lanes, bool plastic) {
  const pssa_hip_model* M = L->model;
  const pssa_hip_config& c = M->cfg;
  const hipStream_t st = L->ctx->stream;
  const int d = (int)c.d_latent, k = (int)c.d_mem_key, r = (int)c.adapter_rank, C = (int)c.mem_capacity;
  const int V = (int)c.d_vocab;
  const size_t n = n_lanes;
  PSSA_RETURN_IF(run_prefill(L, n_lanes, 1, plastic));
  greedy_kernel<<<(unsigned)n, 256, 0, st>>>(L->logits.as<float>(), V, L->ids.as<uint32_t>(),
                                             L->gen_ids.as<uint32_t>(), L->gen_pos.as<int>(), (int)n,
                                             L->surprise.as<float>());
  PSSA_LAUNCH_CHECK("greedy");
  if (plastic) {
    PlasticArgs p{};
    for (size_t l = 0; l < c.depth; ++l) {
      const DevBlock& B = M->blocks[l];
      p.keys[l] = B.keys.as<float>();
      p.norm_sq[l] = B.norm_sq.as<float>();
      p.values[l] = B.values.as<float>();
      p.values_t[l] = B.values_t.p;
      p.conf[l] = B.conf.as<float>();
      p.last_seen[l] = B.last_seen.as<unsigned long long>();
      p.meta[l] = B.meta.as<int>();
      p.up[l] = B.u_fast.as<float>();
      p.slow[l] = B.u_slow.as<float>();
      p.u_eff[l] = B.u_eff.p;
    }
    p.tap_q = L->tap_q.as<float>();
    p.tap_z = L->tap_z.as<float>();
    p.tap_a = L->tap_a.as<float>();
    p.tap_act = L->tap_act.as<float>();
    p.surprise = L->surprise.as<float>();
    p.rate = L->hebb_rate.as<float>();
    p.step = M->step.as<unsigned long long>();
    p.lanes = (int)n;
    p.C = C;
    p.dk = k;
    p.d = d;
    p.r = r;
    p.wt_bf16 = M->dtype == PSSA_HIP_BF16 ? 1 : 0;
    const int depth = (int)c.depth;
    bank_write_kernel<<<depth, 256, bank_write_lds(C, (int)n), st>>>(p);
    PSSA_LAUNCH_CHECK("bank_write");
    hebbian_rate_kernel<<<dim3((unsigned)((n + 255) / 256), depth), 256, 0, st>>>(p);
    PSSA_LAUNCH_CHECK("hebbian_rate");
    hebbian_kernel<<<dim3((unsigned)((d * r + 255) / 256), depth), 256, 0, st>>>(p);
    PSSA_LAUNCH_CHECK("hebbian");
    advance_kernel<<<1, 64, 0, st>>>(M->step.as<unsigned long long>(), L->gen_pos.as<int>());
  } else {
    advance_pos_kernel<<<1, 64, 0, st>>>(L->gen_pos.as<int>());
  }
  PSSA_LAUNCH_CHECK("advance");
  return Status::Ok();
}

}  // namespace pssa

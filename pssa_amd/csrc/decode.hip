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

// 0.02 / (1 + |z_final|) per lane (the Hebbian rate of dream_replay_value;
// the norm is a sequential f64 sum).
__global__ void hebbian_rate_kernel(const float* __restrict__ z, int d, int n_lanes,
                                    float* __restrict__ rate) {
  const int ln = blockIdx.x * blockDim.x + threadIdx.x;
  if (ln >= n_lanes) return;
  const float* zr = z + (size_t)ln * d;
  double acc = 0.0;
  {
#pragma clang fp contract(off)
    for (int i = 0; i < d; ++i) acc = acc + (double)zr[i] * (double)zr[i];
  }
  const double tn = sqrt(acc);
  rate[ln] = 0.02f / (1.0f + (float)fmin(tn, (double)FLT_MAX));
}

// up[i,q] += rate_l * clamp(z_l[i] - a_l[i], -4, 4) * act_l[q] for lanes l in
// order, then the GEMM operand u_eff = up + slow in the weight type.
__global__ void hebbian_kernel(float* __restrict__ up, const float* __restrict__ slow,
                               void* __restrict__ u_eff, int ueff_bf16,
                               const float* __restrict__ z, const float* __restrict__ a,
                               const float* __restrict__ act, const float* __restrict__ rate,
                               int n_lanes, int d, int r) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= d * r) return;
  const int i = e / r, q = e % r;
  float u = up[e];
  for (int ln = 0; ln < n_lanes; ++ln) {
    const float err = fminf(fmaxf(z[(size_t)ln * d + i] - a[(size_t)ln * d + i], -4.0f), 4.0f);
    u = __fadd_rn(u, __fmul_rn(__fmul_rn(rate[ln], err), act[(size_t)ln * r + q]));
  }
  up[e] = u;
  const float eff = u + slow[e];
  if (ueff_bf16) {
    uint32_t b = __float_as_uint(eff);
    b += 0x7FFFu + ((b >> 16) & 1u);
    static_cast<uint16_t*>(u_eff)[e] = (uint16_t)(b >> 16);
  } else {
    static_cast<float*>(u_eff)[e] = eff;
  }
}

// Protected writes of one block's bank for all lanes, in lane order.  The
// accept/defend decisions depend only on the bank's counters, confidences and
// ages, so thread 0 makes them sequentially; the slot contents are then
// copied in parallel, each slot from the last lane in order that wrote it.
__global__ __launch_bounds__(256) void bank_write_kernel(
    float* __restrict__ keys, float* __restrict__ norm_sq, float* __restrict__ values,
    void* __restrict__ values_t, int vt_bf16, float* __restrict__ conf,
    unsigned long long* __restrict__ last_seen, int* __restrict__ meta,
    const unsigned long long* __restrict__ step, const float* __restrict__ q,
    const float* __restrict__ z, const float* __restrict__ surprise, int n_lanes, int C, int dk,
    int d) {
  extern __shared__ int writer[];  // [C]: last lane that wrote the slot this step, or -1
  const int tid = threadIdx.x;
  for (int c = tid; c < C; c += blockDim.x) writer[c] = -1;
  __syncthreads();
  if (tid == 0) {
    const unsigned long long cur = step[0] + 1;
    int count = meta[0], head = meta[1];
    for (int ln = 0; ln < n_lanes; ++ln) {
      const float sp = surprise[ln];
      if (!(sp > 3.5f)) continue;
      int idx;
      if (count < C) {  // insert() into a free slot
        idx = count++;
      } else {
        idx = head;
        // RateLimiterGate::apply_refractory_overwrite (src/defense.rs:45-67).
        const unsigned long long last = last_seen[idx];
        const float dt = (float)(cur > last ? cur - last : 0ull);
        const float lin = 1.0f - expf(-dt / 60.0f);
        const float gain = fmaxf(lin * lin, 0.005f);
        const float damage = 0.08f * sp * gain;
        if (conf[idx] > damage) {
          conf[idx] -= damage;
          last_seen[idx] = cur;
          continue;
        }
        head = (head + 1) % C;
      }
      conf[idx] = 1.0f;
      last_seen[idx] = cur;
      writer[idx] = ln;
    }
    meta[0] = count;
    meta[1] = head;
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
  for (int c = wave; c < C; c += nw) {
    const int ln = writer[c];
    if (ln < 0) continue;
    const float* kq = q + (size_t)ln * dk;
    const float* vz = z + (size_t)ln * d;
    for (int j = lane; j < dk; j += 64) keys[(size_t)c * dk + j] = kq[j];
    for (int j = lane; j < d; j += 64) {
      const float v = vz[j];
      values[(size_t)c * d + j] = v;
      if (vt_bf16) {
        uint32_t b = __float_as_uint(v);
        b += 0x7FFFu + ((b >> 16) & 1u);
        static_cast<uint16_t*>(values_t)[(size_t)j * C + c] = (uint16_t)(b >> 16);
      } else {
        static_cast<float*>(values_t)[(size_t)j * C + c] = v;
      }
    }
    if (lane == 0) {
      // squared_norm (src/memory.rs:181-192): sequential f64 sum.
      double acc = 0.0;
      {
#pragma clang fp contract(off)
        for (int j = 0; j < dk; ++j) acc = acc + (double)kq[j] * (double)kq[j];
      }
      float v = (float)acc;
      if (acc < 1.0 && v == 1.0f) v = __uint_as_float(0x3f7fffffu);
      norm_sq[c] = v;
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
    const bool vbf = M->dtype == PSSA_HIP_BF16;
    for (size_t l = 0; l < c.depth; ++l) {
      const DevBlock& B = M->blocks[l];
      const float* tq = L->tap_q.as<float>() + l * n * k;
      const float* tz = L->tap_z.as<float>() + l * n * d;
      const float* ta = L->tap_a.as<float>() + l * n * d;
      const float* tact = L->tap_act.as<float>() + l * n * r;
      bank_write_kernel<<<1, 256, (size_t)C * sizeof(int), st>>>(
          B.keys.as<float>(), B.norm_sq.as<float>(), B.values.as<float>(), B.values_t.p, vbf ? 1 : 0,
          B.conf.as<float>(), B.last_seen.as<unsigned long long>(), B.meta.as<int>(),
          M->step.as<unsigned long long>(), tq, tz, L->surprise.as<float>(), (int)n, C, k, d);
      PSSA_LAUNCH_CHECK("bank_write");
      hebbian_rate_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(tz, d, (int)n, L->hebb_rate.as<float>());
      PSSA_LAUNCH_CHECK("hebbian_rate");
      hebbian_kernel<<<(unsigned)((d * r + 255) / 256), 256, 0, st>>>(
          B.u_fast.as<float>(), B.u_slow.as<float>(), B.u_eff.p, vbf ? 1 : 0, tz, ta, tact,
          L->hebb_rate.as<float>(), (int)n, d, r);
      PSSA_LAUNCH_CHECK("hebbian");
    }
    advance_kernel<<<1, 64, 0, st>>>(M->step.as<unsigned long long>(), L->gen_pos.as<int>());
  } else {
    advance_pos_kernel<<<1, 64, 0, st>>>(L->gen_pos.as<int>());
  }
  PSSA_LAUNCH_CHECK("advance");
  return Status::Ok();
}

}  // namespace pssa

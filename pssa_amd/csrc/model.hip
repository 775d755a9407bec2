// PSSA layer prefill on gfx950: the reference's per-token forward
// (forward_continuous_inference, src/pssa.rs:1072-1209) evaluated for all
// tokens of all lanes at once, stage by stage, following the batched stage
// decomposition of src/gpu_batch.rs:445-1255:
//
//   norm        x = RMSNorm(h)                                  (one wave/row)
//   gemm_in     [delta|B|C|q_x|gate|ad] = x W_in^T, epilogue softplus/sigmoid/SiLU
//   ssm         fused diagonal scan -> y, carry
//   gemm_qh     q_euc = y W_qh^T + q_x
//   retrieve    project, f64 Poincare distances, softmax weights
//   gemm_read   m_val = weights values
//   gemm_proj   z_raw = y/sqrt(s) + gate * (m_val W_proj^T) + U_eff act
//   gemm_mlp1   a = SiLU(z_raw W1^T)
//   gemm_mlp2   h = z_raw + a W2^T   (layer 0)  /  h += (z_raw + a W2^T)/sqrt(depth)
//   head        logits = h_last U^T / sqrt(d)   (last token of each lane only)
#include "model.h"

#include <algorithm>
#include <cmath>

#include "gemm.h"
#include "memory.h"
#include "ssm.h"

namespace pssa {

const char* const kStageNames[ST_COUNT] = {"embed",     "rmsnorm",   "gemm_in",   "ssm_scan",
                                           "ssm_aux",   "gemm_qh",   "retrieve",  "gemm_read",
                                           "gemm_proj", "gemm_mlp1", "gemm_mlp2", "head"};

__global__ void embed_kernel(const uint32_t* __restrict__ ids, const float* __restrict__ embed,
                             float* __restrict__ X, int d, size_t rows) {
  const size_t r = blockIdx.x;
  if (r >= rows) return;
  const float* src = embed + (size_t)ids[r] * d;
  for (int i = threadIdx.x; i < d; i += blockDim.x) X[r * d + i] = src[i];
}

// Affine RMSNorm with epsilon inside the root (src/pssa.rs:1080-1086).  One
// wave per row.
__device__ __forceinline__ uint16_t bf16_of(float f) { return bf16_bits_dev(f); }

constexpr int RMS_REG = 16;  // rows of up to 1024 columns are held in registers

// Also clears row r of Z (may be null), the readout the scan accumulates into.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ X,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta,
                                                      float* __restrict__ XN,
                                                      uint16_t* __restrict__ XNh, float* __restrict__ Z,
                                                      int d, size_t rows) {
  const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  if (Z)
    for (int i = lane; i < d; i += 64) Z[r * d + i] = 0.0f;
  const float* x = X + r * d;
  if (d % 4 == 0 && d <= 256 * RMS_V4) {  // 16-byte pieces, the decode input product's order
    float4 xv[1][RMS_V4];
    rms_load_v4(x, d, lane, xv[0]);
    float inv1[1];
    rms_inv_v4<1>(xv, d, inv1);
    const float inv = inv1[0];
#pragma unroll
    for (int k = 0; k < RMS_V4; ++k) {
      const int i = 4 * lane + 256 * k;
      if (i < d) {
        const float4 g = *reinterpret_cast<const float4*>(gamma + i);
        const float4 b = *reinterpret_cast<const float4*>(beta + i);
        const float4 x4 = xv[0][k];
        const float4 v = make_float4(rms_apply(x4.x, inv, g.x, b.x), rms_apply(x4.y, inv, g.y, b.y),
                                     rms_apply(x4.z, inv, g.z, b.z), rms_apply(x4.w, inv, g.w, b.w));
        *reinterpret_cast<float4*>(XN + r * d + i) = v;
        if (XNh)
          *reinterpret_cast<uint2*>(XNh + r * d + i) = make_uint2(bf16x2_bits(v.x, v.y), bf16x2_bits(v.z, v.w));
      }
    }
    return;
  }
  if (d <= 64 * RMS_REG) {  // the row stays in registers; all loads issue at once
    float xv[RMS_REG];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < RMS_REG; ++k) {
      const int i = lane + 64 * k;
      xv[k] = i < d ? x[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < RMS_REG; ++k) ss = fmaf(xv[k], xv[k], ss);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = 1.0f / sqrtf(ss / (float)d + 1e-5f);
#pragma unroll
    for (int k = 0; k < RMS_REG; ++k) {
      const int i = lane + 64 * k;
      if (i < d) {
        const float v = rms_apply(xv[k], inv, gamma[i], beta[i]);
        XN[r * d + i] = v;
        if (XNh) XNh[r * d + i] = bf16_of(v);
      }
    }
    return;
  }
  float ss = 0.0f;
  for (int i = lane; i < d; i += 64) ss = fmaf(x[i], x[i], ss);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float inv = 1.0f / sqrtf(ss / (float)d + 1e-5f);
  for (int i = lane; i < d; i += 64) {
    const float v = rms_apply(x[i], inv, gamma[i], beta[i]);
    XN[r * d + i] = v;
    if (XNh) XNh[r * d + i] = bf16_of(v);
  }
}

__global__ void fill_zero_kernel(float* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}
__global__ void mul_kernel(const float* __restrict__ a, const float* __restrict__ b,
                           float* __restrict__ out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] * b[i];
}
__global__ void softplus_kernel(float* __restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float x = p[i];
    p[i] = x > 20.0f ? x : log1pf(expf(x));
  }
}
__global__ void sigmoid_kernel(float* __restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 1.0f / (1.0f + expf(-p[i]));
}
__global__ void check_ids_kernel(const uint32_t* __restrict__ ids, size_t n, uint32_t vocab,
                                 int* __restrict__ bad) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n && ids[i] >= vocab) atomicOr(bad, 1);
}

__global__ void copy_cols_kernel(const float* __restrict__ in, int ld_in, float* __restrict__ out,
                                 int ld_out, size_t rows, int cols) {
  const size_t n = rows * (size_t)cols;
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x)
    out[(e / cols) * ld_out + e % cols] = in[(e / cols) * ld_in + e % cols];
}

Status launch_copy_cols(hipStream_t stream, const float* in, int ld_in, float* out, int ld_out,
                        size_t rows, int cols) {
  const size_t n = rows * (size_t)cols;
  if (!n) return Status::Ok();
  size_t g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  copy_cols_kernel<<<(unsigned)g, 256, 0, stream>>>(in, ld_in, out, ld_out, rows, cols);
  PSSA_LAUNCH_CHECK("copy_cols");
  return Status::Ok();
}

static unsigned grid1d(size_t n, unsigned cap = 65535u * 4) {
  size_t g = (n + 255) / 256;
  if (g == 0) g = 1;
  return (unsigned)(g > cap ? cap : g);
}

Status launch_fill_zero(hipStream_t stream, float* p, size_t n) {
  if (!n) return Status::Ok();
  fill_zero_kernel<<<grid1d(n, 8192), 256, 0, stream>>>(p, n);
  PSSA_LAUNCH_CHECK("fill_zero");
  return Status::Ok();
}
Status launch_mul(hipStream_t stream, const float* a, const float* b, float* out, size_t n) {
  if (!n) return Status::Ok();
  mul_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(a, b, out, n);
  PSSA_LAUNCH_CHECK("mul");
  return Status::Ok();
}
Status launch_softplus(hipStream_t stream, float* p, size_t n) {
  if (!n) return Status::Ok();
  softplus_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(p, n);
  PSSA_LAUNCH_CHECK("softplus");
  return Status::Ok();
}
Status launch_sigmoid(hipStream_t stream, float* p, size_t n) {
  if (!n) return Status::Ok();
  sigmoid_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(p, n);
  PSSA_LAUNCH_CHECK("sigmoid");
  return Status::Ok();
}
Status launch_check_ids(hipStream_t stream, const uint32_t* ids, size_t n, uint32_t vocab, int* bad) {
  if (!n) return Status::Ok();
  check_ids_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(ids, n, vocab, bad);
  PSSA_LAUNCH_CHECK("check_ids");
  return Status::Ok();
}

namespace {

struct Timer {
  pssa_hip_lanes* L;
  hipStream_t s;
  size_t next = 0;
  Status mark(int stage) {
    if (!L || !L->timing) return Status::Ok();
    if (next == L->events.size()) {
      hipEvent_t e;
      PSSA_HIP_TRY(hipEventCreate(&e));
      L->events.push_back(e);
      L->event_stage.push_back(0);
    }
    L->event_stage[next] = stage;
    PSSA_HIP_TRY(hipEventRecord(L->events[next], s));
    ++next;
    return Status::Ok();
  }
  // Closes the last interval and folds all intervals into per-stage totals.
  Status finish() {
    if (!L || !L->timing) return Status::Ok();
    PSSA_RETURN_IF(mark(-1));
    PSSA_HIP_TRY(hipEventSynchronize(L->events[next - 1]));
    L->stage_ms.fill(0.0f);
    L->stage_calls.fill(0);
    for (size_t i = 0; i + 1 < next; ++i) {
      float ms = 0.0f;
      PSSA_HIP_TRY(hipEventElapsedTime(&ms, L->events[i], L->events[i + 1]));
      const int st = L->event_stage[i];
      if (st >= 0) {
        L->stage_ms[st] += ms;
        L->stage_calls[st] += 1;
      }
    }
    return Status::Ok();
  }
};

}  // namespace

// Hybrid write gate of each row: the mean of its memory-injection gate
// activations g[row, 0..d), summed left to right in f32 as
// src/pssa.rs:3724 does (one thread per row).
__global__ void gate_mean_kernel(const float* __restrict__ g, int ld, int d, int rows, float* __restrict__ out) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* x = g + (size_t)r * ld;
  float s = 0.0f;
  for (int i = 0; i < d; ++i) s += x[i];
  out[r] = s / (float)d;
}

// bump_hybrid_ages (src/memory.rs:501-507) `times` times: every live slot's
// age grows by `times`, saturating at 2^64 - 1.
__global__ void hybrid_bump_kernel(unsigned long long* __restrict__ age, const int* __restrict__ meta, int C,
                                   unsigned long long times) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= C || s >= meta[0]) return;
  const unsigned long long a = age[s];
  age[s] = a > ~0ull - times ? ~0ull : a + times;
}

// Cross entropy of one scaled logit row (stage_logits_loss without
// distillation, src/gpu_batch.rs:1211-1247, 1170): loss = (max - l_target) +
// ln(sum_i exp(l_i - max)), stored at the row's packed token index.  A NaN
// logit never becomes the maximum and makes the sum NaN, as in the reference.
// Rows of up to 256 * 4 * CE_V4 aligned logits stay in registers between the
// two reductions (one HBM read); exp is the hardware exp2 of (l - max) log2 e.
constexpr int CE_V4 = 16;

__device__ __forceinline__ float ce_block_max(float v, float* red) {
  for (int o = 32; o >= 1; o >>= 1) {
    const float other = __shfl_xor(v, o, 64);
    v = other > v ? other : v;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < 4; ++w) v = red[w] > v ? red[w] : v;
  return v;
}

__global__ __launch_bounds__(256) void token_ce_kernel(const float* __restrict__ logits, int V,
                                                       const uint32_t* __restrict__ targets,
                                                       const uint32_t* __restrict__ index,
                                                       float* __restrict__ loss) {
  __shared__ float red[8];
  const float* l = logits + (size_t)blockIdx.x * V;
  const int tid = threadIdx.x;
  constexpr float kLog2e = 1.44269504088896341f;
  float sum = 0.0f, mx;
  if (V % 4 == 0 && V <= 256 * 4 * CE_V4) {
    float4 v[CE_V4];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < CE_V4; ++k) {
      const int i = 4 * (tid + 256 * k);
      v[k] = i < V ? *reinterpret_cast<const float4*>(l + i) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      m = v[k].x > m ? v[k].x : m;
      m = v[k].y > m ? v[k].y : m;
      m = v[k].z > m ? v[k].z : m;
      m = v[k].w > m ? v[k].w : m;
    }
    mx = ce_block_max(m, red);
#pragma unroll
    for (int k = 0; k < CE_V4; ++k)
      if (4 * (tid + 256 * k) < V)
        sum += (__builtin_amdgcn_exp2f((v[k].x - mx) * kLog2e) + __builtin_amdgcn_exp2f((v[k].y - mx) * kLog2e)) +
               (__builtin_amdgcn_exp2f((v[k].z - mx) * kLog2e) + __builtin_amdgcn_exp2f((v[k].w - mx) * kLog2e));
  } else {
    float m = -INFINITY;
    for (int i = tid; i < V; i += 256) m = l[i] > m ? l[i] : m;
    mx = ce_block_max(m, red);
    for (int i = tid; i < V; i += 256) sum += __builtin_amdgcn_exp2f((l[i] - mx) * kLog2e);
  }
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = sum;
  __syncthreads();
  if (tid == 0) {
    const float total = (red[4] + red[5]) + (red[6] + red[7]);
    loss[index[blockIdx.x]] = (mx - l[targets[blockIdx.x]]) + logf(total);
  }
}

// x = in + scale * x: a looped layer after the first returns its input plus
// the scaled features its passes left (src/pssa.rs:2370-2372).
__global__ void loop_combine_kernel(float* __restrict__ x, const float* __restrict__ in, float scale, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
#pragma clang fp contract(off)
    x[i] = in[i] + scale * x[i];
  }
}

// Prefill of lanes lane0 .. lane0+n_lanes-1 on stream `st`, enqueued in
// pieces (embed, each layer, head) so that concurrent views can be enqueued
// layer by layer.  Every buffer pointer is offset to the view's rows, so
// disjoint views can run concurrently.  `first_in_done` (may be null) is
// recorded once layer 0's input projection has been issued.
class PrefillView {
 public:
  PrefillView(pssa_hip_lanes* L, hipStream_t st, size_t lane0, size_t n_lanes, size_t T, bool taps, bool timing,
              hipEvent_t first_in_done, float* y_part, const TrainRows* tr, bool concurrent, size_t tap_rows = 0)
      : L_(L), M_(L->model), c_(L->model->cfg), st_(st), n_lanes_(n_lanes), T_(T), taps_(taps),
        first_in_done_(first_in_done), y_part_(y_part), tr_(tr), concurrent_(concurrent),
        tm_{timing ? L : nullptr, st} {
    d_ = (int)c_.d_latent;
    s_ = (int)c_.d_state;
    k_ = (int)c_.d_mem_key;
    C_ = (int)c_.mem_capacity;
    r_ = (int)c_.adapter_rank;
    V_ = (int)c_.d_vocab;
    n_in_ = (int)M_->n_in;
    rows_ = n_lanes * T;
    const size_t row0 = lane0 * T;
    m_ = (int)rows_;
    dt_ = M_->dtype;
    bf16_ = dt_ == PSSA_HIP_BF16;
    const size_t es = bf16_ ? 2 : 4;
    const int d = d_, k = k_, C = C_, V = V_;
    X_ = L->X.as<float>() + row0 * d;
    XN_ = L->XN.as<float>() + row0 * d;
    P_ = L->P.as<float>() + row0 * n_in_;
    Y_ = L->Y.as<float>() + row0 * d;
    Q_ = L->Q.as<float>() + row0 * k;
    Zr_ = L->Zraw.as<float>() + row0 * d;
    // GEMM operands in the model's operand type (aliases of the fp32 buffers
    // in an fp32 model).
    XNh16_ = bf16_ ? L->XNh.as<uint16_t>() + row0 * d : nullptr;
    XNh_ = bf16_ ? (void*)XNh16_ : (void*)XN_;
    Yh_ = bf16_ ? (void*)(L->Yh.as<uint16_t>() + row0 * d) : (void*)Y_;
    Zrh_ = bf16_ ? (void*)(L->Zrawh.as<uint16_t>() + row0 * d) : (void*)Zr_;
    Wm_ = static_cast<char*>(L->Wm.p) + row0 * C * es;
    Mv_ = static_cast<char*>(L->Mval.p) + row0 * d * es;
    H1_ = static_cast<char*>(L->H1.p) + row0 * 2 * d * es;
    ids_ = (tr ? tr->ids : L->ids.as<uint32_t>()) + row0;
    carry_ = (tr ? tr->carry : L->carry.as<float>()) + lane0 * c_.depth * L->loops * (size_t)d * s_;
    logits_ = L->logits.as<float>() + lane0 * (size_t)V;
    row0_ = row0;
    // Taps are [layer][all rows of the step]; a lane group writes its rows.
    tap_rows_ = tap_rows ? tap_rows : rows_;
  }

  Status embed() {
    PSSA_RETURN_IF(tm_.mark(ST_EMBED));
    embed_kernel<<<(unsigned)rows_, 256, 0, st_>>>(ids_, M_->embed.as<float>(), X_, d_, rows_);
    PSSA_LAUNCH_CHECK("embed");
    return Status::Ok();
  }

  // One layer: its loops passes over the view's rows (set_loops,
  // src/pssa.rs:2338-2373).  With one loop the pass is the whole block step
  // (layer 0's output replaces the embedding, deeper ones add
  // output / sqrt(depth)).  With more, every pass adds output / loops to the
  // rows it read, and a layer after the first then returns
  // input + output_sum_rows / sqrt(depth), its input kept in Xin.
  Status layer(size_t l) {
    const size_t loops = L_->loops;
    if (loops == 1) return pass(l, 0);
    const size_t n = rows_ * (size_t)d_;
    float* xin = L_->Xin.as<float>() + row0_ * d_;
    if (l > 0) PSSA_HIP_TRY(hipMemcpyAsync(xin, X_, n * 4, hipMemcpyDeviceToDevice, st_));
    for (size_t lp = 0; lp < loops; ++lp) PSSA_RETURN_IF(pass(l, lp));
    if (l > 0) {
      loop_combine_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 65536), 256, 0, st_>>>(
          X_, xin, 1.0f / sqrtf((float)c_.depth), n);
      PSSA_LAUNCH_CHECK("loop_combine");
    }
    return Status::Ok();
  }

  Status pass(size_t l, size_t lp) {
    const DevBlock& B = M_->blocks[l];
    const int d = d_, s = s_, k = k_, C = C_, r = r_, n_in = n_in_, m = m_, dt = dt_;
    const size_t rows = rows_, T = T_;
    const bool bf16 = bf16_, taps = taps_;
    hipStream_t st = st_;
    // Column offsets inside the fused projection output P.
    const int o_b = d, o_c = d + s, o_qx = d + 2 * s, o_gate = d + 2 * s + k, o_act = 2 * d + 2 * s + k;
    const bool step_y = ssm_step_writes_y((int)T, s);
    // In a bf16 decode step the input product normalises its rows itself.
    const bool fold_norm = bf16 && step_y && gemm_norm_fits(d);
    PSSA_RETURN_IF(tm_.mark(ST_NORM));
    if (!fold_norm) {
      rmsnorm_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(
          X_, B.gamma.as<float>(), B.beta.as<float>(), XN_, XNh16_,
          ssm_needs_zeroed_y(s) && !step_y ? Y_ : nullptr, d, rows);
      PSSA_LAUNCH_CHECK("rmsnorm");
    }

    // [delta | B | C | q_x | gate | adapter act] = x W_in^T with softplus,
    // sigmoid and SiLU applied per column segment.
    PSSA_RETURN_IF(tm_.mark(ST_GEMM_IN));
    EpiParams e_in;
    e_in.kind = EPI_SEGMENTS;
    e_in.seg[0] = d;
    e_in.seg[1] = o_gate;
    e_in.seg[2] = o_act;
    e_in.seg[3] = n_in;
    e_in.out32 = P_;
    e_in.ld32 = n_in;
    if (taps) {  // the adapter activations of this step, for the Hebbian update
      e_in.kind = EPI_SEGMENTS_TAP;
      e_in.tap = L_->tap_act.as<float>() + (l * tap_rows_ + row0_) * r;
      e_in.ld_tap = r;
    }
    if (fold_norm)
      PSSA_RETURN_IF(launch_gemm_norm(st, X_, B.gamma.as<float>(), B.beta.as<float>(), XN_,
                                      static_cast<const uint16_t*>(B.w_in.p), d, m, n_in, d, e_in));
    else
      PSSA_RETURN_IF(launch_gemm(st, dt, XNh_, d, B.w_in.p, d, m, n_in, d, e_in));
    if (l == 0 && first_in_done_) PSSA_HIP_TRY(hipEventRecord(first_in_done_, st));
    if (taps && B.hybrid) {  // the write gate of a gated protected insert
      gate_mean_kernel<<<(unsigned)((rows + 255) / 256), 256, 0, st>>>(P_ + o_gate, n_in, d, (int)rows,
                                                                       L_->tap_gmean.as<float>() + l * tap_rows_ + row0_);
      PSSA_LAUNCH_CHECK("gate_mean");
    }

    PSSA_RETURN_IF(tm_.mark(ST_SSM));
    SsmArgs sa;
    sa.delta = P_;
    sa.ld_delta = n_in;
    sa.bproj = P_ + o_b;
    sa.ld_b = n_in;
    sa.cproj = P_ + o_c;
    sa.ld_c = n_in;
    sa.xn = XN_;
    sa.ld_x = d;
    sa.rates2 = B.rates2.as<float>();
    sa.carry = carry_ + (l * L_->loops + lp) * (size_t)d * s;
    sa.carry_stride = (long)(c_.depth * L_->loops * (size_t)d * s);
    sa.y = Y_;
    sa.ld_y = d;
    sa.T = (int)T;
    sa.d = d;
    sa.s = s;
    sa.lanes = (int)n_lanes_;
    sa.y_part = y_part_;
    sa.concurrent = concurrent_ ? 1 : 0;
    if (bf16 && step_y) {
      sa.y16 = static_cast<uint16_t*>(Yh_);
      sa.ld_y16 = d;
    }
    PSSA_RETURN_IF(launch_ssm_scan(st, sa));
    RetrieveArgs ra;
    ra.q = Q_;
    ra.ld_q = k;
    ra.project = 1;
    ra.keys = B.keys.as<float>();
    ra.norm_sq = B.norm_sq.as<float>();
    ra.n = m;
    ra.dk = k;
    ra.dv = d;
    ra.capacity = C;
    ra.count = C;  // upper bound; the live count is read on the device
    ra.count_dev = B.meta.as<int>();
    ra.tau = c_.tau_mem;
    ra.top_k = B.top_k;
    if (taps) ra.q_pnc = L_->tap_q.as<float>() + (l * tap_rows_ + row0_) * k;
    if (B.hybrid) {  // token t reads with the ages bumped t + 1 times
      ra.hgate = B.hgate.as<float>();
      ra.hage = B.hage.as<unsigned long long>();
      ra.log_lam = std::log((double)B.lam);
      ra.age_T = (int)T;
    }
    if (bf16)
      ra.weights16 = static_cast<uint16_t*>(Wm_);
    else
      ra.weights = static_cast<float*>(Wm_);
    // In a bf16 decode step the soft read forms q itself from y's bf16 copy
    // (the same products and sum as the GEMM below, one launch fewer).
    bool fused_q = false;
    if (bf16 && step_y) {
      ra.qa = static_cast<const uint16_t*>(Yh_);
      ra.ld_qa = d;
      ra.qw = static_cast<const uint16_t*>(B.w_qh.p);
      ra.qk = d;
      ra.qaux = P_ + o_qx;
      ra.ld_qaux = n_in;
      fused_q = retrieve_fuses_query(ra);
      if (!fused_q) {
        ra.qa = nullptr;
        ra.qw = nullptr;
        ra.qaux = nullptr;
      }
    }
    PSSA_RETURN_IF(tm_.mark(ST_GEMM_QH));
    // q_euc = y W_qh^T + q_x.  In a bf16 model y enters the product rounded
    // to bf16: the single-step scan writes that copy itself, otherwise the
    // product rounds the fp32 readout as it loads it.
    if (!fused_q) {
      EpiParams e_q;
      e_q.kind = EPI_ADD_AUX;
      e_q.aux = P_ + o_qx;
      e_q.ld_aux = n_in;
      e_q.out32 = Q_;
      e_q.ld32 = k;
      if (bf16 && !step_y && d % 16 == 0)
        PSSA_RETURN_IF(launch_gemm_f32a(st, Y_, d, static_cast<const uint16_t*>(B.w_qh.p), d, m, k, d, e_q));
      else {
        if (bf16 && !step_y) PSSA_RETURN_IF(launch_to_bf16(st, Y_, d, static_cast<uint16_t*>(Yh_), d, rows, d));
        PSSA_RETURN_IF(launch_gemm(st, dt, Yh_, d, B.w_qh.p, d, m, k, d, e_q));
      }
    }
    PSSA_RETURN_IF(tm_.mark(ST_RETRIEVE));
    PSSA_RETURN_IF(launch_retrieve(st, ra));

    // m_val = weights values (soft read readout).
    PSSA_RETURN_IF(tm_.mark(ST_GEMM_READ));
    {
      // Slots past the live count carry zero weight, so the product runs
      // over the whole capacity.
      EpiParams e_m;
      e_m.out16 = Mv_;
      e_m.ld16 = d;
      PSSA_RETURN_IF(launch_gemm(st, dt, Wm_, C, B.values_t.p, C, m, d, C, e_m));
    }

    // z_raw = y/sqrt(s) + gate * (m_val W_proj^T) + U_eff act.
    PSSA_RETURN_IF(tm_.mark(ST_GEMM_PROJ));
    EpiParams e_z;
    e_z.kind = EPI_ZRAW;
    e_z.y = Y_;
    e_z.ld_y = d;
    e_z.g = P_ + o_gate;
    e_z.ld_g = n_in;
    e_z.act = P_ + o_act;
    e_z.ld_act = n_in;
    e_z.U = B.u_eff.p;
    e_z.rank = r;
    e_z.scale = 1.0f / sqrtf((float)s);
    e_z.out32 = Zr_;
    e_z.ld32 = d;
    if (taps) {
      e_z.tap = L_->tap_a.as<float>() + (l * tap_rows_ + row0_) * d;
      e_z.ld_tap = d;
    }
    if (bf16) {
      e_z.out16 = Zrh_;
      e_z.ld16 = d;
    }
    PSSA_RETURN_IF(launch_gemm(st, dt, Mv_, d, B.w_proj.p, d, m, d, d, e_z));

    // a = SiLU(z_raw W1^T).
    PSSA_RETURN_IF(tm_.mark(ST_GEMM_MLP1));
    EpiParams e_s;
    e_s.kind = EPI_SILU;
    e_s.out16 = H1_;
    e_s.ld16 = 2 * d;
    PSSA_RETURN_IF(launch_gemm(st, dt, Zrh_, d, B.mlp_w1.p, d, m, 2 * d, d, e_s));

    // h = z_raw + a W2^T (layer 0), h += (z_raw + a W2^T) / sqrt(depth).
    PSSA_RETURN_IF(tm_.mark(ST_GEMM_MLP2));
    EpiParams e_r;
    e_r.kind = EPI_RESIDUAL;
    e_r.aux = Zr_;
    e_r.ld_aux = d;
    e_r.first = l == 0 && L_->loops == 1 ? 1 : 0;
    e_r.scale = L_->loops == 1 ? 1.0f / sqrtf((float)c_.depth) : 1.0f / (float)L_->loops;
    e_r.out32 = X_;
    e_r.ld32 = d;
    if (taps) {
      e_r.tap = L_->tap_z.as<float>() + (l * tap_rows_ + row0_) * d;
      e_r.ld_tap = d;
    }
    return launch_gemm(st, dt, H1_, 2 * d, B.mlp_w2.p, 2 * d, m, d, 2 * d, e_r);
  }

  Status head() {
    const int d = d_, V = V_, m = m_, dt = dt_;
    const size_t rows = rows_, T = T_;
    hipStream_t st = st_;
    const float logit_scale = 1.0f / sqrtf((float)d);
    PSSA_RETURN_IF(tm_.mark(ST_HEAD));
    if (tr_ && tr_->logits) {
      // Every row: scaled logits, then its cross-entropy loss.
      const void* hin = X_;
      if (bf16_) {
        PSSA_RETURN_IF(launch_to_bf16(st, X_, d, XNh16_, d, rows, d));
        hin = XNh16_;
      }
      EpiParams e_h;
      e_h.kind = EPI_SCALE;
      e_h.scale = logit_scale;
      e_h.out32 = tr_->logits + row0_ * (size_t)V;
      e_h.ld32 = V;
      PSSA_RETURN_IF(launch_gemm(st, dt, hin, d, M_->unembed.p, d, m, V, d, e_h));
      token_ce_kernel<<<(unsigned)rows, 256, 0, st>>>(tr_->logits + row0_ * (size_t)V, V, tr_->targets + row0_,
                                                     tr_->index + row0_, tr_->loss);
      PSSA_LAUNCH_CHECK("token_ce");
      return tm_.finish();
    }
    // Head on the last token of every lane.
    const float* xlast = X_ + (T - 1) * (size_t)d;
    const void* hin = xlast;
    int ld_h = (int)(T * d);
    if (bf16_) {
      PSSA_RETURN_IF(launch_to_bf16(st, xlast, (int)(T * d), XNh16_, d, n_lanes_, d));
      hin = XNh16_;
      ld_h = d;
    }
    EpiParams e_h;
    e_h.kind = EPI_SCALE;
    e_h.scale = logit_scale;
    e_h.out32 = logits_;
    e_h.ld32 = V;
    PSSA_RETURN_IF(launch_gemm(st, dt, hin, ld_h, M_->unembed.p, d, (int)n_lanes_, V, d, e_h));
    return tm_.finish();
  }

 private:
  pssa_hip_lanes* L_;
  const pssa_hip_model* M_;
  const pssa_hip_config& c_;
  hipStream_t st_;
  size_t n_lanes_, T_;
  bool taps_;
  hipEvent_t first_in_done_;
  float* y_part_;
  const TrainRows* tr_;
  bool concurrent_;
  Timer tm_;
  int d_ = 0, s_ = 0, k_ = 0, C_ = 0, r_ = 0, V_ = 0, n_in_ = 0, m_ = 0, dt_ = 0;
  bool bf16_ = false;
  size_t rows_ = 0, row0_ = 0, tap_rows_ = 0;
  float *X_ = nullptr, *XN_ = nullptr, *P_ = nullptr, *Y_ = nullptr, *Q_ = nullptr, *Zr_ = nullptr;
  uint16_t* XNh16_ = nullptr;
  void *XNh_ = nullptr, *Yh_ = nullptr, *Zrh_ = nullptr, *Wm_ = nullptr, *Mv_ = nullptr, *H1_ = nullptr;
  const uint32_t* ids_ = nullptr;
  float* carry_ = nullptr;
  float* logits_ = nullptr;
};

constexpr int kPrefillLaneGroups = 2;
static_assert(kPrefillLaneGroups <= pssa_hip_lanes::kMaxGroups, "one stream per lane group");

static Status prefill_groups(pssa_hip_lanes* L, size_t n_lanes, size_t T, bool taps, const TrainRows* tr);
static Status bump_hybrid_ages(pssa_hip_lanes* L, size_t T);

Status run_prefill_segment(pssa_hip_lanes* L, size_t n_lanes, size_t T, const TrainRows& rows,
                           const int* lane_map) {
  if (rows.logits) return Status::Invalid("prefill segment: the all-token head belongs to the training forward");
  PSSA_RETURN_IF(prefill_groups(L, n_lanes, T, false, &rows));
  PSSA_RETURN_IF(launch_hist_append(L, rows.ids, n_lanes, T, lane_map));
  return bump_hybrid_ages(L, T);
}

Status run_prefill(pssa_hip_lanes* L, size_t n_lanes, size_t T, bool taps, bool append) {
  PSSA_RETURN_IF(prefill_groups(L, n_lanes, T, taps, nullptr));
  if (append) PSSA_RETURN_IF(launch_hist_append(L, L->ids.as<uint32_t>(), n_lanes, T, nullptr));
  return bump_hybrid_ages(L, T);
}

// One wave per row: the row's last min(T, 64) ids go into its lane's ring.
__global__ __launch_bounds__(64) void hist_append_kernel(uint32_t* __restrict__ hist, int* __restrict__ hist_n,
                                                         int* __restrict__ hist_pos, const uint32_t* __restrict__ ids,
                                                         int T, const int* __restrict__ lane_map) {
  constexpr int H = pssa_hip_lanes::kHist;
  const int row = blockIdx.x, j = threadIdx.x;
  const int lane = lane_map ? lane_map[row] : row;
  const int take = T < H ? T : H;
  const int pos = hist_pos[lane];
  if (j < take) hist[(size_t)lane * H + (pos + j) % H] = ids[(size_t)row * T + (T - take) + j];
  __syncthreads();
  if (j == 0) {
    hist_pos[lane] = (pos + take) % H;
    const int n = hist_n[lane] + take;
    hist_n[lane] = n < H ? n : H;
  }
}

Status launch_hist_append(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t T, const int* lane_map) {
  hist_append_kernel<<<(unsigned)n_lanes, 64, 0, L->ctx->stream>>>(
      L->hist.as<uint32_t>(), L->hist_n.as<int>(), L->hist_pos.as<int>(), ids, (int)T, lane_map);
  PSSA_LAUNCH_CHECK("hist_append");
  return Status::Ok();
}

static Status bump_hybrid_ages(pssa_hip_lanes* L, size_t T) {
  // Every lane read each token with the ages bumped once more; store them.
  const pssa_hip_model* M = L->model;
  const int C = (int)M->cfg.mem_capacity;
  for (const DevBlock& B : M->blocks)
    if (B.hybrid) {
      hybrid_bump_kernel<<<(unsigned)((C + 255) / 256), 256, 0, L->ctx->stream>>>(
          B.hage.as<unsigned long long>(), B.meta.as<int>(), C, (unsigned long long)T);
      PSSA_LAUNCH_CHECK("hybrid_bump");
    }
  return Status::Ok();
}

Status run_train_segment(pssa_hip_lanes* L, size_t n_lanes, size_t T, const TrainRows& tr) {
  for (const DevBlock& B : L->model->blocks)
    if (B.hybrid) return Status::Invalid("hybrid read currently requires the CPU backend");
  return prefill_groups(L, n_lanes, T, false, &tr);
}

static Status prefill_groups(pssa_hip_lanes* L, size_t n_lanes, size_t T, bool taps, const TrainRows* tr) {
  const hipStream_t st = L->ctx->stream;
  if (L->loops > 1)
    for (const DevBlock& B : L->model->blocks)
      if (B.hybrid) return Status{PSSA_HIP_EUNSUPPORTED, "the hybrid read runs one loop here (set_loops 1)"};
  const pssa_hip_config& c = L->model->cfg;
  const int nz = ssm_state_blocks((int)c.d_state);
  float* ypart = L->Ypart.p ? L->Ypart.as<float>() : nullptr;
  // Lane groups on their own streams: the VALU-bound scan of one group runs
  // beside the MFMA-bound GEMMs of the others.  Group g starts once group
  // g-1's first input projection is issued, which keeps them a stage apart,
  // and the groups are enqueued layer by layer, interleaved, so that the
  // later groups' work is queued as early as the first group's.  Two groups
  // measure best at the 32-lane prefill (three and four run 2-3% slower:
  // their smaller scans leave the CUs less evenly loaded).
  // A decode step of many lanes runs lane groups the same way: one group's
  // HBM-bound carry update beside the other groups' chains of latency-bound
  // products, eagerly or as parallel branches of the captured step.  Three
  // groups measured best at 256 lanes (graph replay 1.84 ms per step with
  // one, 1.79 with two, 1.77 with three, 1.80 with four).  The step's groups
  // start together (no stagger: 1.77 -> 1.76 ms; with the products' raised
  // wave priority 1.74), and group sizes rounded to the update's four lanes
  // per workgroup measured the same.
#ifndef PSSA_DECODE_GROUPS
#define PSSA_DECODE_GROUPS 3
#endif
  const bool step_groups = PSSA_DECODE_GROUPS >= 2 && T == 1 && n_lanes >= 64 && !L->timing;
  const int G = (int)std::min<size_t>(step_groups ? PSSA_DECODE_GROUPS : kPrefillLaneGroups, n_lanes);
  if ((!taps && !L->timing && G >= 2 && T >= 64) || (step_groups && G >= 2)) {
    PSSA_HIP_TRY(hipEventRecord(L->ev_fork, st));
    std::vector<PrefillView> views;
    views.reserve(G);
    size_t lane0 = 0;
    for (int g = 0; g < G; ++g) {
      const size_t ng = n_lanes / G + ((size_t)g < n_lanes % G ? 1 : 0);
      const hipStream_t sg = g == 0 ? st : L->aux_stream[g - 1];
      float* yp = ypart ? ypart + (size_t)nz * lane0 * T * c.d_latent : nullptr;
      views.emplace_back(L, sg, lane0, ng, T, taps, false, g + 1 < G && !step_groups ? L->ev_first[g] : nullptr,
                         yp, tr, true, n_lanes * T);
      lane0 += ng;
    }
    for (int g = 0; g < G; ++g) {
      if (g > 0) {
        const hipStream_t sg = L->aux_stream[g - 1];
        PSSA_HIP_TRY(hipStreamWaitEvent(sg, L->ev_fork, 0));
        if (!step_groups) PSSA_HIP_TRY(hipStreamWaitEvent(sg, L->ev_first[g - 1], 0));
      }
      PSSA_RETURN_IF(views[g].embed());
      PSSA_RETURN_IF(views[g].layer(0));
    }
    for (size_t l = 1; l < c.depth; ++l)
      for (int g = 0; g < G; ++g) PSSA_RETURN_IF(views[g].layer(l));
    for (int g = 0; g < G; ++g) PSSA_RETURN_IF(views[g].head());
    for (int g = 1; g < G; ++g) {
      PSSA_HIP_TRY(hipEventRecord(L->ev_join[g - 1], L->aux_stream[g - 1]));
      PSSA_HIP_TRY(hipStreamWaitEvent(st, L->ev_join[g - 1], 0));
    }
    return Status::Ok();
  }
  PrefillView v(L, st, 0, n_lanes, T, taps, L->timing, nullptr, ypart, tr, false);
  PSSA_RETURN_IF(v.embed());
  for (size_t l = 0; l < c.depth; ++l) PSSA_RETURN_IF(v.layer(l));
  return v.head();
}

}  // namespace pssa

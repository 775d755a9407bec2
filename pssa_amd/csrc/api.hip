// C ABI of libpssa_hip (include/pssa_hip.h).  Validation happens before any
// allocation or launch; device failures after a launch are reported as
// PSSA_HIP_EDEVICE (fatal).
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <memory>

#include "gemm.h"
#include "memory.h"
#include "model.h"
#include "ssm.h"

namespace pssa {
Status launch_dense_scan(hipStream_t stream, const float* A, const float* B, const float* H0, float* H,
                         int batch, int L, int s, void* scratch, size_t scratch_bytes);
// Scratch the two-level schedule needs (0: the sequential kernels run).
size_t dense_scan_scratch_bytes(int batch, int L, int s);
Status init_dense_scan_attributes();
}

using pssa::DevBuf;
using pssa::Status;

namespace {

Status upload(DevBuf& dst, const void* src, size_t bytes, hipStream_t st) {
  PSSA_RETURN_IF(dst.alloc(bytes));
  if (bytes) PSSA_HIP_TRY(hipMemcpyAsync(dst.p, src, bytes, hipMemcpyHostToDevice, st));
  return Status::Ok();
}

Status download(void* dst, const DevBuf& src, size_t bytes, hipStream_t st) {
  if (bytes) PSSA_HIP_TRY(hipMemcpyAsync(dst, src.p, bytes, hipMemcpyDeviceToHost, st));
  return Status::Ok();
}

uint16_t bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Weight upload in the model's storage type.
Status upload_weight(DevBuf& dst, const float* src, size_t n, int dtype, hipStream_t st) {
  if (dtype == PSSA_HIP_F32) return upload(dst, src, n * 4, st);
  std::vector<uint16_t> tmp(n);
  for (size_t i = 0; i < n; ++i) tmp[i] = bf16_bits(src[i]);
  PSSA_RETURN_IF(upload(dst, tmp.data(), n * 2, st));
  PSSA_HIP_TRY(hipStreamSynchronize(st));  // tmp must outlive the copy
  return Status::Ok();
}

Status sync(pssa_hip_ctx* ctx) {
  PSSA_HIP_TRY(hipStreamSynchronize(ctx->stream));
  return Status::Ok();
}

Status need(bool cond, const char* msg) { return cond ? Status::Ok() : Status::Invalid(msg); }

Status check_ctx(pssa_hip_ctx* ctx) { return ctx ? Status::Ok() : Status::Invalid("null context"); }

Status check_config(const pssa_hip_config& c) {
  if (c.depth < 1 || c.depth > 32) return Status::Invalid("depth must be in 1..=32");
  if (!c.d_vocab || !c.d_latent || !c.d_state || !c.d_mem_key || !c.mem_capacity || !c.adapter_rank)
    return Status::Invalid("model dimensions and memory capacity must be positive");
  if (!(std::isfinite(c.tau_mem) && c.tau_mem > 0.0f))
    return Status::Invalid("tau_mem must be finite and positive");
  if (c.d_latent > 16384 || c.d_state > 4096 || c.d_mem_key > 4096 || c.mem_capacity > 8192 ||
      c.d_vocab > (1u << 24) || c.adapter_rank > 256)
    return Status::Invalid("model dimensions exceed the supported range");
  return Status::Ok();
}

float softplus_host(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Carries are [lanes, depth, d, s] at the ABI (h_persistent, src/pssa.rs) and
// [lanes, depth] matrices in the scan's channel-blocked layout on the device
// (pssa::carry_at).
Status carry_layout(pssa_hip_lanes* L, const float* in, float* out, bool to_device) {
  const pssa_hip_config& c = L->model->cfg;
  return pssa::launch_carry_convert(L->ctx->stream, in, out, L->lanes * c.depth * L->loops, (int)c.d_latent,
                                    (int)c.d_state, to_device);
}

// Clamps every slot of a block's bank values to `cap` (set_value_cap,
// src/memory.rs:121-134) and rebuilds the transposed readout operand.
// Every slot's value of each given block clamped to `cap` (clamp_value,
// src/memory.rs:150-170), committed only when no slot of any of them has a
// non-finite norm: such a slot fails the call, as the reference's assertion
// (src/memory.rs:151-152) does, and leaves every bank unchanged.
Status cap_bank_values(pssa_hip_model* M, const std::vector<pssa::DevBlock*>& blocks, float cap) {
  const hipStream_t st = M->ctx->stream;
  const int C = (int)M->cfg.mem_capacity, d = (int)M->cfg.d_latent;
  const size_t bytes = (size_t)C * d * 4;
  pssa::ValueCaps caps{};
  caps.c[0] = cap;
  std::vector<DevBuf> capped(blocks.size());
  DevBuf tmp, bad;
  PSSA_RETURN_IF(bad.alloc(4));
  PSSA_RETURN_IF(pssa::launch_fill_zero(st, bad.as<float>(), 1));
  for (size_t i = 0; i < blocks.size(); ++i) {
    PSSA_RETURN_IF(capped[i].alloc(bytes));
    PSSA_RETURN_IF(pssa::launch_clamp_rows(st, blocks[i]->values.as<float>(), capped[i].as<float>(), C, d,
                                           (size_t)d, caps, C, bad.as<int>()));
  }
  int flag = 0;
  PSSA_RETURN_IF(download(&flag, bad, 4, st));
  PSSA_RETURN_IF(sync(M->ctx));
  if (flag) return Status::Invalid("capped memory value must be finite");
  if (M->dtype == PSSA_HIP_BF16) PSSA_RETURN_IF(tmp.alloc(bytes));
  for (size_t i = 0; i < blocks.size(); ++i) {
    pssa::DevBlock& B = *blocks[i];
    PSSA_HIP_TRY(hipMemcpyAsync(B.values.p, capped[i].p, bytes, hipMemcpyDeviceToDevice, st));
    if (M->dtype == PSSA_HIP_F32) {
      PSSA_RETURN_IF(pssa::launch_transpose(st, B.values.as<float>(), B.values_t.as<float>(), 1, C, d, 1.0f));
    } else {
      PSSA_RETURN_IF(pssa::launch_transpose(st, B.values.as<float>(), tmp.as<float>(), 1, C, d, 1.0f));
      PSSA_RETURN_IF(pssa::launch_to_bf16(st, tmp.as<float>(), C, B.values_t.as<uint16_t>(), C, d, C));
    }
  }
  return sync(M->ctx);  // the staging buffers are freed at return
}

// Empties every lane's repetition-penalty window (a new generation,
// src/inference.rs:345-347).  Fill kernels, so the call may sit in a graph.
Status clear_history(pssa_hip_lanes* L) {
  PSSA_RETURN_IF(pssa::launch_fill_zero(L->ctx->stream, static_cast<float*>(L->hist_n.p), L->lanes));
  return pssa::launch_fill_zero(L->ctx->stream, static_cast<float*>(L->hist_pos.p), L->lanes);
}

// The device copy of a GEMM weight (CudaContext::weight_buffer,
// src/cuda.rs:198-227): reused while current, uploaded again when stale,
// uploaded and kept on first use.  Called with ctx->mu held.
Status cached_weight(pssa_hip_ctx* ctx, const void* host, size_t n, int dtype, const void** out) {
  const size_t bytes = n * (dtype == PSSA_HIP_BF16 ? 2 : 4);
  auto key = std::make_tuple((uintptr_t)host, n, dtype);
  auto it = ctx->weights.find(key);
  if (it == ctx->weights.end()) {
    pssa_hip_ctx::CachedWeight cw;
    PSSA_RETURN_IF(upload(cw.buf, host, bytes, ctx->stream));
    it = ctx->weights.emplace(key, std::move(cw)).first;
  } else if (!it->second.current) {
    PSSA_HIP_TRY(hipMemcpyAsync(it->second.buf.p, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    it->second.current = true;
  }
  *out = it->second.buf.p;
  return Status::Ok();
}

Status stage_ids_locked(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t T) {
  PSSA_RETURN_IF(need(ids != nullptr, "null ids"));
  PSSA_RETURN_IF(need(T > 0, "prefill requires at least one token"));
  PSSA_RETURN_IF(need(n_lanes > 0 && n_lanes <= L->lanes, "n_lanes must be in 1..=lanes"));
  PSSA_RETURN_IF(need(n_lanes * T <= L->max_tokens, "n_lanes*seq_len exceeds max_tokens"));
  const uint32_t V = (uint32_t)L->model->cfg.d_vocab;
  for (size_t i = 0; i < n_lanes * T; ++i)
    if (ids[i] >= V)
      return Status::Invalid("prompt ID " + std::to_string(ids[i]) + " outside model vocabulary");
  PSSA_HIP_TRY(hipMemcpyAsync(L->ids.p, ids, n_lanes * T * 4, hipMemcpyHostToDevice, L->ctx->stream));
  L->staged_lanes = n_lanes;
  L->staged_len = T;
  return Status::Ok();
}

}  // namespace

extern "C" {

int pssa_hip_abi_version(void) { return PSSA_HIP_ABI_VERSION; }

int pssa_hip_is_fatal(int code) { return code == PSSA_HIP_EDEVICE ? 1 : 0; }

int pssa_hip_init(int device, pssa_hip_ctx** out, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    if (!out) return Status::Invalid("null output handle");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
      (void)hipGetLastError();
      return Status::NoDev("no HIP device visible");
    }
    if (device < 0 || device >= n) return Status::NoDev("device index out of range");
    hipDeviceProp_t prop;
    PSSA_HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      return Status::NoDev(std::string("device is ") + prop.gcnArchName + ", this build targets gfx950");
    PSSA_HIP_TRY(hipSetDevice(device));
    auto ctx = std::make_unique<pssa_hip_ctx>();
    ctx->device = device;
    ctx->name = prop.name;
    ctx->cu_count = prop.multiProcessorCount;
    PSSA_HIP_TRY(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    PSSA_RETURN_IF(pssa::init_gemm_attributes());
    PSSA_RETURN_IF(pssa::init_retrieve_attributes());
    PSSA_RETURN_IF(pssa::init_decode_attributes());
    PSSA_RETURN_IF(pssa::init_dense_scan_attributes());
    PSSA_RETURN_IF(pssa::noalloc_scratch_address(&ctx->noalloc_scratch));
    *out = ctx.release();
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

void pssa_hip_destroy(pssa_hip_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
  }
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  delete ctx;
}

int pssa_hip_device_name(const pssa_hip_ctx* ctx, char* out, size_t out_len) {
  if (!ctx || !out || !out_len) return PSSA_HIP_EINVAL;
  std::snprintf(out, out_len, "hip:%s (gfx950, %d CUs)", ctx->name.c_str(), ctx->cu_count);
  return PSSA_HIP_OK;
}

int pssa_hip_device_alloc(pssa_hip_ctx* ctx, size_t bytes, void** out, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(out != nullptr, "null output handle"));
    *out = nullptr;
    PSSA_RETURN_IF(need(bytes > 0 && bytes <= ((size_t)1 << 40), "allocation size must be in 1..=2^40"));
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return Status::NoMem(std::string("hipMalloc: ") + hipGetErrorString(e));
    }
    *out = p;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

void pssa_hip_device_free(pssa_hip_ctx* ctx, void* p) {
  if (!ctx || !p) return;
  std::lock_guard<std::mutex> g(ctx->mu);
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipFree(p);
}

int pssa_hip_memcpy(pssa_hip_ctx* ctx, void* dst, const void* src, size_t bytes, int kind, char* err,
                    size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(dst && src, "memcpy: null pointer"));
    PSSA_RETURN_IF(need(kind == PSSA_HIP_H2D || kind == PSSA_HIP_D2H || kind == PSSA_HIP_D2D, "memcpy: unknown kind"));
    if (bytes == 0) return Status::Ok();
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    const hipMemcpyKind k = kind == PSSA_HIP_H2D ? hipMemcpyHostToDevice
                            : kind == PSSA_HIP_D2H ? hipMemcpyDeviceToHost
                                                   : hipMemcpyDeviceToDevice;
    PSSA_HIP_TRY(hipMemcpyAsync(dst, src, bytes, k, ctx->stream));
    return sync(ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_synchronize(pssa_hip_ctx* ctx, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    return sync(ctx);
  };
  return pssa::finish(body(), err, err_len);
}

// ------------------------------------------------------------------- GEMM
int pssa_hip_gemm_xwt(pssa_hip_ctx* ctx, const float* x, size_t x_len, const void* w, size_t w_len,
                      int w_dtype, size_t m, size_t n, size_t k, size_t batch, float* y,
                      size_t y_len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(x && w && y, "gemm: null buffer"));
    PSSA_RETURN_IF(need(m && n && k && batch, "GEMM dimensions must be positive"));
    PSSA_RETURN_IF(need(w_dtype == PSSA_HIP_F32 || w_dtype == PSSA_HIP_BF16, "gemm: unknown dtype"));
    size_t rows = 0, xin = 0, win = 0, yout = 0;
    PSSA_RETURN_IF(pssa::checked_count({m, batch}, &rows, "gemm rows"));
    PSSA_RETURN_IF(pssa::checked_count({rows, k}, &xin, "gemm input"));
    PSSA_RETURN_IF(pssa::checked_count({n, k}, &win, "gemm weights"));
    PSSA_RETURN_IF(pssa::checked_count({rows, n}, &yout, "gemm output"));
    if (x_len != xin || w_len != win)
      return Status::Invalid("GEMM operand lengths must be " + std::to_string(xin) + " and " +
                             std::to_string(win) + ", got " + std::to_string(x_len) + " and " +
                             std::to_string(w_len));
    if (y_len != yout) return Status::Invalid("GEMM output length mismatch");
    if (rows > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return Status::Invalid("gemm: too large");
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    DevBuf dx, dxh, dy;
    PSSA_RETURN_IF(upload(dx, x, xin * 4, ctx->stream));
    const void* dw = nullptr;
    PSSA_RETURN_IF(cached_weight(ctx, w, win, w_dtype, &dw));
    PSSA_RETURN_IF(dy.alloc(yout * 4));
    const void* a = dx.p;
    if (w_dtype == PSSA_HIP_BF16) {
      // bf16 weights multiply bf16-rounded activations (fp32 accumulation).
      PSSA_RETURN_IF(dxh.alloc(xin * 2));
      PSSA_RETURN_IF(pssa::launch_to_bf16(ctx->stream, dx.as<float>(), (int)k, dxh.as<uint16_t>(), (int)k, rows, (int)k));
      a = dxh.p;
    }
    pssa::EpiParams ep;
    ep.out32 = dy.as<float>();
    ep.ld32 = (int)n;
    PSSA_RETURN_IF(pssa::launch_gemm(ctx->stream, w_dtype, a, (int)k, dw, (int)k, (int)rows, (int)n, (int)k, ep));
    PSSA_RETURN_IF(download(y, dy, yout * 4, ctx->stream));
    return sync(ctx);
  };
  return pssa::finish(body(), err, err_len);
}

// Shared body of gemm_nn and gemm_tn_accumulate: y = x w^T on the device
// after transposing the operands the layout asks for (`x_t`: x arrives as
// [kx, rows]; `w_t`: w arrives as [k, n]); `accumulate` adds the product to
// the caller's y.
static Status gemm_transposed(pssa_hip_ctx* ctx, const float* x, const float* w, size_t rows, size_t n, size_t k,
                              bool x_t, bool w_t, bool accumulate, float* y) {
  std::lock_guard<std::mutex> g(ctx->mu);
  PSSA_HIP_TRY(hipSetDevice(ctx->device));
  const hipStream_t st = ctx->stream;
  DevBuf dx, dw, dxt, dwt, dy, dacc;
  PSSA_RETURN_IF(upload(dx, x, rows * k * 4, st));
  PSSA_RETURN_IF(upload(dw, w, n * k * 4, st));
  const float* xa = dx.as<float>();
  const float* wa = dw.as<float>();
  if (x_t) {  // [k, rows] -> [rows, k]
    PSSA_RETURN_IF(dxt.alloc(rows * k * 4));
    PSSA_RETURN_IF(pssa::launch_transpose(st, xa, dxt.as<float>(), 1, (int)k, (int)rows, 1.0f));
    xa = dxt.as<float>();
  }
  if (w_t) {  // [k, n] -> [n, k]
    PSSA_RETURN_IF(dwt.alloc(n * k * 4));
    PSSA_RETURN_IF(pssa::launch_transpose(st, wa, dwt.as<float>(), 1, (int)k, (int)n, 1.0f));
    wa = dwt.as<float>();
  }
  PSSA_RETURN_IF(dy.alloc(rows * n * 4));
  pssa::EpiParams ep;
  ep.out32 = dy.as<float>();
  ep.ld32 = (int)n;
  if (accumulate) {
    PSSA_RETURN_IF(upload(dacc, y, rows * n * 4, st));
    ep.kind = pssa::EPI_ADD_AUX;
    ep.aux = dacc.as<float>();
    ep.ld_aux = (int)n;
  }
  PSSA_RETURN_IF(pssa::launch_gemm(st, PSSA_HIP_F32, xa, (int)k, wa, (int)k, (int)rows, (int)n, (int)k, ep));
  PSSA_RETURN_IF(download(y, dy, rows * n * 4, st));
  return sync(ctx);
}

static Status gemm_dims(size_t m, size_t k, size_t n, size_t a_len, size_t b_len, size_t out_len, size_t a_exp,
                        size_t b_exp, size_t out_exp) {
  PSSA_RETURN_IF(need(m && k && n, "GEMM dimensions must be positive"));
  if (a_exp > INT32_MAX || b_exp > INT32_MAX || out_exp > INT32_MAX) return Status::Invalid("gemm: too large");
  if (a_len != a_exp || b_len != b_exp || out_len != out_exp)
    return Status::Invalid("GEMM operand lengths must be " + std::to_string(a_exp) + ", " + std::to_string(b_exp) +
                           " and " + std::to_string(out_exp));
  return Status::Ok();
}

int pssa_hip_gemm_nn(pssa_hip_ctx* ctx, const float* a, size_t a_len, const float* b, size_t b_len, size_t m,
                     size_t k, size_t n, float* out, size_t out_len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(a && b && out, "gemm: null buffer"));
    size_t ae = 0, be = 0, oe = 0;
    PSSA_RETURN_IF(pssa::checked_count({m, k}, &ae, "gemm lhs"));
    PSSA_RETURN_IF(pssa::checked_count({k, n}, &be, "gemm rhs"));
    PSSA_RETURN_IF(pssa::checked_count({m, n}, &oe, "gemm output"));
    PSSA_RETURN_IF(gemm_dims(m, k, n, a_len, b_len, out_len, ae, be, oe));
    return gemm_transposed(ctx, a, b, m, n, k, false, true, false, out);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_gemm_tn_accumulate(pssa_hip_ctx* ctx, const float* a, size_t a_len, const float* b, size_t b_len,
                                size_t m, size_t k, size_t n, float* out, size_t out_len, char* err,
                                size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(a && b && out, "gemm: null buffer"));
    size_t ae = 0, be = 0, oe = 0;
    PSSA_RETURN_IF(pssa::checked_count({m, k}, &ae, "gemm lhs"));
    PSSA_RETURN_IF(pssa::checked_count({m, n}, &be, "gemm rhs"));
    PSSA_RETURN_IF(pssa::checked_count({k, n}, &oe, "gemm output"));
    PSSA_RETURN_IF(gemm_dims(m, k, n, a_len, b_len, out_len, ae, be, oe));
    // C(K,N) += A^T B: rows = K, reduction over M; A [M,K] and B [M,N] both
    // arrive reduction-major.
    return gemm_transposed(ctx, a, b, k, n, m, true, true, true, out);
  };
  return pssa::finish(body(), err, err_len);
}

void pssa_hip_invalidate_weights(pssa_hip_ctx* ctx) {
  if (!ctx) return;
  std::lock_guard<std::mutex> g(ctx->mu);
  for (auto& kv : ctx->weights) kv.second.current = false;
}

int pssa_hip_invalidate_weights_only(pssa_hip_ctx* ctx, const pssa_hip_weight_key* keys, size_t n_keys,
                                     char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(keys || n_keys == 0, "null weight keys"));
    std::lock_guard<std::mutex> g(ctx->mu);
    for (auto& kv : ctx->weights)
      for (size_t i = 0; i < n_keys; ++i)
        if (std::get<0>(kv.first) == (uintptr_t)keys[i].ptr && std::get<1>(kv.first) == keys[i].len)
          kv.second.current = false;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_weight_cache_stats(pssa_hip_ctx* ctx, size_t* entries, size_t* current, size_t* bytes) {
  if (!ctx) return PSSA_HIP_EINVAL;
  std::lock_guard<std::mutex> g(ctx->mu);
  size_t e = 0, c = 0, b = 0;
  for (const auto& kv : ctx->weights) {
    ++e;
    c += kv.second.current ? 1 : 0;
    b += kv.second.buf.bytes;
  }
  if (entries) *entries = e;
  if (current) *current = c;
  if (bytes) *bytes = b;
  return PSSA_HIP_OK;
}

int pssa_hip_softplus_in_place(pssa_hip_ctx* ctx, float* values, size_t len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(values || len == 0, "softplus: null buffer"));
    if (len == 0) return Status::Ok();
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    DevBuf dv;
    PSSA_RETURN_IF(upload(dv, values, len * 4, ctx->stream));
    PSSA_RETURN_IF(pssa::launch_softplus(ctx->stream, dv.as<float>(), len));
    PSSA_RETURN_IF(download(values, dv, len * 4, ctx->stream));
    return sync(ctx);
  };
  return pssa::finish(body(), err, err_len);
}

// -------------------------------------------------------------- SSM stage
// Device results of one stage-API scan (the reference's SSM tape fields,
// src/gpu_batch.rs:392-437): y [L,d], the final carry (state-major [s,d]),
// and when materialised bar_a, bar_b [L*d*s] and states [(L+1)*d*s].
struct SsmTape {
  size_t L = 0, d = 0, s = 0;
  DevBuf y, carry, carry_ds, bar_a, bar_b, states;
};

static Status check_ssm_shapes(size_t seq_len, size_t d_m, size_t d_s, size_t delta_len, size_t b_len,
                               size_t x_len, size_t rates_len, size_t c_len, size_t initial_len) {
  PSSA_RETURN_IF(need(seq_len && d_m && d_s, "ssm: dimensions must be positive"));
  size_t ld = 0, ls = 0, w = 0, lw1 = 0;
  PSSA_RETURN_IF(pssa::checked_count({seq_len, d_m}, &ld, "ssm"));
  PSSA_RETURN_IF(pssa::checked_count({seq_len, d_s}, &ls, "ssm"));
  PSSA_RETURN_IF(pssa::checked_count({d_m, d_s}, &w, "ssm"));
  PSSA_RETURN_IF(pssa::checked_count({seq_len + 1, w}, &lw1, "ssm"));
  if (delta_len != ld || x_len != ld) return Status::Invalid("ssm: delta/x_norm/y_ssm must be seq_len*d_m");
  if (b_len != ls || c_len != ls) return Status::Invalid("ssm: b_proj/c_proj must be seq_len*d_s");
  if (rates_len != w || initial_len != w) return Status::Invalid("ssm: rates/initial must be d_m*d_s");
  if (seq_len > INT32_MAX || d_m > INT32_MAX || d_s > INT32_MAX) return Status::Invalid("ssm: too large");
  return Status::Ok();
}

// Runs the scan of the stage API into `t` (called with ctx->mu held).
static Status run_stage_ssm(pssa_hip_ctx* ctx, const float* delta, const float* b_proj, const float* x_norm,
                            const float* rates, const float* c_proj, const float* initial, size_t seq_len,
                            size_t d_m, size_t d_s, bool materialize, SsmTape& t) {
  const hipStream_t st = ctx->stream;
  const size_t ld = seq_len * d_m, ls = seq_len * d_s, w = d_m * d_s;
  t.L = seq_len;
  t.d = d_m;
  t.s = d_s;
  DevBuf dd, db, dx, dr, dc, dr2;
  PSSA_RETURN_IF(upload(dd, delta, ld * 4, st));
  PSSA_RETURN_IF(upload(db, b_proj, ls * 4, st));
  PSSA_RETURN_IF(upload(dx, x_norm, ld * 4, st));
  PSSA_RETURN_IF(upload(dr, rates, w * 4, st));
  PSSA_RETURN_IF(upload(dc, c_proj, ls * 4, st));
  PSSA_RETURN_IF(upload(t.carry_ds, initial, w * 4, st));
  PSSA_RETURN_IF(t.y.alloc(ld * 4));
  // The scan keeps rates state-major ([s, d]) and states channel-blocked
  // (pssa::carry_at); the stage API speaks the reference's [d, s].
  PSSA_RETURN_IF(dr2.alloc(w * 4));
  PSSA_RETURN_IF(t.carry.alloc(w * 4));
  PSSA_RETURN_IF(pssa::launch_transpose(st, dr.as<float>(), dr2.as<float>(), 1, (int)d_m, (int)d_s,
                                        1.4426950408889634f));
  PSSA_RETURN_IF(pssa::launch_carry_convert(st, t.carry_ds.as<float>(), t.carry.as<float>(), 1, (int)d_m, (int)d_s,
                                            true));
  PSSA_RETURN_IF(pssa::launch_fill_zero(st, t.y.as<float>(), ld));
  pssa::SsmArgs a;
  a.delta = dd.as<float>();
  a.ld_delta = (int)d_m;
  a.bproj = db.as<float>();
  a.ld_b = (int)d_s;
  a.cproj = dc.as<float>();
  a.ld_c = (int)d_s;
  a.xn = dx.as<float>();
  a.ld_x = (int)d_m;
  a.rates2 = dr2.as<float>();
  a.carry = t.carry.as<float>();
  a.carry_stride = (long)w;
  a.y = t.y.as<float>();
  a.ld_y = (int)d_m;
  a.T = (int)seq_len;
  a.d = (int)d_m;
  a.s = (int)d_s;
  a.lanes = 1;
  DevBuf dpart;
  const int nz = pssa::ssm_state_blocks((int)d_s);
  if (!materialize && nz > 2) {
    PSSA_RETURN_IF(dpart.alloc((size_t)nz * ld * 4));
    a.y_part = dpart.as<float>();
  }
  if (materialize) {
    PSSA_RETURN_IF(t.bar_a.alloc(seq_len * w * 4));
    PSSA_RETURN_IF(t.bar_b.alloc(seq_len * w * 4));
    PSSA_RETURN_IF(t.states.alloc((seq_len + 1) * w * 4));
    a.bar_a = t.bar_a.as<float>();
    a.bar_b = t.bar_b.as<float>();
    a.states = t.states.as<float>();
  }
  PSSA_RETURN_IF(pssa::launch_ssm_scan(st, a));
  // Sources of the scan's inputs are freed at return: finish first.
  return sync(ctx);
}

// Copies the tape's host outputs (any may be NULL).
static Status download_ssm(pssa_hip_ctx* ctx, SsmTape& t, float* bar_a, float* bar_b, float* states, float* y_ssm,
                           float* final_state) {
  const hipStream_t st = ctx->stream;
  const size_t ld = t.L * t.d, w = t.d * t.s;
  if (y_ssm) PSSA_RETURN_IF(download(y_ssm, t.y, ld * 4, st));
  if (final_state) {
    PSSA_RETURN_IF(pssa::launch_carry_convert(st, t.carry.as<float>(), t.carry_ds.as<float>(), 1, (int)t.d, (int)t.s,
                                              false));
    PSSA_RETURN_IF(download(final_state, t.carry_ds, w * 4, st));
  }
  if (bar_a) PSSA_RETURN_IF(download(bar_a, t.bar_a, t.L * w * 4, st));
  if (bar_b) PSSA_RETURN_IF(download(bar_b, t.bar_b, t.L * w * 4, st));
  if (states) PSSA_RETURN_IF(download(states, t.states, (t.L + 1) * w * 4, st));
  return sync(ctx);
}

int pssa_hip_ssm_forward(pssa_hip_ctx* ctx, const float* delta, size_t delta_len,
                         const float* delta_raw, const float* b_proj, size_t b_len,
                         const float* x_norm, size_t x_len, const float* rates, size_t rates_len,
                         const float* rate_deriv, const float* c_proj, size_t c_len,
                         const float* initial, size_t initial_len, size_t seq_len, size_t d_m,
                         size_t d_s, float* bar_a, float* bar_b, float* states, float* y_ssm,
                         size_t y_len, float* final_state, char* err, size_t err_len) {
  (void)delta_raw;
  (void)rate_deriv;
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(delta && b_proj && x_norm && rates && c_proj && initial && y_ssm, "ssm: null input"));
    PSSA_RETURN_IF(need((bar_a == nullptr) == (bar_b == nullptr) && (bar_a == nullptr) == (states == nullptr),
                        "ssm: bar_a, bar_b and states are materialised together"));
    PSSA_RETURN_IF(check_ssm_shapes(seq_len, d_m, d_s, delta_len, b_len, x_len, rates_len, c_len, initial_len));
    PSSA_RETURN_IF(need(y_len == seq_len * d_m, "ssm: delta/x_norm/y_ssm must be seq_len*d_m"));
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    SsmTape t;
    PSSA_RETURN_IF(run_stage_ssm(ctx, delta, b_proj, x_norm, rates, c_proj, initial, seq_len, d_m, d_s,
                                 bar_a != nullptr, t));
    return download_ssm(ctx, t, bar_a, bar_b, states, y_ssm, final_state);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_ssm_forward_resident(pssa_hip_ctx* ctx, const float* delta, size_t delta_len, const float* delta_raw,
                                  const float* b_proj, size_t b_len, const float* x_norm, size_t x_len,
                                  const float* rates, size_t rates_len, const float* c_proj, size_t c_len,
                                  const float* initial, size_t initial_len, size_t seq_len, size_t d_m,
                                  size_t d_s, char* err, size_t err_len) {
  (void)delta_raw;
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(delta && b_proj && x_norm && rates && c_proj && initial, "ssm: null input"));
    PSSA_RETURN_IF(check_ssm_shapes(seq_len, d_m, d_s, delta_len, b_len, x_len, rates_len, c_len, initial_len));
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    ctx->ssm_tape.reset();
    auto t = std::make_shared<SsmTape>();
    PSSA_RETURN_IF(run_stage_ssm(ctx, delta, b_proj, x_norm, rates, c_proj, initial, seq_len, d_m, d_s, true, *t));
    ctx->ssm_tape = t;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

// ----------------------------------------------------------- memory stage
static Status check_memory_args(size_t seq_len, size_t d_m, size_t d_k, size_t d_val, size_t capacity,
                                size_t count, float tau, size_t top_k) {
  PSSA_RETURN_IF(need(seq_len && d_m && d_k && d_val && capacity, "memory: dimensions must be positive"));
  PSSA_RETURN_IF(need(d_val == d_m, "memory: the model path reads values of width d_latent"));
  PSSA_RETURN_IF(need(count <= capacity, "memory: count exceeds capacity"));
  PSSA_RETURN_IF(need(top_k <= (size_t)pssa::kMaxTopK, "memory: top_k must be at most 64"));
  PSSA_RETURN_IF(need(std::isfinite(tau) && tau > 0.0f, "tau must be positive and finite"));
  if (seq_len > INT32_MAX / 4 || d_m > 16384 || d_k > 4096 || capacity > 8192)
    return Status::Invalid("memory: shape exceeds the supported range");
  return Status::Ok();
}

// The memory stage of the stage API on the device copy `dy` of y_ssm
// (called with ctx->mu held).
static Status run_stage_memory(pssa_hip_ctx* ctx, const float* x_norm, const float* dy_ptr, const float* w_qx,
                               const float* w_qh, const float* w_gate, const float* w_proj, const float* keys,
                               const float* norm_sq, const float* values, size_t seq_len, size_t d_m,
                               size_t d_k, size_t capacity, size_t count, float tau, size_t top_k,
                               float* q_euc, float* q_pnc, float* q_norm, float* weights, float* m_val,
                               float* g_mem, float* m_proj, float* m_inj) {
  const hipStream_t st = ctx->stream;
  const int L = (int)seq_len, d = (int)d_m, k = (int)d_k, C = (int)capacity;
  DevBuf dx, dwqx, dwqh, dwg, dwp, dk_, dn, dv, dvt, qx, qe, qp, qn, wts, mv, gm, mp, mi;
  PSSA_RETURN_IF(upload(dx, x_norm, (size_t)L * d * 4, st));
  PSSA_RETURN_IF(upload(dwqx, w_qx, (size_t)k * d * 4, st));
  PSSA_RETURN_IF(upload(dwqh, w_qh, (size_t)k * d * 4, st));
  PSSA_RETURN_IF(upload(dwg, w_gate, (size_t)d * d * 4, st));
  PSSA_RETURN_IF(upload(dwp, w_proj, (size_t)d * d * 4, st));
  PSSA_RETURN_IF(upload(dk_, keys, (size_t)C * k * 4, st));
  PSSA_RETURN_IF(upload(dn, norm_sq, (size_t)C * 4, st));
  PSSA_RETURN_IF(upload(dv, values, (size_t)C * d * 4, st));
  std::vector<float> vt((size_t)d * C);
  for (int s2 = 0; s2 < C; ++s2)
    for (int j = 0; j < d; ++j) vt[(size_t)j * C + s2] = values[(size_t)s2 * d + j];
  PSSA_RETURN_IF(upload(dvt, vt.data(), vt.size() * 4, st));
  for (DevBuf* b : {&qx, &qe, &qp}) PSSA_RETURN_IF(b->alloc((size_t)L * k * 4));
  PSSA_RETURN_IF(qn.alloc((size_t)L * 4));
  PSSA_RETURN_IF(wts.alloc((size_t)L * C * 4));
  for (DevBuf* b : {&mv, &gm, &mp, &mi}) PSSA_RETURN_IF(b->alloc((size_t)L * d * 4));
  // q_euc = x W_qx^T + y W_qh^T, as dot(row_x, x) + dot(row_h, y) (src/pssa.rs:1147-1152).
  pssa::EpiParams ex;
  ex.out32 = qx.as<float>();
  ex.ld32 = k;
  PSSA_RETURN_IF(pssa::launch_gemm(st, PSSA_HIP_F32, dx.p, d, dwqx.p, d, L, k, d, ex));
  pssa::EpiParams eq;
  eq.kind = pssa::EPI_ADD_AUX;
  eq.aux = qx.as<float>();
  eq.ld_aux = k;
  eq.out32 = qe.as<float>();
  eq.ld32 = k;
  PSSA_RETURN_IF(pssa::launch_gemm(st, PSSA_HIP_F32, dy_ptr, d, dwqh.p, d, L, k, d, eq));
  pssa::RetrieveArgs ra;
  ra.q = qe.as<float>();
  ra.ld_q = k;
  ra.project = 1;
  ra.q_pnc = qp.as<float>();
  ra.q_norm = qn.as<float>();
  ra.keys = dk_.as<float>();
  ra.norm_sq = dn.as<float>();
  ra.values = dv.as<float>();
  ra.n = L;
  ra.dk = k;
  ra.dv = d;
  ra.capacity = C;
  ra.count = (int)count;
  ra.tau = tau;
  ra.top_k = (int)top_k;
  ra.weights = wts.as<float>();
  const bool sparse = top_k > 0 && top_k < count;
  if (sparse) ra.out_val = mv.as<float>();
  PSSA_RETURN_IF(pssa::launch_retrieve(st, ra));
  if (!sparse) {
    if (count > 0) {
      pssa::EpiParams em;
      em.out32 = mv.as<float>();
      em.ld32 = d;
      PSSA_RETURN_IF(pssa::launch_gemm(st, PSSA_HIP_F32, wts.p, C, dvt.p, C, L, d, (int)count, em));
    } else {
      PSSA_RETURN_IF(pssa::launch_fill_zero(st, mv.as<float>(), (size_t)L * d));
    }
  }
  pssa::EpiParams eg;
  eg.kind = pssa::EPI_SEGMENTS;
  eg.seg[0] = 0;
  eg.seg[1] = 0;
  eg.seg[2] = d;
  eg.seg[3] = d;
  eg.out32 = gm.as<float>();
  eg.ld32 = d;
  PSSA_RETURN_IF(pssa::launch_gemm(st, PSSA_HIP_F32, dx.p, d, dwg.p, d, L, d, d, eg));
  pssa::EpiParams ep2;
  ep2.out32 = mp.as<float>();
  ep2.ld32 = d;
  PSSA_RETURN_IF(pssa::launch_gemm(st, PSSA_HIP_F32, mv.p, d, dwp.p, d, L, d, d, ep2));
  PSSA_RETURN_IF(pssa::launch_mul(st, gm.as<float>(), mp.as<float>(), mi.as<float>(), (size_t)L * d));
  if (q_euc) PSSA_RETURN_IF(download(q_euc, qe, (size_t)L * k * 4, st));
  if (q_pnc) PSSA_RETURN_IF(download(q_pnc, qp, (size_t)L * k * 4, st));
  if (q_norm) PSSA_RETURN_IF(download(q_norm, qn, (size_t)L * 4, st));
  if (weights) PSSA_RETURN_IF(download(weights, wts, (size_t)L * C * 4, st));
  if (m_val) PSSA_RETURN_IF(download(m_val, mv, (size_t)L * d * 4, st));
  if (g_mem) PSSA_RETURN_IF(download(g_mem, gm, (size_t)L * d * 4, st));
  if (m_proj) PSSA_RETURN_IF(download(m_proj, mp, (size_t)L * d * 4, st));
  PSSA_RETURN_IF(download(m_inj, mi, (size_t)L * d * 4, st));
  return sync(ctx);
}

int pssa_hip_memory_forward(pssa_hip_ctx* ctx, const float* x_norm, const float* y_ssm,
                            const float* w_qx, const float* w_qh, const float* w_gate,
                            const float* w_proj, const float* keys, const float* norm_sq,
                            const float* values, size_t seq_len, size_t d_m, size_t d_k,
                            size_t d_val, size_t capacity, size_t count, float tau, size_t top_k,
                            float* q_euc, float* q_pnc, float* q_norm, float* weights,
                            float* m_val, float* g_mem, float* m_proj, float* m_inj, char* err,
                            size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(check_memory_args(seq_len, d_m, d_k, d_val, capacity, count, tau, top_k));
    PSSA_RETURN_IF(need(x_norm && y_ssm && w_qx && w_qh && w_gate && w_proj && keys && norm_sq &&
                            values && m_inj,
                        "memory: null input"));
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    DevBuf dy;
    PSSA_RETURN_IF(upload(dy, y_ssm, seq_len * d_m * 4, ctx->stream));
    return run_stage_memory(ctx, x_norm, dy.as<float>(), w_qx, w_qh, w_gate, w_proj, keys, norm_sq, values,
                            seq_len, d_m, d_k, capacity, count, tau, top_k, q_euc, q_pnc, q_norm, weights, m_val,
                            g_mem, m_proj, m_inj);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_memory_forward_after_ssm(pssa_hip_ctx* ctx, const float* x_norm, const float* w_qx,
                                      const float* w_qh, const float* w_gate, const float* w_proj,
                                      const float* keys, const float* norm_sq, const float* values,
                                      size_t seq_len, size_t d_m, size_t d_k, size_t d_val, size_t capacity,
                                      size_t count, float tau, size_t top_k, float* bar_a, float* bar_b,
                                      float* states, float* y_ssm, float* q_euc, float* q_pnc, float* q_norm,
                                      float* weights, float* m_val, float* g_mem, float* m_proj, float* m_inj,
                                      char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(check_memory_args(seq_len, d_m, d_k, d_val, capacity, count, tau, top_k));
    PSSA_RETURN_IF(need(x_norm && w_qx && w_qh && w_gate && w_proj && keys && norm_sq && values && m_inj,
                        "memory: null input"));
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_RETURN_IF(need(ctx->ssm_tape && ctx->ssm_tape->L == seq_len && ctx->ssm_tape->d == d_m,
                        "memory_forward_after_ssm: no resident SSM tape of this shape "
                        "(pssa_hip_ssm_forward_resident comes first)"));
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    std::shared_ptr<SsmTape> t = std::move(ctx->ssm_tape);  // consumed by this call
    PSSA_RETURN_IF(run_stage_memory(ctx, x_norm, t->y.as<float>(), w_qx, w_qh, w_gate, w_proj, keys, norm_sq,
                                    values, seq_len, d_m, d_k, capacity, count, tau, top_k, q_euc, q_pnc, q_norm,
                                    weights, m_val, g_mem, m_proj, m_inj));
    return download_ssm(ctx, *t, bar_a, bar_b, states, y_ssm, nullptr);
  };
  return pssa::finish(body(), err, err_len);
}

}  // extern "C"

// Points ra.scratch at the context's scratch, grown to what the launch needs.
// Called with ctx->mu held; the previous buffer is released only once the
// stream has drained.
static Status bind_retrieve_scratch(pssa_hip_ctx* ctx, pssa::RetrieveArgs& ra) {
  const size_t need_bytes = pssa::retrieve_scratch_bytes(ra);
  if (!need_bytes) return Status::Ok();
  if (ctx->scratch_bytes < need_bytes) {
    PSSA_HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (ctx->scratch) PSSA_HIP_TRY(hipFree(ctx->scratch));
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    PSSA_HIP_TRY(hipMalloc(&ctx->scratch, need_bytes));
    ctx->scratch_bytes = need_bytes;
  }
  ra.scratch = ctx->scratch;
  ra.scratch_bytes = ctx->scratch_bytes;
  return Status::Ok();
}

// Grows the context's scratch to what the two-level dense scan needs.
// Called with ctx->mu held.
static Status bind_dense_scan_scratch(pssa_hip_ctx* ctx, int batch, int L, int s) {
  const size_t need_bytes = pssa::dense_scan_scratch_bytes(batch, L, s);
  if (!need_bytes || ctx->scratch_bytes >= need_bytes) return Status::Ok();
  PSSA_HIP_TRY(hipStreamSynchronize(ctx->stream));
  if (ctx->scratch) PSSA_HIP_TRY(hipFree(ctx->scratch));
  ctx->scratch = nullptr;
  ctx->scratch_bytes = 0;
  PSSA_HIP_TRY(hipMalloc(&ctx->scratch, need_bytes));
  ctx->scratch_bytes = need_bytes;
  return Status::Ok();
}

extern "C" {

// Host-buffer retrieval; gate/age (both or neither) select the hybrid read.
static int retrieve_host(pssa_hip_ctx* ctx, const float* q_pnc, size_t n_q, const float* keys,
                         const float* norm_sq, const float* values, size_t capacity, size_t count,
                         size_t d_key, size_t d_val, float tau, size_t top_k, const float* gate,
                         const uint64_t* age, float lam, float* out_val, float* out_min, uint32_t* out_idx,
                         float* out_weights, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(n_q && d_key && d_val && capacity, "retrieve: dimensions must be positive"));
    PSSA_RETURN_IF(need(count <= capacity, "retrieve: count exceeds capacity"));
    PSSA_RETURN_IF(need(top_k <= (size_t)pssa::kMaxTopK, "retrieve: top_k must be at most 64"));
    PSSA_RETURN_IF(need(std::isfinite(tau) && tau > 0.0f, "tau must be positive and finite"));
    PSSA_RETURN_IF(need(q_pnc && keys && norm_sq && values && out_val, "retrieve: null buffer"));
    PSSA_RETURN_IF(need(!out_idx || top_k > 0, "retrieve: indices need top_k > 0"));
    const bool hybrid = gate != nullptr;
    if (hybrid) {
      PSSA_RETURN_IF(need(age != nullptr, "retrieve: the hybrid read needs gates and ages"));
      PSSA_RETURN_IF(need(std::isfinite(lam) && lam > 0.0f && lam <= 1.0f, "hybrid decay lam must be in (0.0, 1.0]"));
      for (size_t q = 0; q < count; ++q)
        PSSA_RETURN_IF(need(std::isfinite(gate[q]) && gate[q] >= 0.0f,
                            "hybrid write gate must be finite and nonnegative"));
    }
    if (n_q > INT32_MAX / 4 || d_key > 4096 || d_val > 65536 || capacity > 8192)
      return Status::Invalid("retrieve: shape exceeds the supported range");
    // The query must lie in the open ball (retrieve_soft_into's assertion).
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    const hipStream_t st = ctx->stream;
    DevBuf dq, dk_, dn, dv, dval, dmin, didx, dw, dg, da;
    PSSA_RETURN_IF(upload(dq, q_pnc, n_q * d_key * 4, st));
    PSSA_RETURN_IF(upload(dk_, keys, capacity * d_key * 4, st));
    PSSA_RETURN_IF(upload(dn, norm_sq, capacity * 4, st));
    PSSA_RETURN_IF(upload(dv, values, capacity * d_val * 4, st));
    if (hybrid && count > 0) {
      PSSA_RETURN_IF(upload(dg, gate, count * 4, st));
      PSSA_RETURN_IF(upload(da, age, count * 8, st));
    }
    PSSA_RETURN_IF(dval.alloc(n_q * d_val * 4));
    if (out_min) PSSA_RETURN_IF(dmin.alloc(n_q * 4));
    if (out_idx) PSSA_RETURN_IF(didx.alloc(n_q * top_k * 4));
    if (out_weights) PSSA_RETURN_IF(dw.alloc(n_q * capacity * 4));
    pssa::RetrieveArgs ra;
    ra.q = dq.as<float>();
    ra.ld_q = (int)d_key;
    ra.project = 0;
    ra.keys = dk_.as<float>();
    ra.norm_sq = dn.as<float>();
    ra.values = dv.as<float>();
    ra.n = (int)n_q;
    ra.dk = (int)d_key;
    ra.dv = (int)d_val;
    ra.capacity = (int)capacity;
    ra.count = (int)count;
    ra.tau = tau;
    ra.top_k = (int)top_k;
    ra.weights = out_weights ? dw.as<float>() : nullptr;
    ra.out_val = dval.as<float>();
    ra.out_min = out_min ? dmin.as<float>() : nullptr;
    ra.out_idx = out_idx ? didx.as<uint32_t>() : nullptr;
    if (hybrid && count > 0) {
      ra.hgate = dg.as<float>();
      ra.hage = da.as<unsigned long long>();
      ra.log_lam = std::log((double)lam);
    }
    PSSA_RETURN_IF(bind_retrieve_scratch(ctx, ra));
    PSSA_RETURN_IF(pssa::launch_retrieve(st, ra));
    PSSA_RETURN_IF(download(out_val, dval, n_q * d_val * 4, st));
    if (out_min) PSSA_RETURN_IF(download(out_min, dmin, n_q * 4, st));
    if (out_idx) PSSA_RETURN_IF(download(out_idx, didx, n_q * top_k * 4, st));
    if (out_weights) PSSA_RETURN_IF(download(out_weights, dw, n_q * capacity * 4, st));
    return sync(ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_retrieve(pssa_hip_ctx* ctx, const float* q_pnc, size_t n_q, const float* keys,
                      const float* norm_sq, const float* values, size_t capacity, size_t count,
                      size_t d_key, size_t d_val, float tau, size_t top_k, float* out_val,
                      float* out_min, uint32_t* out_idx, float* out_weights, char* err, size_t err_len) {
  return retrieve_host(ctx, q_pnc, n_q, keys, norm_sq, values, capacity, count, d_key, d_val, tau, top_k,
                       nullptr, nullptr, 1.0f, out_val, out_min, out_idx, out_weights, err, err_len);
}

int pssa_hip_retrieve_hybrid(pssa_hip_ctx* ctx, const float* q_pnc, size_t n_q, const float* keys,
                             const float* norm_sq, const float* values, size_t capacity, size_t count,
                             size_t d_key, size_t d_val, float tau, size_t top_k, const float* gate,
                             const uint64_t* age, float lam, float* out_val, float* out_min,
                             uint32_t* out_idx, float* out_weights, char* err, size_t err_len) {
  if (!gate || !age) {
    if (err && err_len) std::snprintf(err, err_len, "retrieve: the hybrid read needs gates and ages");
    return PSSA_HIP_EINVAL;
  }
  return retrieve_host(ctx, q_pnc, n_q, keys, norm_sq, values, capacity, count, d_key, d_val, tau, top_k, gate,
                       age, lam, out_val, out_min, out_idx, out_weights, err, err_len);
}

// Device-buffer retrieval.  no_alloc: the ranked path's scratch is the
// device's static array (kNoallocChunk queries per pass) instead of the
// context's grown buffer, so nothing is allocated.
static int retrieve_resident(pssa_hip_ctx* ctx, const float* d_q_pnc, size_t n_q, const float* d_keys,
                             const float* d_norm_sq, const float* d_values, size_t capacity, size_t count,
                             size_t d_key, size_t d_val, float tau, size_t top_k, float* d_out_val,
                             float* d_out_min, uint32_t* d_out_idx, bool no_alloc, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(n_q && d_key && d_val && capacity, "retrieve: dimensions must be positive"));
    PSSA_RETURN_IF(need(count <= capacity, "retrieve: count exceeds capacity"));
    PSSA_RETURN_IF(need(top_k <= (size_t)pssa::kMaxTopK, "retrieve: top_k must be at most 64"));
    PSSA_RETURN_IF(need(std::isfinite(tau) && tau > 0.0f, "tau must be positive and finite"));
    PSSA_RETURN_IF(need(d_q_pnc && d_keys && d_norm_sq && d_values && d_out_val, "retrieve: null buffer"));
    PSSA_RETURN_IF(need(!d_out_idx || top_k > 0, "retrieve: indices need top_k > 0"));
    if (n_q > INT32_MAX / 4 || d_key > 4096 || d_val > 65536 || capacity > 8192)
      return Status::Invalid("retrieve: shape exceeds the supported range");
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    pssa::RetrieveArgs ra;
    ra.q = d_q_pnc;
    ra.ld_q = (int)d_key;
    ra.project = 0;
    ra.keys = d_keys;
    ra.norm_sq = d_norm_sq;
    ra.values = d_values;
    ra.n = (int)n_q;
    ra.dk = (int)d_key;
    ra.dv = (int)d_val;
    ra.capacity = (int)capacity;
    ra.count = (int)count;
    ra.tau = tau;
    ra.top_k = (int)top_k;
    ra.out_val = d_out_val;
    ra.out_min = d_out_min;
    ra.out_idx = d_out_idx;
    if (no_alloc) {
      ra.chunk = pssa::kNoallocChunk;
      const size_t need_bytes = pssa::retrieve_scratch_bytes(ra);
      if (need_bytes > pssa::kNoallocScratchBytes)
        return Status::Invalid("retrieve (allocation-free): needs " + std::to_string(need_bytes) +
                               " bytes of scratch, the static scratch holds " +
                               std::to_string(pssa::kNoallocScratchBytes));
      if (!ctx->noalloc_scratch) return Status::Device("retrieve (allocation-free): scratch address unresolved");
      ra.scratch = ctx->noalloc_scratch;
      ra.scratch_bytes = pssa::kNoallocScratchBytes;
    } else {
      PSSA_RETURN_IF(bind_retrieve_scratch(ctx, ra));
    }
    return pssa::launch_retrieve(ctx->stream, ra);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_retrieve_resident(pssa_hip_ctx* ctx, const float* d_q_pnc, size_t n_q, const float* d_keys,
                               const float* d_norm_sq, const float* d_values, size_t capacity,
                               size_t count, size_t d_key, size_t d_val, float tau, size_t top_k,
                               float* d_out_val, float* d_out_min, uint32_t* d_out_idx,
                               char* err, size_t err_len) {
  return retrieve_resident(ctx, d_q_pnc, n_q, d_keys, d_norm_sq, d_values, capacity, count, d_key, d_val, tau,
                           top_k, d_out_val, d_out_min, d_out_idx, false, err, err_len);
}

int pssa_hip_retrieve_resident_noalloc(pssa_hip_ctx* ctx, const float* d_q_pnc, size_t n_q, const float* d_keys,
                                       const float* d_norm_sq, const float* d_values, size_t capacity,
                                       size_t count, size_t d_key, size_t d_val, float tau, size_t top_k,
                                       float* d_out_val, float* d_out_min, uint32_t* d_out_idx, char* err,
                                       size_t err_len) {
  return retrieve_resident(ctx, d_q_pnc, n_q, d_keys, d_norm_sq, d_values, capacity, count, d_key, d_val, tau,
                           top_k, d_out_val, d_out_min, d_out_idx, true, err, err_len);
}

// ------------------------------------------------------------------ model
int pssa_hip_model_load(pssa_hip_ctx* ctx, const pssa_hip_weights* w, int weight_dtype,
                        pssa_hip_model** out, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(out != nullptr, "null output handle"));
    *out = nullptr;
    PSSA_RETURN_IF(need(w && w->embed && w->unembed && w->blocks, "weights: null pointer"));
    PSSA_RETURN_IF(need(weight_dtype == PSSA_HIP_F32 || weight_dtype == PSSA_HIP_BF16, "unknown weight dtype"));
    const pssa_hip_config& c = w->cfg;
    PSSA_RETURN_IF(check_config(c));
    const size_t V = c.d_vocab, d = c.d_latent, s = c.d_state, k = c.d_mem_key, C = c.mem_capacity,
                 r = c.adapter_rank;
    for (size_t l = 0; l < c.depth; ++l) {
      const pssa_hip_block& b = w->blocks[l];
      PSSA_RETURN_IF(need(b.norm_gamma && b.norm_beta && b.a_raw && b.w_delta && b.w_b && b.w_c &&
                              b.w_qx && b.w_qh && b.w_gate && b.w_proj && b.adapter_down &&
                              b.adapter_up && b.adapter_slow && b.mlp_w1 && b.mlp_w2 && b.mem_keys &&
                              b.mem_values && b.mem_norm_sq,
                          "weights: null block tensor"));
      PSSA_RETURN_IF(need(b.mem_count <= C, "memory count exceeds capacity"));
      PSSA_RETURN_IF(need(std::isfinite(b.mem_value_cap) && b.mem_value_cap >= 0.0f,
                          "memory value cap must be positive and finite"));
      PSSA_RETURN_IF(need(b.mem_top_k <= (uint64_t)pssa::kMaxTopK, "memory top-k above 64 is not supported"));
      if (b.mem_hybrid_enabled)
        PSSA_RETURN_IF(need(std::isfinite(b.mem_hybrid_lam) && b.mem_hybrid_lam > 0.0f && b.mem_hybrid_lam <= 1.0f,
                            "hybrid decay lam must be in (0.0, 1.0]"));
      if (b.mem_hybrid_gate)
        for (size_t q = 0; q < b.mem_count; ++q)
          PSSA_RETURN_IF(need(std::isfinite(b.mem_hybrid_gate[q]) && b.mem_hybrid_gate[q] >= 0.0f,
                              "hybrid write gate must be finite and nonnegative"));
      for (size_t q = 0; q < b.mem_count; ++q)
        PSSA_RETURN_IF(need(std::isfinite(b.mem_norm_sq[q]) && b.mem_norm_sq[q] >= 0.0f && b.mem_norm_sq[q] < 1.0f,
                            "memory key norms must lie in [0, 1)"));
    }
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    const hipStream_t st = ctx->stream;
    auto m = std::make_unique<pssa_hip_model>();
    m->ctx = ctx;
    m->cfg = c;
    m->dtype = weight_dtype;
    m->n_in = 2 * d + 2 * s + k + r;
    PSSA_RETURN_IF(upload(m->embed, w->embed, V * d * 4, st));
    PSSA_RETURN_IF(upload_weight(m->unembed, w->unembed, V * d, weight_dtype, st));
    m->blocks.resize(c.depth);
    std::vector<float> tmp;
    for (size_t l = 0; l < c.depth; ++l) {
      const pssa_hip_block& b = w->blocks[l];
      pssa::DevBlock& B = m->blocks[l];
      // Fused input projection rows: W_delta | W_B | W_C | W_qx | W_gate | D.
      tmp.assign(m->n_in * d, 0.0f);
      float* p = tmp.data();
      auto put = [&](const float* src, size_t rows) {
        std::memcpy(p, src, rows * d * 4);
        p += rows * d;
      };
      put(b.w_delta, d);
      put(b.w_b, s);
      put(b.w_c, s);
      put(b.w_qx, k);
      put(b.w_gate, d);
      put(b.adapter_down, r);
      PSSA_RETURN_IF(upload_weight(B.w_in, tmp.data(), tmp.size(), weight_dtype, st));
      PSSA_RETURN_IF(upload_weight(B.w_qh, b.w_qh, k * d, weight_dtype, st));
      PSSA_RETURN_IF(upload_weight(B.w_proj, b.w_proj, d * d, weight_dtype, st));
      PSSA_RETURN_IF(upload_weight(B.mlp_w1, b.mlp_w1, 2 * d * d, weight_dtype, st));
      PSSA_RETURN_IF(upload_weight(B.mlp_w2, b.mlp_w2, d * 2 * d, weight_dtype, st));
      std::vector<float> ueff(d * r), rates(d * s), vt(d * C);
      for (size_t i = 0; i < d * r; ++i) ueff[i] = b.adapter_up[i] + b.adapter_slow[i];
      // State-major [s, d] for the scan.
      for (size_t i = 0; i < d; ++i)
        for (size_t j = 0; j < s; ++j) rates[j * d + i] = -softplus_host(b.a_raw[i * s + j]) * 1.4426950408889634f;
      for (size_t q = 0; q < C; ++q)
        for (size_t j = 0; j < d; ++j) vt[j * C + q] = b.mem_values[q * d + j];
      PSSA_RETURN_IF(upload_weight(B.u_eff, ueff.data(), ueff.size(), weight_dtype, st));
      PSSA_RETURN_IF(upload(B.u_fast, b.adapter_up, d * r * 4, st));
      PSSA_RETURN_IF(upload(B.u_slow, b.adapter_slow, d * r * 4, st));
      std::vector<float> conf(C, 1.0f);
      std::vector<unsigned long long> last(C, 0ull);
      if (b.mem_confidence) std::memcpy(conf.data(), b.mem_confidence, C * 4);
      if (b.mem_last_seen)
        for (size_t q = 0; q < C; ++q) last[q] = b.mem_last_seen[q];
      const int meta[2] = {(int)b.mem_count, (int)(b.mem_write_head % C)};
      std::vector<float> hg(C, 1.0f);
      std::vector<unsigned long long> ha(C, 0ull);
      if (b.mem_hybrid_gate) std::memcpy(hg.data(), b.mem_hybrid_gate, C * 4);
      if (b.mem_hybrid_age)
        for (size_t q = 0; q < C; ++q) ha[q] = b.mem_hybrid_age[q];
      B.hybrid = b.mem_hybrid_enabled != 0;
      B.lam = b.mem_hybrid_lam;
      B.top_k = (int)b.mem_top_k;
      B.value_cap = b.mem_value_cap;
      PSSA_RETURN_IF(upload(B.hgate, hg.data(), C * 4, st));
      PSSA_RETURN_IF(upload(B.hage, ha.data(), C * 8, st));
      PSSA_RETURN_IF(upload(B.conf, conf.data(), C * 4, st));
      PSSA_RETURN_IF(upload(B.last_seen, last.data(), C * 8, st));
      PSSA_RETURN_IF(upload(B.meta, meta, sizeof(meta), st));
      PSSA_RETURN_IF(upload(B.rates2, rates.data(), rates.size() * 4, st));
      PSSA_RETURN_IF(upload(B.gamma, b.norm_gamma, d * 4, st));
      PSSA_RETURN_IF(upload(B.beta, b.norm_beta, d * 4, st));
      PSSA_RETURN_IF(upload(B.keys, b.mem_keys, C * k * 4, st));
      PSSA_RETURN_IF(upload(B.norm_sq, b.mem_norm_sq, C * 4, st));
      PSSA_RETURN_IF(upload(B.values, b.mem_values, C * d * 4, st));
      PSSA_RETURN_IF(upload_weight(B.values_t, vt.data(), vt.size(), weight_dtype, st));
      PSSA_RETURN_IF(sync(ctx));  // host staging vectors are reused
      // Values of a capped bank are capped (a no-op for values that were).
      if (B.value_cap > 0.0f) PSSA_RETURN_IF(cap_bank_values(m.get(), {&B}, B.value_cap));
    }
    const unsigned long long step0 = 0;
    PSSA_RETURN_IF(upload(m->step, &step0, 8, st));
    PSSA_RETURN_IF(sync(ctx));
    *out = m.release();
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

void pssa_hip_model_free(pssa_hip_model* model) {
  if (!model) return;
  (void)hipSetDevice(model->ctx->device);
  (void)hipStreamSynchronize(model->ctx->stream);
  delete model;
}

int pssa_hip_lanes_create(pssa_hip_ctx* ctx, const pssa_hip_model* model, size_t lanes,
                          size_t max_tokens, pssa_hip_lanes** out, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(model && out, "null model or output handle"));
    *out = nullptr;
    PSSA_RETURN_IF(need(lanes > 0 && max_tokens >= lanes, "lanes must be positive and max_tokens >= lanes"));
    PSSA_RETURN_IF(need(max_tokens <= (1u << 24), "max_tokens exceeds 2^24"));
    const pssa_hip_config& c = model->cfg;
    const size_t d = c.d_latent, s = c.d_state, k = c.d_mem_key, C = c.mem_capacity;
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    auto L = std::make_unique<pssa_hip_lanes>();
    L->ctx = ctx;
    L->model = model;
    L->lanes = lanes;
    L->max_tokens = max_tokens;
    const size_t n = max_tokens;
    PSSA_RETURN_IF(L->carry.alloc(lanes * c.depth * d * s * 4));
    PSSA_RETURN_IF(L->ids.alloc(n * 4));
    const size_t es = model->dtype == PSSA_HIP_BF16 ? 2 : 4;  // operand element size
    PSSA_RETURN_IF(L->X.alloc(n * d * 4));
    PSSA_RETURN_IF(L->XN.alloc(n * d * 4));
    PSSA_RETURN_IF(L->P.alloc(n * model->n_in * 4));
    PSSA_RETURN_IF(L->Y.alloc(n * d * 4));
    PSSA_RETURN_IF(L->Q.alloc(n * k * 4));
    PSSA_RETURN_IF(L->Zraw.alloc(n * d * 4));
    if (es == 2) {
      PSSA_RETURN_IF(L->XNh.alloc(n * d * 2));
      PSSA_RETURN_IF(L->Yh.alloc(n * d * 2));
      PSSA_RETURN_IF(L->Zrawh.alloc(n * d * 2));
    }
    PSSA_RETURN_IF(L->Wm.alloc(n * C * es));
    PSSA_RETURN_IF(L->Mval.alloc(n * d * es));
    PSSA_RETURN_IF(L->H1.alloc(n * 2 * d * es));
    PSSA_RETURN_IF(L->logits.alloc(lanes * c.d_vocab * 4));
    const int nz = pssa::ssm_state_blocks((int)s);
    if (nz > 2) PSSA_RETURN_IF(L->Ypart.alloc((size_t)nz * n * d * 4));
    PSSA_RETURN_IF(pssa::launch_fill_zero(ctx->stream, L->carry.as<float>(), lanes * c.depth * d * s));
    PSSA_RETURN_IF(L->hist.alloc(lanes * pssa_hip_lanes::kHist * 4));
    PSSA_RETURN_IF(L->hist_n.alloc(lanes * 4));
    PSSA_RETURN_IF(L->hist_pos.alloc(lanes * 4));
    // [0] non-finite logits, [1] non-finite capped bank value, [2] invalid sampling mass
    PSSA_RETURN_IF(L->nonfinite.alloc(16));
    PSSA_RETURN_IF(clear_history(L.get()));
    PSSA_HIP_TRY(hipEventCreateWithFlags(&L->ev_fork, hipEventDisableTiming));
    PSSA_HIP_TRY(hipEventCreateWithFlags(&L->ev_tail_fork, hipEventDisableTiming));
    PSSA_HIP_TRY(hipEventCreateWithFlags(&L->ev_tail_join, hipEventDisableTiming));
    for (int g = 0; g < pssa_hip_lanes::kMaxGroups - 1; ++g) {
      PSSA_HIP_TRY(hipStreamCreateWithFlags(&L->aux_stream[g], hipStreamNonBlocking));
      PSSA_HIP_TRY(hipEventCreateWithFlags(&L->ev_first[g], hipEventDisableTiming));
      PSSA_HIP_TRY(hipEventCreateWithFlags(&L->ev_join[g], hipEventDisableTiming));
    }
    PSSA_RETURN_IF(sync(ctx));
    *out = L.release();
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

void pssa_hip_lanes_free(pssa_hip_lanes* lanes) {
  if (!lanes) return;
  (void)hipSetDevice(lanes->ctx->device);
  (void)hipStreamSynchronize(lanes->ctx->stream);
  delete lanes;
}

int pssa_hip_lanes_reset(pssa_hip_lanes* L, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    const pssa_hip_config& c = L->model->cfg;
    PSSA_RETURN_IF(pssa::launch_fill_zero(L->ctx->stream, L->carry.as<float>(),
                                          L->lanes * c.depth * L->loops * c.d_latent * c.d_state));
    PSSA_RETURN_IF(clear_history(L));
    // No prefill logits to continue from (reset_recurrent_state is followed
    // by a fresh prefill, src/inference.rs:347-355).
    L->logit_lanes = 0;
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_get_carry(pssa_hip_lanes* L, float* out, size_t len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L && out, "null argument"));
    const pssa_hip_config& c = L->model->cfg;
    const size_t n = L->lanes * c.depth * L->loops * c.d_latent * c.d_state;
    PSSA_RETURN_IF(need(len == n, "carry length must be lanes*depth*loops*d_latent*d_state"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    DevBuf tmp;
    PSSA_RETURN_IF(tmp.alloc(n * 4));
    PSSA_RETURN_IF(carry_layout(L, L->carry.as<float>(), tmp.as<float>(), false));
    PSSA_RETURN_IF(download(out, tmp, n * 4, L->ctx->stream));
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_set_carry(pssa_hip_lanes* L, const float* in, size_t len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L && in, "null argument"));
    const pssa_hip_config& c = L->model->cfg;
    const size_t n = L->lanes * c.depth * L->loops * c.d_latent * c.d_state;
    PSSA_RETURN_IF(need(len == n, "carry length must be lanes*depth*loops*d_latent*d_state"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    DevBuf tmp;
    PSSA_RETURN_IF(upload(tmp, in, n * 4, L->ctx->stream));
    PSSA_RETURN_IF(carry_layout(L, tmp.as<float>(), L->carry.as<float>(), true));
    // The prefill logits belong to the replaced carries.
    L->logit_lanes = 0;
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

static Status invalid_prefix_locked(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t T);

int pssa_hip_prefill(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t seq_len,
                     float* logits_last, size_t logits_len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    const size_t V = L->model->cfg.d_vocab;
    if (logits_last) PSSA_RETURN_IF(need(logits_len == n_lanes * V, "logits length must be n_lanes*d_vocab"));
    PSSA_RETURN_IF(need(ids != nullptr, "null ids"));
    PSSA_RETURN_IF(need(seq_len > 0, "prefill requires at least one token"));
    PSSA_RETURN_IF(need(n_lanes > 0 && n_lanes <= L->lanes, "n_lanes must be in 1..=lanes"));
    PSSA_RETURN_IF(need(n_lanes * seq_len <= L->max_tokens, "n_lanes*seq_len exceeds max_tokens"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    PSSA_RETURN_IF(invalid_prefix_locked(L, ids, n_lanes, seq_len));
    PSSA_RETURN_IF(stage_ids_locked(L, ids, n_lanes, seq_len));
    PSSA_RETURN_IF(pssa::run_prefill(L, n_lanes, seq_len));
    L->logit_lanes = n_lanes;
    if (logits_last) PSSA_RETURN_IF(download(logits_last, L->logits, n_lanes * V * 4, L->ctx->stream));
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_forward_inference(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, float* logits,
                               size_t logits_len, char* err, size_t err_len) {
  return pssa_hip_prefill(L, ids, n_lanes, 1, logits, logits_len, err, err_len);
}

// Ragged prefill with L->ctx->mu held: lane i consumes lens[i] ids (0 leaves
// the lane untouched), packed in lane order.  Each lane's last-token logits
// end in row i of lanes->logits (lanes of length 0: undefined).
static Status ragged_locked(pssa_hip_lanes* L, const uint32_t* ids, const uint64_t* lens, size_t n_lanes) {
  const pssa_hip_config& c = L->model->cfg;
  const size_t V = c.d_vocab;
  const hipStream_t st = L->ctx->stream;
  const size_t cw = c.depth * L->loops * c.d_latent * c.d_state;
  size_t tokens = 0;
  for (size_t i = 0; i < n_lanes; ++i) tokens += lens[i];
  if (tokens == 0) return Status::Ok();
  // Lanes in order of decreasing length, so that the lanes still running
  // are always a prefix (the segments of pssa_hip_batch_forward).
  std::vector<size_t> offset(n_lanes), order(n_lanes);
  for (size_t i = 0, o = 0; i < n_lanes; o += lens[i], ++i) offset[i] = o;
  for (size_t i = 0; i < n_lanes; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return lens[a] > lens[b]; });
  size_t n_active = 0;
  while (n_active < n_lanes && lens[order[n_active]] > 0) ++n_active;
  bool identity = true;
  for (size_t i = 0; i < n_active; ++i) identity &= order[i] == i;
  float* carry = L->carry.as<float>();
  float* work = carry;
  if (!identity) {
    if (!L->carry_work.p) PSSA_RETURN_IF(L->carry_work.alloc(L->lanes * cw * 4));
    work = L->carry_work.as<float>();
    for (size_t i = 0; i < n_active; ++i)
      PSSA_HIP_TRY(hipMemcpyAsync(work + i * cw, carry + order[i] * cw, cw * 4, hipMemcpyDeviceToDevice, st));
  }
  std::vector<uint32_t> ids_h(tokens);
  struct Segment {
    size_t T, n_active, row;
  };
  std::vector<Segment> segs;
  size_t t0 = 0, row = 0;
  while (n_active > 0) {
    const size_t t1 = lens[order[n_active - 1]], T = t1 - t0;
    for (size_t i = 0; i < n_active; ++i)
      for (size_t t = 0; t < T; ++t) ids_h[row + i * T + t] = ids[offset[order[i]] + t0 + t];
    segs.push_back({T, n_active, row});
    row += n_active * T;
    t0 = t1;
    while (n_active > 0 && lens[order[n_active - 1]] == t1) --n_active;
  }
  PSSA_HIP_TRY(hipMemcpyAsync(L->ids.p, ids_h.data(), tokens * 4, hipMemcpyHostToDevice, st));
  // Row i of every segment is lane order[i] (its penalty window).
  std::vector<int> map_h(n_lanes);
  for (size_t i = 0; i < n_lanes; ++i) map_h[i] = (int)order[i];
  DevBuf dmap, lg;
  PSSA_RETURN_IF(upload(dmap, map_h.data(), n_lanes * 4, st));
  for (const Segment& sg : segs) {
    pssa::TrainRows rows;
    rows.ids = L->ids.as<uint32_t>() + sg.row;
    rows.carry = work;
    PSSA_RETURN_IF(pssa::run_prefill_segment(L, sg.n_active, sg.T, rows, dmap.as<int>()));
  }
  // Each lane's last logits sit in row (its place in length order); put
  // carries and logits back in lane order.
  if (!identity) {
    PSSA_RETURN_IF(lg.alloc(n_lanes * V * 4));
    for (size_t i = 0; i < n_lanes; ++i) {
      if (lens[order[i]] == 0) continue;
      PSSA_HIP_TRY(hipMemcpyAsync(carry + order[i] * cw, work + i * cw, cw * 4, hipMemcpyDeviceToDevice, st));
      PSSA_HIP_TRY(hipMemcpyAsync(lg.as<float>() + order[i] * V, L->logits.as<float>() + i * V, V * 4,
                                  hipMemcpyDeviceToDevice, st));
    }
    PSSA_HIP_TRY(hipMemcpyAsync(L->logits.p, lg.p, n_lanes * V * 4, hipMemcpyDeviceToDevice, st));
  }
  return sync(L->ctx);  // the staging vectors and buffers above are freed at return
}

// Ids [n_lanes, T] after the reference's rule for invalid ids (src/pssa.rs:
// 2411-2418: every token before the first invalid one is processed, then the
// call fails and leaves the logits alone), with L->ctx->mu held.  Returns
// Ok when every id is valid (nothing run); otherwise advances each lane
// through its valid prefix and returns the error of the first invalid id.
static Status invalid_prefix_locked(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t T) {
  const uint32_t V = (uint32_t)L->model->cfg.d_vocab;
  std::vector<uint64_t> lens(n_lanes);
  bool all = true;
  uint32_t first_bad = 0;
  for (size_t i = 0; i < n_lanes; ++i) {
    size_t v = 0;
    while (v < T && ids[i * T + v] < V) ++v;
    lens[i] = v;
    if (v < T && all) first_bad = ids[i * T + v];
    all &= v == T;
  }
  if (all) return Status::Ok();
  std::vector<uint32_t> packed;
  for (size_t i = 0; i < n_lanes; ++i) packed.insert(packed.end(), ids + i * T, ids + i * T + lens[i]);
  PSSA_RETURN_IF(ragged_locked(L, packed.data(), lens.data(), n_lanes));
  L->staged_lanes = L->staged_len = 0;
  L->logit_lanes = 0;  // no decode continues from a failed prompt
  return Status::Invalid("prompt ID " + std::to_string(first_bad) + " outside model vocabulary");
}

int pssa_hip_prefill_ragged(pssa_hip_lanes* L, const uint32_t* ids, const uint64_t* lens, size_t n_lanes,
                            float* logits_last, size_t logits_len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L && ids && lens, "null argument"));
    PSSA_RETURN_IF(need(n_lanes > 0 && n_lanes <= L->lanes, "n_lanes must be in 1..=lanes"));
    const size_t V = L->model->cfg.d_vocab;
    size_t tokens = 0;
    for (size_t i = 0; i < n_lanes; ++i) {
      PSSA_RETURN_IF(need(lens[i] > 0, "prefill requires at least one token"));
      PSSA_RETURN_IF(need(lens[i] <= L->max_tokens, "the lanes' tokens exceed max_tokens"));
      tokens += lens[i];
    }
    PSSA_RETURN_IF(need(tokens <= L->max_tokens, "the lanes' tokens exceed max_tokens"));
    for (size_t i = 0; i < tokens; ++i)
      if (ids[i] >= V) return Status::Invalid("prompt ID " + std::to_string(ids[i]) + " outside model vocabulary");
    if (logits_last) PSSA_RETURN_IF(need(logits_len == n_lanes * V, "logits length must be n_lanes*d_vocab"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    PSSA_RETURN_IF(ragged_locked(L, ids, lens, n_lanes));
    L->staged_lanes = L->staged_len = 0;  // `ids` holds the packed prompts
    L->logit_lanes = n_lanes;             // decode may continue from these logits
    if (logits_last) PSSA_RETURN_IF(download(logits_last, L->logits, n_lanes * V * 4, L->ctx->stream));
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_prefill_cancellable(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t seq_len,
                                 size_t chunk, pssa_hip_cancel_fn cancelled, void* user, float* logits_last,
                                 size_t logits_len, size_t* processed, char* err, size_t err_len) {
  bool was_cancelled = false;
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr && ids != nullptr, "null argument"));
    PSSA_RETURN_IF(need(seq_len > 0, "prefill requires at least one token"));
    PSSA_RETURN_IF(need(n_lanes > 0 && n_lanes <= L->lanes, "n_lanes must be in 1..=lanes"));
    PSSA_RETURN_IF(need(chunk > 0, "chunk must be positive"));
    const size_t c = std::min(chunk, seq_len);
    PSSA_RETURN_IF(need(n_lanes * c <= L->max_tokens, "n_lanes*chunk exceeds max_tokens"));
    const size_t V = L->model->cfg.d_vocab;
    if (logits_last) PSSA_RETURN_IF(need(logits_len == n_lanes * V, "logits length must be n_lanes*d_vocab"));
    if (processed) *processed = 0;
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    std::vector<uint32_t> part(n_lanes * c);
    for (size_t t0 = 0; t0 < seq_len; t0 += c) {
      // The reference asks before every token (src/pssa.rs:2412-2415); here
      // before every chunk of `chunk` tokens (1: every token).
      if (cancelled && cancelled(user)) {
        was_cancelled = true;
        L->staged_lanes = L->staged_len = 0;
        L->logit_lanes = 0;
        return Status::Ok();
      }
      const size_t T = std::min(c, seq_len - t0);
      for (size_t i = 0; i < n_lanes; ++i)
        std::memcpy(&part[i * T], ids + i * seq_len + t0, T * 4);
      PSSA_RETURN_IF(invalid_prefix_locked(L, part.data(), n_lanes, T));
      PSSA_HIP_TRY(hipMemcpyAsync(L->ids.p, part.data(), n_lanes * T * 4, hipMemcpyHostToDevice, L->ctx->stream));
      PSSA_RETURN_IF(pssa::run_prefill(L, n_lanes, T));
      PSSA_RETURN_IF(sync(L->ctx));  // `part` is refilled next
      if (processed) *processed = t0 + T;
    }
    L->staged_lanes = L->staged_len = 0;  // `ids` holds the last chunk
    L->logit_lanes = n_lanes;
    if (logits_last) PSSA_RETURN_IF(download(logits_last, L->logits, n_lanes * V * 4, L->ctx->stream));
    return sync(L->ctx);
  };
  const int rc = pssa::finish(body(), err, err_len);
  return rc == PSSA_HIP_OK && was_cancelled ? PSSA_HIP_CANCELLED : rc;
}

int pssa_hip_batch_forward(pssa_hip_lanes* L, const pssa_hip_sequence* seqs, size_t n_seqs, float* out_loss,
                           float* token_losses, size_t token_losses_len, float* logits, size_t logits_len,
                           char* err, size_t err_len) {
  auto body = [&]() -> Status {
    // Validation in SequenceBatch::forward's order (src/sequence_batch.rs:243-272),
    // all before any carry changes.
    PSSA_RETURN_IF(need(L && out_loss, "null lanes or loss output"));
    PSSA_RETURN_IF(need(n_seqs >= 1 && n_seqs <= L->lanes && seqs,
                        "sequence count must be between 1 and the configured batch size"));
    const pssa_hip_model* M = L->model;
    const pssa_hip_config& c = M->cfg;
    const size_t V = c.d_vocab;
    if (L->loops != 1)
      return Status{PSSA_HIP_EUNSUPPORTED, "the batched training forward runs one loop here (set_loops 1)"};
    std::vector<char> used(L->lanes, 0);
    size_t tokens = 0;
    for (size_t i = 0; i < n_seqs; ++i) {
      const pssa_hip_sequence& q = seqs[i];
      PSSA_RETURN_IF(need(q.lane < L->lanes && !used[q.lane],
                          "each sequence needs a distinct lane within the configured batch size"));
      used[q.lane] = 1;
      PSSA_RETURN_IF(need(q.inputs && q.targets && q.len > 0 && q.len <= L->max_tokens,
                          "each sequence needs matching nonempty input/target slices no longer than max_tokens"));
      tokens += q.len;
    }
    PSSA_RETURN_IF(need(tokens <= L->max_tokens, "the batch's tokens exceed the lanes' max_tokens"));
    for (size_t i = 0; i < n_seqs; ++i)
      for (size_t t = 0; t < seqs[i].len; ++t)
        if (seqs[i].inputs[t] >= V || seqs[i].targets[t] >= V)
          return Status::Invalid("batch token ID is outside the model vocabulary");
    for (const pssa::DevBlock& B : M->blocks)
      PSSA_RETURN_IF(need(!B.hybrid, "hybrid read currently requires the CPU backend"));
    if (token_losses)
      PSSA_RETURN_IF(need(token_losses_len == tokens, "token_losses length must equal the batch's token count"));
    if (logits) PSSA_RETURN_IF(need(logits_len == tokens * V, "logits length must be tokens*d_vocab"));

    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    const hipStream_t st = L->ctx->stream;
    const size_t cw = c.depth * L->loops * c.d_latent * c.d_state;  // floats of one lane's carry
    if (!L->tok_logits.p) {
      PSSA_RETURN_IF(L->tok_logits.alloc(L->max_tokens * V * 4));
      PSSA_RETURN_IF(L->tok_meta.alloc(2 * L->max_tokens * 4));
      PSSA_RETURN_IF(L->tok_loss.alloc(L->max_tokens * 4));
    }
    L->logit_lanes = 0;  // lanes->logits no longer follows a prefill

    // Packed token offsets in the given order; the device works in order of
    // decreasing length so that the lanes still running are always a prefix.
    std::vector<size_t> offset(n_seqs), order(n_seqs);
    for (size_t i = 0, o = 0; i < n_seqs; o += seqs[i].len, ++i) offset[i] = o;
    for (size_t i = 0; i < n_seqs; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(),
                     [&](size_t a, size_t b) { return seqs[a].len > seqs[b].len; });
    bool identity = true;
    for (size_t i = 0; i < n_seqs; ++i) identity &= seqs[order[i]].lane == i;

    float* carry = L->carry.as<float>();
    for (size_t i = 0; i < n_seqs; ++i)
      if (seqs[i].reset) PSSA_RETURN_IF(pssa::launch_fill_zero(st, carry + seqs[i].lane * cw, cw));
    float* work = carry;
    if (!identity) {
      if (!L->carry_work.p) PSSA_RETURN_IF(L->carry_work.alloc(L->lanes * cw * 4));
      work = L->carry_work.as<float>();
      for (size_t i = 0; i < n_seqs; ++i)
        PSSA_HIP_TRY(hipMemcpyAsync(work + i * cw, carry + seqs[order[i]].lane * cw, cw * 4,
                                    hipMemcpyDeviceToDevice, st));
    }

    // Segments: times [t0, t1) of the n_active longest sequences.
    struct Segment {
      size_t t0, t1, n_active, row;
    };
    std::vector<Segment> segs;
    std::vector<uint32_t> ids_h(tokens), meta_h(2 * tokens);
    size_t n_active = n_seqs, t0 = 0, row = 0;
    while (n_active > 0) {
      const size_t t1 = seqs[order[n_active - 1]].len;
      const size_t T = t1 - t0;
      for (size_t i = 0; i < n_active; ++i) {
        const pssa_hip_sequence& q = seqs[order[i]];
        for (size_t t = 0; t < T; ++t) {
          const size_t r = row + i * T + t;
          ids_h[r] = q.inputs[t0 + t];
          meta_h[r] = q.targets[t0 + t];
          meta_h[tokens + r] = (uint32_t)(offset[order[i]] + t0 + t);
        }
      }
      segs.push_back({t0, t1, n_active, row});
      row += n_active * T;
      t0 = t1;
      while (n_active > 0 && seqs[order[n_active - 1]].len == t1) --n_active;
    }
    PSSA_HIP_TRY(hipMemcpyAsync(L->ids.p, ids_h.data(), tokens * 4, hipMemcpyHostToDevice, st));
    PSSA_HIP_TRY(hipMemcpyAsync(L->tok_meta.p, meta_h.data(), 2 * tokens * 4, hipMemcpyHostToDevice, st));
    const uint32_t* dmeta = L->tok_meta.as<uint32_t>();
    for (const Segment& sg : segs) {
      pssa::TrainRows tr;
      tr.ids = L->ids.as<uint32_t>() + sg.row;
      tr.targets = dmeta + sg.row;
      tr.index = dmeta + tokens + sg.row;
      tr.logits = L->tok_logits.as<float>() + sg.row * V;
      tr.loss = L->tok_loss.as<float>();
      tr.carry = work;
      PSSA_RETURN_IF(pssa::run_train_segment(L, sg.n_active, sg.t1 - sg.t0, tr));
    }
    if (!identity)
      for (size_t i = 0; i < n_seqs; ++i)
        PSSA_HIP_TRY(hipMemcpyAsync(carry + seqs[order[i]].lane * cw, work + i * cw, cw * 4,
                                    hipMemcpyDeviceToDevice, st));

    std::vector<float> loss_h(tokens);
    PSSA_HIP_TRY(hipMemcpyAsync(loss_h.data(), L->tok_loss.p, tokens * 4, hipMemcpyDeviceToHost, st));
    if (logits)
      for (const Segment& sg : segs) {
        const size_t T = sg.t1 - sg.t0;
        for (size_t i = 0; i < sg.n_active; ++i)
          PSSA_HIP_TRY(hipMemcpyAsync(logits + (offset[order[i]] + sg.t0) * V,
                                      L->tok_logits.as<float>() + (sg.row + i * T) * V, T * V * 4,
                                      hipMemcpyDeviceToHost, st));
      }
    PSSA_RETURN_IF(sync(L->ctx));
    // The token mean in packed order, summed left to right in f32
    // (stage_logits_loss, src/gpu_batch.rs:1246-1249).
    float total = 0.0f;
    for (size_t i = 0; i < tokens; ++i) total += loss_h[i];
    const float loss = total / (float)tokens;
    if (token_losses) std::memcpy(token_losses, loss_h.data(), tokens * 4);
    *out_loss = loss;
    if (!std::isfinite(loss)) return Status::Invalid("batch forward: non-finite training loss");
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_stage_ids(pssa_hip_lanes* L, const uint32_t* ids, size_t n_lanes, size_t seq_len,
                             char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    PSSA_RETURN_IF(stage_ids_locked(L, ids, n_lanes, seq_len));
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_prefill_staged(pssa_hip_lanes* L, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    PSSA_RETURN_IF(need(L->staged_len > 0, "no ids staged"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    PSSA_RETURN_IF(pssa::run_prefill(L, L->staged_lanes, L->staged_len));
    L->logit_lanes = L->staged_lanes;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_read_logits(pssa_hip_lanes* L, float* out, size_t len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L && out, "null argument"));
    const size_t n = L->logit_lanes * L->model->cfg.d_vocab;
    PSSA_RETURN_IF(need(n > 0, "no prefill logits to read"));
    PSSA_RETURN_IF(need(len == n, "logits length must be the last prefill's lanes*d_vocab"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    PSSA_RETURN_IF(download(out, L->logits, n * 4, L->ctx->stream));
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_stage_times(pssa_hip_lanes* L, int enable, const char** names, float* ms, size_t cap) {
  if (!L) return PSSA_HIP_EINVAL;
  if (enable >= 0) L->timing = enable != 0;
  size_t n = 0;
  for (int s2 = 0; s2 < pssa::ST_COUNT && n < cap; ++s2) {
    if (names) names[n] = pssa::kStageNames[s2];
    if (ms) ms[n] = L->stage_ms[s2];
    ++n;
  }
  return (int)n;
}

int pssa_hip_model_get_plastic(pssa_hip_model* M, size_t layer, float* adapter_up, float* keys,
                               float* values, float* norm_sq, float* confidence, uint64_t* last_seen,
                               uint64_t* count, uint64_t* write_head, uint64_t* step, char* err,
                               size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(M != nullptr, "null model"));
    const pssa_hip_config& c = M->cfg;
    PSSA_RETURN_IF(need(layer < c.depth, "layer out of range"));
    std::lock_guard<std::mutex> g(M->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(M->ctx->device));
    const hipStream_t st = M->ctx->stream;
    const pssa::DevBlock& B = M->blocks[layer];
    const size_t d = c.d_latent, k = c.d_mem_key, C = c.mem_capacity, r = c.adapter_rank;
    if (adapter_up) PSSA_RETURN_IF(download(adapter_up, B.u_fast, d * r * 4, st));
    if (keys) PSSA_RETURN_IF(download(keys, B.keys, C * k * 4, st));
    if (values) PSSA_RETURN_IF(download(values, B.values, C * d * 4, st));
    if (norm_sq) PSSA_RETURN_IF(download(norm_sq, B.norm_sq, C * 4, st));
    if (confidence) PSSA_RETURN_IF(download(confidence, B.conf, C * 4, st));
    std::vector<unsigned long long> last(C);
    if (last_seen) PSSA_RETURN_IF(download(last.data(), B.last_seen, C * 8, st));
    int meta[2] = {0, 0};
    PSSA_RETURN_IF(download(meta, B.meta, sizeof(meta), st));
    unsigned long long stp = 0;
    PSSA_RETURN_IF(download(&stp, M->step, 8, st));
    PSSA_RETURN_IF(sync(M->ctx));
    if (last_seen)
      for (size_t q = 0; q < C; ++q) last_seen[q] = last[q];
    if (count) *count = (uint64_t)meta[0];
    if (write_head) *write_head = (uint64_t)meta[1];
    if (step) *step = stp;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_model_set_hybrid_read(pssa_hip_model* M, int enabled, float lam, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(M != nullptr, "null model"));
    PSSA_RETURN_IF(need(std::isfinite(lam) && lam > 0.0f && lam <= 1.0f, "hybrid decay lam must be in (0.0, 1.0]"));
    std::lock_guard<std::mutex> g(M->ctx->mu);
    for (auto& B : M->blocks) {
      B.hybrid = enabled != 0;
      B.lam = lam;
    }
    ++M->hybrid_epoch;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_model_set_value_cap(pssa_hip_model* M, float cap, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(M != nullptr, "null model"));
    PSSA_RETURN_IF(need(std::isfinite(cap) && cap >= 0.0f, "memory value cap must be positive and finite"));
    std::lock_guard<std::mutex> g(M->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(M->ctx->device));
    std::vector<pssa::DevBlock*> all;
    for (pssa::DevBlock& B : M->blocks) all.push_back(&B);
    if (cap > 0.0f) PSSA_RETURN_IF(cap_bank_values(M, all, cap));
    for (pssa::DevBlock& B : M->blocks) B.value_cap = cap;
    ++M->hybrid_epoch;  // captured bank writes hold the old cap
    return sync(M->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_model_set_memory_top_k(pssa_hip_model* M, size_t top_k, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(M != nullptr, "null model"));
    PSSA_RETURN_IF(need(top_k <= (size_t)pssa::kMaxTopK, "memory top-k above 64 is not supported"));
    std::lock_guard<std::mutex> g(M->ctx->mu);
    for (pssa::DevBlock& B : M->blocks) B.top_k = (int)top_k;
    ++M->hybrid_epoch;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_model_get_hybrid(pssa_hip_model* M, size_t layer, float* gate, uint64_t* age, char* err,
                              size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(M != nullptr, "null model"));
    PSSA_RETURN_IF(need(layer < M->cfg.depth, "layer out of range"));
    std::lock_guard<std::mutex> g(M->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(M->ctx->device));
    const hipStream_t st = M->ctx->stream;
    const pssa::DevBlock& B = M->blocks[layer];
    const size_t C = M->cfg.mem_capacity;
    if (gate) PSSA_RETURN_IF(download(gate, B.hgate, C * 4, st));
    std::vector<unsigned long long> a(C);
    if (age) PSSA_RETURN_IF(download(a.data(), B.hage, C * 8, st));
    PSSA_RETURN_IF(sync(M->ctx));
    if (age)
      for (size_t q = 0; q < C; ++q) age[q] = a[q];
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

}  // extern "C"

namespace {

// Recurrent depth loops and the hybrid read are not combined on the device.
Status loops_allow_hybrid(const pssa_hip_lanes* L) {
  if (L->loops > 1)
    for (const pssa::DevBlock& B : L->model->blocks)
      if (B.hybrid) return Status{PSSA_HIP_EUNSUPPORTED, "the hybrid read runs one loop here (set_loops 1)"};
  return Status::Ok();
}

Status ensure_decode_buffers(pssa_hip_lanes* L, size_t n_lanes, size_t steps) {
  const pssa_hip_config& c = L->model->cfg;
  if (L->dec_lanes < L->lanes) {
    const size_t n = L->lanes, D = c.depth;
    PSSA_RETURN_IF(L->tap_q.alloc(D * n * c.d_mem_key * 4));
    PSSA_RETURN_IF(L->tap_z.alloc(D * n * c.d_latent * 4));
    PSSA_RETURN_IF(L->tap_a.alloc(D * n * c.d_latent * 4));
    PSSA_RETURN_IF(L->tap_act.alloc(D * n * c.adapter_rank * 4));
    PSSA_RETURN_IF(L->tap_gmean.alloc(D * n * 4));
    PSSA_RETURN_IF(L->tap_zcap.alloc(D * n * c.d_latent * 4));
    PSSA_RETURN_IF(L->surprise.alloc(n * 4));
    PSSA_RETURN_IF(L->hebb_rate.alloc(D * n * 4));  // [depth, lanes]
    PSSA_RETURN_IF(L->bank_writer.alloc(D * c.mem_capacity * 4));
    PSSA_RETURN_IF(L->gen_pos.alloc(4));
    L->dec_lanes = n;
  }
  if (L->gen_cap < steps) {
    const size_t cap = std::max<size_t>(steps, 128);
    PSSA_RETURN_IF(L->gen_ids.alloc(cap * L->lanes * 4));
    L->gen_cap = cap;
    // The captured step holds the old buffer's address.
    if (L->graph_exec) (void)hipGraphExecDestroy(L->graph_exec);
    if (L->graph) (void)hipGraphDestroy(L->graph);
    L->graph_exec = nullptr;
    L->graph = nullptr;
    L->graph_lanes = 0;
  }
  (void)n_lanes;
  return Status::Ok();
}

Status capture_decode_step(pssa_hip_lanes* L, size_t n_lanes, bool plastic) {
  if (L->graph_exec && L->graph_lanes == n_lanes && L->graph_plastic == (plastic ? 1 : 0) &&
      L->graph_hybrid_epoch == L->model->hybrid_epoch && L->graph_penalty == L->rep_penalty &&
      L->graph_temperature == L->temperature && L->graph_top_p == L->top_p && L->graph_top_k == L->top_k)
    return Status::Ok();
  if (L->graph_exec) (void)hipGraphExecDestroy(L->graph_exec);
  if (L->graph) (void)hipGraphDestroy(L->graph);
  L->graph_exec = nullptr;
  L->graph = nullptr;
  const hipStream_t st = L->ctx->stream;
  const bool timing = L->timing;
  L->timing = false;  // no event records inside the graph
  PSSA_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  Status s = pssa::run_decode_step(L, n_lanes, plastic);
  hipGraph_t graph = nullptr;
  const hipError_t e = hipStreamEndCapture(st, &graph);
  L->timing = timing;
  PSSA_RETURN_IF(s);
  if (e != hipSuccess) return Status::Device(std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
  L->graph = graph;
  PSSA_HIP_TRY(hipGraphInstantiate(&L->graph_exec, graph, nullptr, nullptr, 0));
  L->graph_lanes = n_lanes;
  L->graph_plastic = plastic ? 1 : 0;
  L->graph_hybrid_epoch = L->model->hybrid_epoch;
  L->graph_penalty = L->rep_penalty;
  L->graph_temperature = L->temperature;
  L->graph_top_p = L->top_p;
  L->graph_top_k = L->top_k;
  return Status::Ok();
}

}  // namespace

extern "C" {

int pssa_hip_lanes_get_taps(pssa_hip_lanes* L, size_t layer, size_t n_lanes, float* q_pnc, float* z_final,
                            float* ad_out, float* act, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    const pssa_hip_config& c = L->model->cfg;
    PSSA_RETURN_IF(need(L->tap_lanes > 0, "no plastic decode step has recorded taps"));
    PSSA_RETURN_IF(need(n_lanes == L->tap_lanes, "n_lanes must be the last plastic step's lane count"));
    PSSA_RETURN_IF(need(layer < c.depth, "layer out of range"));
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    const hipStream_t st = L->ctx->stream;
    const size_t n = n_lanes, d = c.d_latent, k = c.d_mem_key, r = c.adapter_rank;
    auto part = [&](float* dst, const DevBuf& src, size_t w) -> Status {
      if (!dst) return Status::Ok();
      PSSA_HIP_TRY(hipMemcpyAsync(dst, src.as<float>() + layer * n * w, n * w * 4, hipMemcpyDeviceToHost, st));
      return Status::Ok();
    };
    PSSA_RETURN_IF(part(q_pnc, L->tap_q, k));
    PSSA_RETURN_IF(part(z_final, L->tap_z, d));
    PSSA_RETURN_IF(part(ad_out, L->tap_a, d));
    PSSA_RETURN_IF(part(act, L->tap_act, r));
    return sync(L->ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_set_repetition_penalty(pssa_hip_lanes* L, float penalty, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    PSSA_RETURN_IF(need(std::isfinite(penalty) && penalty >= 1.0f, "repetition penalty must be finite and >= 1"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    L->rep_penalty = penalty;
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_set_loops(pssa_hip_lanes* L, size_t loops, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    PSSA_RETURN_IF(need(loops >= 1 && loops <= 32, "--loops must be between 1 and 32; use --loops 1 for the original model"));
    std::lock_guard<std::mutex> g(L->ctx->mu);
    if (loops == L->loops) return Status::Ok();
    if (loops > 1)
      for (const pssa::DevBlock& B : L->model->blocks)
        if (B.hybrid) return Status{PSSA_HIP_EUNSUPPORTED, "the hybrid read runs one loop here (set_loops 1)"};
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    const hipStream_t st = L->ctx->stream;
    const pssa_hip_config& c = L->model->cfg;
    const size_t hs = c.d_latent * c.d_state, per = L->lanes * c.depth;
    // Loop 0 keeps each block's persistent carry; the other loops start from
    // zero, as resize_loop_tape leaves them (src/pssa.rs:2147-2167).
    DevBuf carry;
    PSSA_RETURN_IF(carry.alloc(per * loops * hs * 4));
    PSSA_RETURN_IF(pssa::launch_fill_zero(st, carry.as<float>(), per * loops * hs));
    PSSA_HIP_TRY(hipMemcpy2DAsync(carry.p, loops * hs * 4, L->carry.p, L->loops * hs * 4, hs * 4, per,
                                  hipMemcpyDeviceToDevice, st));
    if (loops > 1 && !L->Xin.p) PSSA_RETURN_IF(L->Xin.alloc(L->max_tokens * c.d_latent * 4));
    PSSA_RETURN_IF(sync(L->ctx));
    std::swap(L->carry, carry);
    L->loops = loops;
    // The captured step and the prefill logits belong to the old carries.
    if (L->graph_exec) (void)hipGraphExecDestroy(L->graph_exec);
    if (L->graph) (void)hipGraphDestroy(L->graph);
    L->graph_exec = nullptr;
    L->graph = nullptr;
    L->graph_lanes = 0;
    L->logit_lanes = 0;
    L->carry_work = DevBuf();
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_lanes_set_sampling(pssa_hip_lanes* L, float temperature, float top_p, size_t top_k, uint64_t seed,
                                char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    // InferenceConfig validation (src/inference.rs:87-100).
    PSSA_RETURN_IF(need(std::isfinite(temperature) && temperature >= 0.0f, "temperature must be finite and >= 0"));
    PSSA_RETURN_IF(need(std::isfinite(top_p) && top_p > 0.0f && top_p <= 1.0f, "top-p must be finite in (0, 1]"));
    PSSA_RETURN_IF(need(top_k > 0, "top-k must be positive"));
    if (temperature > 0.0f && top_k > 64)
      return Status{PSSA_HIP_EUNSUPPORTED, "sampling on the device supports top-k up to 64"};
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    const hipStream_t st = L->ctx->stream;
    if (temperature > 0.0f) {
      if (!L->rng.p) PSSA_RETURN_IF(L->rng.alloc(L->lanes * 8));
      if (!L->probs.p) PSSA_RETURN_IF(L->probs.alloc(L->lanes * L->model->cfg.d_vocab * 4));
      // SimpleRng::new (src/linalg.rs:7-11): every lane starts from `seed`.
      std::vector<uint64_t> st0(L->lanes, seed == 0 ? 0x853c49e6748fea9bULL : seed);
      PSSA_HIP_TRY(hipMemcpyAsync(L->rng.p, st0.data(), L->lanes * 8, hipMemcpyHostToDevice, st));
      PSSA_RETURN_IF(sync(L->ctx));
    }
    L->temperature = temperature;
    L->top_p = top_p;
    L->top_k = (int)std::min<size_t>(top_k, 64);
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_decode(pssa_hip_lanes* L, const uint32_t* first_ids, size_t n_lanes, size_t steps,
                    int flags, uint32_t* out_ids, size_t out_len, float* logits_last,
                    size_t logits_len, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(need(L != nullptr, "null lanes"));
    PSSA_RETURN_IF(need((flags & ~(PSSA_HIP_DECODE_PLASTIC | PSSA_HIP_DECODE_GRAPH)) == 0, "unknown decode flags"));
    PSSA_RETURN_IF(need(n_lanes > 0 && n_lanes <= L->lanes, "n_lanes must be in 1..=lanes"));
    PSSA_RETURN_IF(need(steps > 0 && steps <= (1u << 20), "steps must be in 1..=2^20"));
    PSSA_RETURN_IF(need(out_ids != nullptr && out_len == steps * n_lanes, "out_ids length must be steps*n_lanes"));
    const size_t V = L->model->cfg.d_vocab;
    if (logits_last) PSSA_RETURN_IF(need(logits_len == n_lanes * V, "logits length must be n_lanes*d_vocab"));
    if (first_ids) {
      for (size_t i = 0; i < n_lanes; ++i)
        if (first_ids[i] >= V)
          return Status::Invalid("prompt ID " + std::to_string(first_ids[i]) + " outside model vocabulary");
    } else {
      PSSA_RETURN_IF(need(L->logit_lanes == n_lanes, "decode without first ids continues the last prefill of n_lanes lanes"));
    }
    const bool plastic = (flags & PSSA_HIP_DECODE_PLASTIC) != 0;
    if (plastic && L->loops != 1)
      return Status{PSSA_HIP_EUNSUPPORTED, "plastic decode runs one loop here (set_loops 1)"};
    // Refused before the choice kernel runs: it records a token and advances
    // every lane's generator.
    PSSA_RETURN_IF(loops_allow_hybrid(L));
    if (plastic) {
      PSSA_RETURN_IF(need(pssa::bank_write_lds((int)L->model->cfg.mem_capacity, (int)n_lanes) <= 160 * 1024,
                          "plastic decode: mem_capacity and n_lanes exceed the bank-write LDS budget"));
      PSSA_RETURN_IF(need(L->model->cfg.adapter_rank <= 256 &&
                              pssa::hebbian_lds((int)L->model->cfg.adapter_rank, (int)n_lanes) <= 160 * 1024,
                          "plastic decode: adapter rank and n_lanes exceed the Hebbian-update LDS budget"));
    }
    std::lock_guard<std::mutex> g(L->ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(L->ctx->device));
    const hipStream_t st = L->ctx->stream;
    PSSA_RETURN_IF(ensure_decode_buffers(L, n_lanes, steps));
    PSSA_RETURN_IF(pssa::launch_fill_zero(st, static_cast<float*>(L->nonfinite.p), 3));
    const int zero = 0;
    PSSA_HIP_TRY(hipMemcpyAsync(L->gen_pos.p, &zero, 4, hipMemcpyHostToDevice, st));
    // After a prefill the first generated token is the choice from its logits
    // (src/inference.rs:367-379), and each later one costs a forward step of
    // the token before it; given first ids, every token costs a step.
    size_t fwd_steps = steps;
    if (first_ids) {
      PSSA_HIP_TRY(hipMemcpyAsync(L->ids.p, first_ids, n_lanes * 4, hipMemcpyHostToDevice, st));
    } else {
      PSSA_RETURN_IF(pssa::run_greedy_from_logits(L, n_lanes, true));
      fwd_steps = steps - 1;
    }
    if (fwd_steps > 0 && (flags & PSSA_HIP_DECODE_GRAPH)) {
      PSSA_RETURN_IF(capture_decode_step(L, n_lanes, plastic));
      for (size_t t = 0; t < fwd_steps; ++t) PSSA_HIP_TRY(hipGraphLaunch(L->graph_exec, st));
    } else {
      for (size_t t = 0; t < fwd_steps; ++t) PSSA_RETURN_IF(pssa::run_decode_step(L, n_lanes, plastic));
    }
    PSSA_RETURN_IF(download(out_ids, L->gen_ids, steps * n_lanes * 4, st));
    if (logits_last) PSSA_RETURN_IF(download(logits_last, L->logits, n_lanes * V * 4, st));
    int nonfinite[3] = {0, 0, 0};
    PSSA_RETURN_IF(download(nonfinite, L->nonfinite, 12, st));
    // The last generated token has not been consumed: a continuation passes
    // it as first_ids.  `ids` now holds the step tokens.
    L->staged_lanes = L->staged_len = 0;
    L->logit_lanes = 0;
    PSSA_RETURN_IF(sync(L->ctx));
    // sample() refuses non-finite logits (src/inference.rs:110-112).
    if (nonfinite[0]) return Status::Invalid("model emitted non-finite logits");
    // clamp_value refuses a non-finite value (src/memory.rs:151-152).
    if (nonfinite[1]) return Status::Invalid("capped memory value must be finite");
    if (nonfinite[2]) return Status::Invalid("invalid sampling probability mass");
    return Status::Ok();
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_dense_scan(pssa_hip_ctx* ctx, const float* a, const float* b, const float* h0,
                        size_t batch, size_t seq_len, size_t d_state, float* h, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(a && b && h, "dense scan: null buffer"));
    PSSA_RETURN_IF(need(batch && seq_len && d_state, "dense scan: dimensions must be positive"));
    PSSA_RETURN_IF(need(d_state <= 64, "dense scan: d_state above 64 is not supported"));
    size_t na = 0, nb = 0;
    PSSA_RETURN_IF(pssa::checked_count({batch, seq_len, d_state, d_state}, &na, "dense scan"));
    PSSA_RETURN_IF(pssa::checked_count({batch, seq_len, d_state}, &nb, "dense scan"));
    if (batch > INT32_MAX || seq_len > INT32_MAX) return Status::Invalid("dense scan: too large");
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    const hipStream_t st = ctx->stream;
    DevBuf da, db, dh0, dh;
    PSSA_RETURN_IF(upload(da, a, na * 4, st));
    PSSA_RETURN_IF(upload(db, b, nb * 4, st));
    if (h0) PSSA_RETURN_IF(upload(dh0, h0, batch * d_state * 4, st));
    PSSA_RETURN_IF(dh.alloc(nb * 4));
    PSSA_RETURN_IF(bind_dense_scan_scratch(ctx, (int)batch, (int)seq_len, (int)d_state));
    PSSA_RETURN_IF(pssa::launch_dense_scan(st, da.as<float>(), db.as<float>(), h0 ? dh0.as<float>() : nullptr,
                                           dh.as<float>(), (int)batch, (int)seq_len, (int)d_state, ctx->scratch,
                                           ctx->scratch_bytes));
    PSSA_RETURN_IF(download(h, dh, nb * 4, st));
    return sync(ctx);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_dense_scan_resident(pssa_hip_ctx* ctx, const float* d_a, const float* d_b,
                                 const float* d_h0, size_t batch, size_t seq_len, size_t d_state,
                                 float* d_h, char* err, size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(d_a && d_b && d_h, "dense scan: null buffer"));
    PSSA_RETURN_IF(need(batch && seq_len && d_state, "dense scan: dimensions must be positive"));
    PSSA_RETURN_IF(need(d_state <= 64, "dense scan: d_state above 64 is not supported"));
    if (batch > INT32_MAX || seq_len > INT32_MAX) return Status::Invalid("dense scan: too large");
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    PSSA_RETURN_IF(bind_dense_scan_scratch(ctx, (int)batch, (int)seq_len, (int)d_state));
    return pssa::launch_dense_scan(ctx->stream, d_a, d_b, d_h0, d_h, (int)batch, (int)seq_len, (int)d_state,
                                   ctx->scratch, ctx->scratch_bytes);
  };
  return pssa::finish(body(), err, err_len);
}

int pssa_hip_dense_scan_reserve(pssa_hip_ctx* ctx, size_t batch, size_t seq_len, size_t d_state, char* err,
                                size_t err_len) {
  auto body = [&]() -> Status {
    PSSA_RETURN_IF(check_ctx(ctx));
    PSSA_RETURN_IF(need(batch && seq_len && d_state, "dense scan: dimensions must be positive"));
    PSSA_RETURN_IF(need(d_state <= 64, "dense scan: d_state above 64 is not supported"));
    if (batch > INT32_MAX || seq_len > INT32_MAX) return Status::Invalid("dense scan: too large");
    std::lock_guard<std::mutex> g(ctx->mu);
    PSSA_HIP_TRY(hipSetDevice(ctx->device));
    return bind_dense_scan_scratch(ctx, (int)batch, (int)seq_len, (int)d_state);
  };
  return pssa::finish(body(), err, err_len);
}

}  // extern "C"

// Shared host/device helpers for libpssa_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/pssa_hip.h"

namespace pssa {

// Error carrier used inside the library; converted to (code, message) at the
// C boundary.
struct Status {
  int code = PSSA_HIP_OK;
  std::string msg;
  bool ok() const { return code == PSSA_HIP_OK; }
  static Status Ok() { return {}; }
  static Status Invalid(const std::string& m) { return {PSSA_HIP_EINVAL, m}; }
  static Status Device(const std::string& m) { return {PSSA_HIP_EDEVICE, m}; }
  static Status NoMem(const std::string& m) { return {PSSA_HIP_ENOMEM, m}; }
  static Status NoDev(const std::string& m) { return {PSSA_HIP_ENODEV, m}; }
};

inline int finish(const Status& s, char* err, size_t err_len) {
  if (err && err_len) {
    if (s.ok()) {
      err[0] = 0;
    } else {
      std::snprintf(err, err_len, "%s", s.msg.c_str());
    }
  }
  return s.code;
}

#define PSSA_RETURN_IF(st) \
  do {                     \
    Status _s = (st);      \
    if (!_s.ok()) return _s; \
  } while (0)

#define PSSA_HIP_TRY(expr)                                                              \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      return Status::Device(std::string(#expr) + ": " + hipGetErrorString(_e));          \
  } while (0)

// Launch check: a failed launch configuration is reported at the call site.
#define PSSA_LAUNCH_CHECK(name)                                                         \
  do {                                                                                  \
    hipError_t _e = hipGetLastError();                                                  \
    if (_e != hipSuccess)                                                               \
      return Status::Device(std::string("launch ") + (name) + ": " + hipGetErrorString(_e)); \
  } while (0)

inline bool mul_ok(size_t a, size_t b, size_t* out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}
inline Status checked_count(std::initializer_list<size_t> dims, size_t* out, const char* what) {
  size_t n = 1;
  for (size_t d : dims)
    if (!mul_ok(n, d, &n)) return Status::Invalid(std::string(what) + ": element count overflow");
  if (n > ((size_t)1 << 40)) return Status::Invalid(std::string(what) + ": too large");
  *out = n;
  return Status::Ok();
}

// Device buffer owned by RAII.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) {
    o.p = nullptr;
    o.bytes = 0;
  }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      release();
      p = o.p;
      bytes = o.bytes;
      o.p = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  Status alloc(size_t n) {
    release();
    n = (n + 255) & ~(size_t)255;  // whole 256-byte granules: fills may round up to a vector
    if (n == 0) n = 256;
    hipError_t e = hipMalloc(&p, n);
    if (e != hipSuccess) {
      p = nullptr;
      (void)hipGetLastError();
      return Status::NoMem("hipMalloc(" + std::to_string(n) + "): " + hipGetErrorString(e));
    }
    bytes = n;
    return Status::Ok();
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// fp32 -> bf16 bits, rounded to nearest even, on gfx950's v_cvt_pk_bf16_f32
// (one instruction per pair; the same bits as the integer rounding
// u + 0x7FFF + lsb for every finite value).
typedef __bf16 bf16x2_cvt_t __attribute__((ext_vector_type(2)));
typedef float f32x2_cvt_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_bits(float lo, float hi) {
  const f32x2_cvt_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_cvt_t));
}
__device__ __forceinline__ uint16_t bf16_bits_dev(float f) { return (uint16_t)bf16x2_bits(f, 0.0f); }

// RMSNorm of one row by one wave (src/pssa.rs:1080-1086).  Lane L holds
// x[4L + 256k .. +3] for k < RMS_V4 (zero past d; d % 4 == 0, rows 16-byte
// aligned); the squares are summed per lane in (k, component) order, then
// across the wave by the xor butterfly.  Every kernel that normalises rows
// (the standalone norm and the decode input product) goes through these two
// functions, so they agree bit for bit.
constexpr int RMS_V4 = 4;  // float4s per lane: rows of up to 1024 columns
__device__ __forceinline__ void rms_load_v4(const float* x, int d, int lane, float4 (&xv)[RMS_V4]) {
#pragma unroll
  for (int k = 0; k < RMS_V4; ++k) {
    const int i = 4 * lane + 256 * k;
    xv[k] = i < d ? *reinterpret_cast<const float4*>(x + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}
// 1 / sqrt(mean square + 1e-5) of each of R rows a wave holds (rms_load_v4):
// per row the same chain, the rows' butterfly steps interleaved so their
// cross-lane exchanges are in flight together.
template <int R>
__device__ __forceinline__ void rms_inv_v4(const float4 (&xv)[R][RMS_V4], int d, float (&inv)[R]) {
  float ss[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    ss[q] = 0.0f;
#pragma unroll
    for (int k = 0; k < RMS_V4; ++k) {
      ss[q] = fmaf(xv[q][k].x, xv[q][k].x, ss[q]);
      ss[q] = fmaf(xv[q][k].y, xv[q][k].y, ss[q]);
      ss[q] = fmaf(xv[q][k].z, xv[q][k].z, ss[q]);
      ss[q] = fmaf(xv[q][k].w, xv[q][k].w, ss[q]);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float o[R];
#pragma unroll
    for (int q = 0; q < R; ++q) o[q] = __shfl_xor(ss[q], off, 64);
#pragma unroll
    for (int q = 0; q < R; ++q) ss[q] += o[q];
  }
#pragma unroll
  for (int q = 0; q < R; ++q) inv[q] = 1.0f / sqrtf(ss[q] / (float)d + 1e-5f);
}
// gamma * (x * inv) + beta, the multiply-add rounded once.
__device__ __forceinline__ float rms_apply(float x, float inv, float g, float b) { return fmaf(g, x * inv, b); }

// s_waitcnt immediate for vmcnt(v) alone (gfx9: vmcnt bits [3:0] and [15:14],
// expcnt and lgkmcnt left at their no-wait maxima).
constexpr int vmcnt_only(int v) { return (v & 0xF) | (((v >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8); }

}  // namespace pssa

// The opaque context handed out through the C ABI.
struct pssa_hip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name;
  int cu_count = 0;
  std::mutex mu;
  // Kernel scratch reused across calls (grown on demand, freed with the
  // context); calls on one context are serialised by `mu` on one stream.
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // Device address of this device's static scratch array (the
  // allocation-free retrieval), resolved when the context is created.
  void* noalloc_scratch = nullptr;
  // Device copies of GEMM weights keyed by (host address, element count,
  // storage dtype), as the reference's CUDA weight cache keys them by
  // (address, length).  A stale entry is uploaded again on its next use.
  struct CachedWeight {
    pssa::DevBuf buf;
    bool current = true;
  };
  std::map<std::tuple<uintptr_t, size_t, int>, CachedWeight> weights;
  // The SSM tape left on the device by pssa_hip_ssm_forward_resident for
  // the next pssa_hip_memory_forward_after_ssm (opaque here).
  std::shared_ptr<struct SsmTape> ssm_tape;
};

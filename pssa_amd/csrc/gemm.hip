// MFMA GEMM for gfx950: C[M,N] = epilogue(A[M,K] * B[N,K]^T).
//
// A holds fp32 activations.  B holds weights, fp32 or bf16:
//   bf16 weights -> v_mfma_f32_32x32x16_bf16 (A is rounded to bf16 as it is
//                   staged in LDS), fp32 accumulation;
//   fp32 weights -> v_mfma_f32_32x32x2_f32, exact fp32 products.
// One 256-thread workgroup computes a 128x128 tile; each of its four waves
// owns a 64x64 quadrant (2x2 MFMA 32x32 tiles, 64 accumulators per lane).
// K advances in LDS-staged slabs, with the next slab prefetched into
// registers while the current one feeds the matrix cores.  Tiles are handed
// out so that each XCD (eight per device, each with its own L2) walks a
// contiguous run of the output, keeping the activation row-panel in one L2.
#include "gemm.h"

namespace pssa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Maps the hardware block id to a tile so that the blocks an XCD receives
// (block ids congruent mod 8) cover one contiguous range of tiles.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
  const int per = total / 8, rem = total % 8;
  const int xcd = bid % 8, idx = bid / 8;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

__device__ __forceinline__ float apply_epilogue(const EpiParams& ep, float acc, int row, int col,
                                                float* __restrict__ C, int ldc) {
  switch (ep.kind) {
    case EPI_STORE:
      return acc;
    case EPI_SCALE:
      return acc * ep.scale;
    case EPI_SEGMENTS: {
      if (col < ep.seg[0]) return softplus_f(acc);
      if (col < ep.seg[1]) return acc;
      if (col < ep.seg[2]) return sigmoid_f(acc);
      if (col < ep.seg[3]) return acc * sigmoid_f(acc);
      return acc;
    }
    case EPI_ADD_AUX:
      return acc + ep.aux[(size_t)row * ep.ld_aux + col];
    case EPI_SILU:
      return acc * sigmoid_f(acc);
    case EPI_ZRAW: {
      // z_raw = (y * ssm_scale) + (g * m_proj) + adapter, in the reference's
      // left-to-right order (src/pssa.rs:1190-1192).
      const float* act = ep.act + (size_t)row * ep.ld_act;
      const float* u = ep.U + (size_t)col * ep.rank;
      float ad = 0.0f;
      for (int r = 0; r < ep.rank; ++r) ad = fmaf(u[r], act[r], ad);
      const float yv = ep.y[(size_t)row * ep.ld_y + col];
      const float gv = ep.g[(size_t)row * ep.ld_g + col];
      return (yv * ep.scale + gv * acc) + ad;
    }
    case EPI_RESIDUAL: {
      // z_final = z_raw + mlp_out; layer 0 publishes it, deeper layers add
      // it with the 1/sqrt(depth) residual scale (src/pssa.rs:2332-2337).
      const float zf = ep.zraw[(size_t)row * ep.ld_zraw + col] + acc;
      if (ep.first) return zf;
      return C[(size_t)row * ldc + col] + ep.scale * zf;
    }
    default:
      return acc;
  }
}

constexpr int BM = 128, BN = 128;

template <bool BF16>
struct Cfg;
template <>
struct Cfg<true> {
  static constexpr int BK = 64;
  static constexpr int LDS_LD = BK + 8;  // bf16 elements; 144-byte rows keep b128 reads conflict-free
  using elem = uint16_t;
};
template <>
struct Cfg<false> {
  static constexpr int BK = 32;
  static constexpr int LDS_LD = BK + 4;  // floats; 144-byte rows
  using elem = float;
};

// VEC: K, lda, ldb are multiples of the vector width and pointers are
// 16-byte aligned, so slabs move as 16-byte vectors.  Otherwise every
// element is loaded with its own bounds check (small or ragged shapes).
template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void gemm_xwt_kernel(const float* __restrict__ A, int lda,
                                                       const void* __restrict__ Bv, int ldb,
                                                       float* __restrict__ C, int ldc, int M,
                                                       int N, int K, EpiParams ep) {
  using CF = Cfg<BF16>;
  using elem = typename CF::elem;
  constexpr int BK = CF::BK, LD = CF::LDS_LD;
  __shared__ __attribute__((aligned(16))) elem sA[BM * LD];
  __shared__ __attribute__((aligned(16))) elem sB[BN * LD];

  const int tilesN = (N + BN - 1) / BN, tilesM = (M + BM - 1) / BM;
  const int tile = xcd_tile(blockIdx.x, tilesM * tilesN);
  const int m0 = (tile / tilesN) * BM, n0 = (tile % tilesN) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- register prefetch of one slab ------------------------------------
  // fp32 A slab: BM x BK floats = BM*BK/4 float4; bf16 mode uses BK=64 so
  // A needs 8 float4 per thread, fp32 mode 4.
  constexpr int A_VEC = BM * BK / 4 / 256;
  constexpr int B_VEC = BF16 ? (BN * BK / 8 / 256) : (BN * BK / 4 / 256);
  float4 ra[A_VEC];
  float4 rb[B_VEC];  // bf16: 8 bf16 bit patterns per float4

  auto load_slab = [&](int k0) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < A_VEC; ++i) {
        const int v = tid + 256 * i;
        const int r = v / (BK / 4), c = (v % (BK / 4)) * 4;
        const int gr = m0 + r, gk = k0 + c;
        ra[i] = (gr < M && gk < K) ? *reinterpret_cast<const float4*>(A + (size_t)gr * lda + gk)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < B_VEC; ++i) {
        const int v = tid + 256 * i;
        if constexpr (BF16) {
          const int r = v / (BK / 8), c = (v % (BK / 8)) * 8;
          const int gn = n0 + r, gk = k0 + c;
          const uint16_t* B = static_cast<const uint16_t*>(Bv);
          rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const float4*>(B + (size_t)gn * ldb + gk)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
          const int r = v / (BK / 4), c = (v % (BK / 4)) * 4;
          const int gn = n0 + r, gk = k0 + c;
          const float* B = static_cast<const float*>(Bv);
          rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const float4*>(B + (size_t)gn * ldb + gk)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_VEC; ++i) {
        const int v = tid + 256 * i;
        const int r = v / (BK / 4), c = (v % (BK / 4)) * 4;
        const int gr = m0 + r;
        float t[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gk = k0 + c + q;
          t[q] = (gr < M && gk < K) ? A[(size_t)gr * lda + gk] : 0.0f;
        }
        ra[i] = make_float4(t[0], t[1], t[2], t[3]);
      }
#pragma unroll
      for (int i = 0; i < B_VEC; ++i) {
        const int v = tid + 256 * i;
        if constexpr (BF16) {
          const int r = v / (BK / 8), c = (v % (BK / 8)) * 8;
          const int gn = n0 + r;
          const uint16_t* B = static_cast<const uint16_t*>(Bv);
          uint16_t t[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int gk = k0 + c + q;
            t[q] = (gn < N && gk < K) ? B[(size_t)gn * ldb + gk] : (uint16_t)0;
          }
          uint32_t w[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) w[q] = (uint32_t)t[2 * q] | ((uint32_t)t[2 * q + 1] << 16);
          rb[i] = make_float4(__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]),
                              __uint_as_float(w[3]));
        } else {
          const int r = v / (BK / 4), c = (v % (BK / 4)) * 4;
          const int gn = n0 + r;
          const float* B = static_cast<const float*>(Bv);
          float t[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int gk = k0 + c + q;
            t[q] = (gn < N && gk < K) ? B[(size_t)gn * ldb + gk] : 0.0f;
          }
          rb[i] = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
    }
  };

  auto store_slab = [&]() {
#pragma unroll
    for (int i = 0; i < A_VEC; ++i) {
      const int v = tid + 256 * i;
      const int r = v / (BK / 4), c = (v % (BK / 4)) * 4;
      if constexpr (BF16) {
        const uint32_t lo = (uint32_t)f32_to_bf16_bits(ra[i].x) | ((uint32_t)f32_to_bf16_bits(ra[i].y) << 16);
        const uint32_t hi = (uint32_t)f32_to_bf16_bits(ra[i].z) | ((uint32_t)f32_to_bf16_bits(ra[i].w) << 16);
        *reinterpret_cast<uint2*>(&sA[r * LD + c]) = make_uint2(lo, hi);
      } else {
        *reinterpret_cast<float4*>(&sA[r * LD + c]) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_VEC; ++i) {
      const int v = tid + 256 * i;
      if constexpr (BF16) {
        const int r = v / (BK / 8), c = (v % (BK / 8)) * 8;
        *reinterpret_cast<float4*>(&sB[r * LD + c]) = rb[i];
      } else {
        const int r = v / (BK / 4), c = (v % (BK / 4)) * 4;
        *reinterpret_cast<float4*>(&sB[r * LD + c]) = rb[i];
      }
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  load_slab(0);
  store_slab();
  __syncthreads();
  const int half = lane >> 5, l32 = lane & 31;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_slab((kt + 1) * BK);
    if constexpr (BF16) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8_t af[2], bf[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int ar = wm * 64 + t * 32 + l32;
          const int br = wn * 64 + t * 32 + l32;
          af[t] = *reinterpret_cast<const bf16x8_t*>(&sA[ar * LD + kk * 16 + half * 8]);
          bf[t] = *reinterpret_cast<const bf16x8_t*>(&sB[br * LD + kk * 16 + half * 8]);
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bf[b], acc[a][b], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < BK / 8; ++kk) {
        float4 af[2], bf[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int ar = wm * 64 + t * 32 + l32;
          const int br = wn * 64 + t * 32 + l32;
          af[t] = *reinterpret_cast<const float4*>(&sA[ar * LD + kk * 8 + half * 4]);
          bf[t] = *reinterpret_cast<const float4*>(&sB[br * LD + kk * 8 + half * 4]);
        }
        // Lane half h contributes k = kk*8 + 4h + q to the q-th product; A and
        // B use the same assignment, so the sum over k is complete.
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b) {
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].x, bf[b].x, acc[a][b], 0, 0, 0);
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].y, bf[b].y, acc[a][b], 0, 0, 0);
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].z, bf[b].z, acc[a][b], 0, 0, 0);
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].w, bf[b].w, acc[a][b], 0, 0, 0);
          }
      }
    }
    __syncthreads();
    if (kt + 1 < nk) {
      store_slab();
      __syncthreads();
    }
  }

  // ---- epilogue: 32x32 accumulator layout, lane l holds column l%32 and
  // rows 8*(i/4) + 4*(l/32) + i%4 of its tile. ------------------------------
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int col = n0 + wn * 64 + b * 32 + l32;
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = m0 + wm * 64 + a * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
        if (row < M) {
          const float v = apply_epilogue(ep, acc[a][b][i], row, col, C, ldc);
          C[(size_t)row * ldc + col] = v;
        }
      }
    }
}

Status launch_gemm_xwt(hipStream_t stream, const float* A, int lda, const void* B, int ldb,
                       int b_dtype, float* C, int ldc, int M, int N, int K, const EpiParams& ep) {
  if (M <= 0 || N <= 0 || K <= 0) return Status::Invalid("gemm: dimensions must be positive");
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const bool bf16 = b_dtype == PSSA_HIP_BF16;
  const int vw = bf16 ? 8 : 4;
  const bool vec = (K % vw == 0) && (lda % 4 == 0) && (ldb % vw == 0) &&
                   ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0);
  dim3 grid(tiles), block(256);
  if (bf16) {
    if (vec)
      gemm_xwt_kernel<true, true><<<grid, block, 0, stream>>>(A, lda, B, ldb, C, ldc, M, N, K, ep);
    else
      gemm_xwt_kernel<true, false><<<grid, block, 0, stream>>>(A, lda, B, ldb, C, ldc, M, N, K, ep);
  } else {
    if (vec)
      gemm_xwt_kernel<false, true><<<grid, block, 0, stream>>>(A, lda, B, ldb, C, ldc, M, N, K, ep);
    else
      gemm_xwt_kernel<false, false><<<grid, block, 0, stream>>>(A, lda, B, ldb, C, ldc, M, N, K, ep);
  }
  PSSA_LAUNCH_CHECK("gemm_xwt");
  return Status::Ok();
}

}  // namespace pssa

// MFMA GEMM for gfx950: C[M,N] = epilogue(A[M,K] * B[N,K]^T).
//
// A holds activations (token rows), B holds weights; both are K-contiguous
// and share one operand type:
//   bf16 -> v_mfma_f32_32x32x16_bf16, fp32 accumulation;
//   fp32 -> v_mfma_f32_32x32x2_f32, exact fp32 products.
//
// A 128-thread workgroup (two waves) computes a 128x128 tile; each wave owns
// 64 token rows x 128 weight rows (2x4 MFMA 32x32 tiles, 128 accumulators
// per lane).  The weights are the MFMA's first operand, so the accumulator
// holds the tile transposed: a lane keeps one token row and runs of four
// consecutive output columns, which the epilogue reads and writes as 16-byte
// vectors.  K advances in LDS-staged slabs; the next slab is prefetched into
// registers while the current one feeds the matrix cores.  Rows are padded
// to an odd multiple of 16 bytes so the fragment reads are bank-conflict
// free.  Tiles are handed out so that each XCD (eight per device, each with
// its own L2) walks a contiguous run of tiles in token-row-major order,
// keeping the activation row panel in one L2.
#include "gemm.h"

namespace pssa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return bf16_bits_dev(f); }
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return bf16x2_bits(lo, hi); }

// ln(u) for finite u >= 1: the hardware log2 times ln 2 taken in two parts
// (ln 2 = C_HI + C_LO), the instruction sequence __logf compiles to for
// normal finite inputs, without its rescaling of denormal inputs and its
// infinity check, which cannot apply here.
__device__ __forceinline__ float ln_ge1(float u) {
#pragma clang fp contract(off)
  constexpr float C_HI = 0x1.62e42ep-1f, C_LO = 0x1.efa39ep-25f;
  const float l2 = __builtin_amdgcn_logf(u);
  const float r = l2 * C_HI;
  const float e = __builtin_fmaf(l2, C_LO, __builtin_fmaf(l2, C_HI, -r));
  return __builtin_fmaf(C_HI, l2, e);
}

// softplus(x) = x > 20 ? x : ln(1 + e^x) (src/linalg.rs:548-551).  ln(1+t) is
// evaluated as ln(u) * t / (u - 1) with u = 1 + t, which cancels the rounding
// of u (relative error a few ulp), and as t - t^2/2 for t < 2^-12.
__device__ __forceinline__ float softplus_f(float x) {
#pragma clang fp contract(off)
  if (x > 20.0f) return x;
  const float t = __expf(x);
  if (t < 2.44140625e-4f) return t - 0.5f * t * t;
  const float u = 1.0f + t;
  return ln_ge1(u) * (t * __builtin_amdgcn_rcpf(u - 1.0f));
}
// sigmoid(x) = 1 / (1 + e^-x) (src/linalg.rs:553-555), with the hardware
// reciprocal (1 ulp).
__device__ __forceinline__ float sigmoid_f(float x) {
#pragma clang fp contract(off)
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// The input projection's column segments (src/pssa.rs:1091-1116): softplus,
// identity, sigmoid, SiLU, identity.  The segment is the same for every
// column a wave holds in practice (the boundaries fall on 32-column tiles at
// the model's shapes), so the branches do not diverge and each element
// evaluates only its own function.
__device__ __forceinline__ float segment_f(const int (&seg)[4], float x, int col) {
#pragma clang fp contract(off)
  if (col < seg[0]) return softplus_f(x);
  if (col < seg[1]) return x;
  if (col < seg[2]) return sigmoid_f(x);
  if (col < seg[3]) return x * sigmoid_f(x);
  return x;
}

// One output element of an epilogue: the accumulator a, the row operands p
// and q of its row and column (z_raw: y and g; add-aux and residual: aux and
// the running out32), the adapter output ad; the tap value goes to tp.
// Every operation rounds on its own (no contraction into fused multiply-
// adds), as the reference evaluates them, so that each kernel's epilogue
// gives the same bits whatever its instruction schedule:
//   z_raw     r = (y * ssm_scale) + (g * m_proj) + adapter, left to right
//             (src/pssa.rs:1190-1192), tap = adapter;
//   residual  z_final = z_raw + mlp_out, tap = z_final; layer 0 publishes it,
//             deeper layers add it with the 1/sqrt(depth) residual scale
//             (src/pssa.rs:2332-2337).
template <int KIND>
__device__ __forceinline__ float epi_value(const EpiParams& ep, float a, float p, float q, float ad, int col,
                                           float& tp) {
#pragma clang fp contract(off)
  tp = 0.0f;
  if constexpr (KIND == EPI_STORE) {
    return a;
  } else if constexpr (KIND == EPI_SCALE) {
    return a * ep.scale;
  } else if constexpr (KIND == EPI_SEGMENTS || KIND == EPI_SEGMENTS_TAP) {
    return segment_f(ep.seg, a, col);
  } else if constexpr (KIND == EPI_ADD_AUX) {
    return a + p;
  } else if constexpr (KIND == EPI_SILU) {
    return a * sigmoid_f(a);
  } else if constexpr (KIND == EPI_ZRAW) {
    tp = ad;
    return (p * ep.scale + q * a) + ad;
  } else {  // EPI_RESIDUAL
    const float zf = p + a;
    tp = zf;
    return ep.first ? zf : q + ep.scale * zf;
  }
}

// Maps the hardware block id to a tile so that the blocks one XCD receives
// (block ids congruent mod 8) cover one contiguous range of tiles.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
  const int per = total / 8, rem = total % 8;
  const int xcd = bid % 8, idx = bid / 8;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

#ifndef PSSA_GEMM_GROUP_M
#define PSSA_GEMM_GROUP_M 8
#endif
// Row and column tile of tile index t: with GROUP_M > 0, groups of GROUP_M
// row panels are walked column by column, so the tiles in flight on one XCD
// share a few row panels and a few weight panels in its L2; 0: row-major.
__device__ __forceinline__ void tile_coords(int t, int tilesM, int tilesN, int& mt, int& nt) {
  constexpr int GM = PSSA_GEMM_GROUP_M;
  if (GM == 0) {
    mt = t / tilesN;
    nt = t % tilesN;
    return;
  }
  const int group = t / (GM * tilesN), first = group * GM;
  const int gs = min(GM, tilesM - first), idx = t - group * GM * tilesN;
  mt = first + idx % gs;
  nt = idx / gs;
}

template <typename T>
struct Op;
template <>
struct Op<uint16_t> {
  static constexpr int BK = 32;  // K per slab
  static constexpr int LD = 40;  // LDS row pitch (elements): 80 bytes
  static constexpr int VE = 8;   // elements per 16-byte vector
};
template <>
struct Op<float> {
  static constexpr int BK = 16;
  static constexpr int LD = 20;
  static constexpr int VE = 4;
};

constexpr int BM = 128, BN = 128, NT = 128;

// Four consecutive columns col..col+3 of one row.  `vec`: all four are in
// range and every operand row is 16-byte aligned at col.
// Row operands an epilogue reads at four consecutive columns (z_raw: y and
// g; add-aux and residual: aux and, for deeper residual layers, the running
// out32).  A tile loads them for all its quads before its first store: the
// operand pointers may alias the outputs, so loads written between the
// stores would each wait out a full memory round trip.
constexpr bool epi_reads(int kind) { return kind == EPI_ZRAW || kind == EPI_ADD_AUX || kind == EPI_RESIDUAL; }

struct QuadIn {
  float4 p, q;
};

template <int KIND>
__device__ __forceinline__ void load_quad(const EpiParams& ep, int row, int col, QuadIn& in) {
  if constexpr (KIND == EPI_ZRAW) {
    in.p = *reinterpret_cast<const float4*>(ep.y + (size_t)row * ep.ld_y + col);
    in.q = *reinterpret_cast<const float4*>(ep.g + (size_t)row * ep.ld_g + col);
  } else if constexpr (KIND == EPI_ADD_AUX || KIND == EPI_RESIDUAL) {
    in.p = *reinterpret_cast<const float4*>(ep.aux + (size_t)row * ep.ld_aux + col);
    in.q = make_float4(0.f, 0.f, 0.f, 0.f);
    if (KIND == EPI_RESIDUAL && !ep.first)
      in.q = *reinterpret_cast<const float4*>(ep.out32 + (size_t)row * ep.ld32 + col);
  }
}

// The epilogue of four consecutive columns col..col+3 of one row.  With `vec`
// all four are in range and every operand row is 16-byte aligned at col: the
// row operands are the ones `in` holds and the stores are vectors.
// Otherwise each column in range is read and written on its own.  The
// arithmetic (epi_value) is the same for both.
template <typename T, int KIND>
__device__ __forceinline__ void epi_quad(const EpiParams& ep, int row, int col, int N, bool vec,
                                         const float (&acc)[4], const float (&ad)[4], const QuadIn& in) {
  float p4[4] = {0.f, 0.f, 0.f, 0.f}, q4[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (epi_reads(KIND)) {
    if (vec) {
      p4[0] = in.p.x, p4[1] = in.p.y, p4[2] = in.p.z, p4[3] = in.p.w;
      q4[0] = in.q.x, q4[1] = in.q.y, q4[2] = in.q.z, q4[3] = in.q.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < N) {
          if constexpr (KIND == EPI_ZRAW) {
            p4[e] = ep.y[(size_t)row * ep.ld_y + col + e];
            q4[e] = ep.g[(size_t)row * ep.ld_g + col + e];
          } else {
            p4[e] = ep.aux[(size_t)row * ep.ld_aux + col + e];
            if (KIND == EPI_RESIDUAL && !ep.first) q4[e] = ep.out32[(size_t)row * ep.ld32 + col + e];
          }
        }
    }
  }
  float r[4], tp[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = epi_value<KIND>(ep, acc[e], p4[e], q4[e], ad[e], col + e, tp[e]);
  constexpr bool tap4 = KIND == EPI_ZRAW || KIND == EPI_RESIDUAL;
  if (vec) {
    if (tap4 && ep.tap)
      *reinterpret_cast<float4*>(ep.tap + (size_t)row * ep.ld_tap + col) = make_float4(tp[0], tp[1], tp[2], tp[3]);
    if (ep.out32)
      *reinterpret_cast<float4*>(ep.out32 + (size_t)row * ep.ld32 + col) = make_float4(r[0], r[1], r[2], r[3]);
    if (ep.out16) {
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(ep.out16) + (size_t)row * ep.ld16 + col) =
            make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
      } else {
        *reinterpret_cast<float4*>(static_cast<float*>(ep.out16) + (size_t)row * ep.ld16 + col) =
            make_float4(r[0], r[1], r[2], r[3]);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (col + e < N) {
        if (tap4 && ep.tap) ep.tap[(size_t)row * ep.ld_tap + col + e] = tp[e];
        if (ep.out32) ep.out32[(size_t)row * ep.ld32 + col + e] = r[e];
        if (ep.out16) {
          if constexpr (sizeof(T) == 2)
            static_cast<uint16_t*>(ep.out16)[(size_t)row * ep.ld16 + col + e] = (uint16_t)f32_to_bf16_bits(r[e]);
          else
            static_cast<float*>(ep.out16)[(size_t)row * ep.ld16 + col + e] = r[e];
        }
      }
  }
  if constexpr (KIND == EPI_SEGMENTS_TAP) {
    // The SiLU segment's columns also go to the adapter-activation tap.
    if (ep.tap)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < N && col + e >= ep.seg[2] && col + e < ep.seg[3])
          ep.tap[(size_t)row * ep.ld_tap + (col + e - ep.seg[2])] = r[e];
  }
}


// Epilogue of one 32x32 accumulator tile whose weight rows start at column
// n32.  Accumulator layout (weights as the MFMA's first operand): lane l
// holds token row `row` (= tile row + l%32) and output columns
// n32 + 8*(i/4) + 4*(l/32) + i%4 for i = 0..15.
// bf16 pairs of the adapter activations act[row, q0 + 8*half .. +7] (zero
// past the rank or the rows): the B fragment of the adapter MFMA.  One row's
// fragment serves every output tile of that row.
__device__ __forceinline__ void adapter_act_frag(const EpiParams& ep, int row, int M, int q0, int half,
                                                 uint32_t (&wa)[4]) {
  const int q = q0 + half * 8;
  const float* src = ep.act + (size_t)row * ep.ld_act + q;
  if (row < M && q + 8 <= ep.rank && ((uintptr_t)src & 15) == 0) {
    const float4 a0 = *reinterpret_cast<const float4*>(src);
    const float4 a1 = *reinterpret_cast<const float4*>(src + 4);
    wa[0] = pack_bf16x2(a0.x, a0.y);
    wa[1] = pack_bf16x2(a0.z, a0.w);
    wa[2] = pack_bf16x2(a1.x, a1.y);
    wa[3] = pack_bf16x2(a1.z, a1.w);
    return;
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float a0 = (row < M && q + 2 * p < ep.rank) ? src[2 * p] : 0.0f;
    const float a1 = (row < M && q + 2 * p + 1 < ep.rank) ? src[2 * p + 1] : 0.0f;
    wa[p] = pack_bf16x2(a0, a1);
  }
}

// bf16 pairs of U[urow, q0 + 8*half .. +7] (zero past the rank or the
// columns): the A fragment of the adapter MFMA for weight row urow.
__device__ __forceinline__ void adapter_u_frag(const EpiParams& ep, int urow, int N, int q0, int half,
                                               uint32_t (&wu)[4]) {
  const int q = q0 + half * 8;
  const uint16_t* us = static_cast<const uint16_t*>(ep.U) + (size_t)urow * ep.rank + q;
  if (urow < N && q + 8 <= ep.rank && ((uintptr_t)us & 15) == 0) {
    const uint4 v = *reinterpret_cast<const uint4*>(us);
    wu[0] = v.x, wu[1] = v.y, wu[2] = v.z, wu[3] = v.w;
    return;
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t u0 = (urow < N && q + 2 * p < ep.rank) ? us[2 * p] : 0u;
    const uint32_t u1 = (urow < N && q + 2 * p + 1 < ep.rank) ? us[2 * p + 1] : 0u;
    wu[p] = u0 | (u1 << 16);
  }
}

// Epilogue of one 32x32 accumulator tile whose weight rows start at column
// n32.  Accumulator layout (weights as the MFMA's first operand): lane l
// holds token row `row` (= tile row + l%32) and output columns
// n32 + 8*(i/4) + 4*(l/32) + i%4 for i = 0..15.  `act0` (bf16 GEMMs with
// the z_raw epilogue, may be null) is the row's adapter fragment for
// q0 = 0, loaded once by the caller for all tiles of the row.
// The row operands of one tile's four quads (see QuadIn).
template <int KIND, bool CLAMP>
__device__ __forceinline__ void epi_tile_load(const EpiParams& ep, int row, int n32, int M, int N,
                                              int vec_epi, int half, QuadIn (&in)[4]) {
  const int nb = n32 + half * 4;
  // CLAMP, with vec_epi (every operand row 16-byte aligned): the quads load
  // from a row clamped to M - 1 and a column clamped to the last aligned
  // in-range quad, unguarded, so all four are in flight together (a load
  // under the per-lane guard ended its block with a full wait).  epi_quad
  // uses a quad only when it is wholly in range.  It costs registers: the
  // tiled kernels take it for z_raw only (the residual tile would drop to
  // three waves per SIMD beside the scan).
  const bool clamp = CLAMP && vec_epi && N >= 4;
  const int rr = min(row, M - 1), cmax = (N - 4) & ~3;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    in[g].p = in[g].q = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (epi_reads(KIND)) {
      const int col = nb + g * 8;
      if (clamp)
        load_quad<KIND>(ep, rr, min(col, cmax), in[g]);
      else if (row < M && vec_epi && col + 3 < N)
        load_quad<KIND>(ep, row, col, in[g]);
    }
  }
}

// Adapter up-projection sum_q U[col,q] * act[row,q] of a z_raw tile on the
// matrix cores, in the same accumulator layout as the main product (zero
// for other epilogues).
template <typename T, int KIND>
__device__ __forceinline__ f32x16_t epi_adapter(const EpiParams& ep, int row, int n32, int M, int N, int half,
                                                int l32, const uint32_t* act0, const uint32_t* u0) {
  f32x16_t adv;
#pragma unroll
  for (int i = 0; i < 16; ++i) adv[i] = 0.0f;
  if constexpr (KIND == EPI_ZRAW) {
    const int urow = n32 + l32;
    if constexpr (sizeof(T) == 2) {
      for (int q0 = 0; q0 < ep.rank; q0 += 16) {
        uint32_t wa[4], wu[4];
        if (q0 == 0 && act0) {
#pragma unroll
          for (int p = 0; p < 4; ++p) wa[p] = act0[p];
        } else {
          adapter_act_frag(ep, row, M, q0, half, wa);
        }
        if (q0 == 0 && u0) {
#pragma unroll
          for (int p = 0; p < 4; ++p) wu[p] = u0[p];
        } else {
          adapter_u_frag(ep, urow, N, q0, half, wu);
        }
        bf16x8_t fa, fu;
        __builtin_memcpy(&fa, wa, 16);
        __builtin_memcpy(&fu, wu, 16);
        adv = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fu, fa, adv, 0, 0, 0);
      }
    } else {
      const float* U = static_cast<const float*>(ep.U);
      for (int q0 = 0; q0 < ep.rank; q0 += 2) {
        const int q = q0 + half;
        const float a = (row < M && q < ep.rank) ? ep.act[(size_t)row * ep.ld_act + q] : 0.0f;
        const float w = (urow < N && q < ep.rank) ? U[(size_t)urow * ep.rank + q] : 0.0f;
        adv = __builtin_amdgcn_mfma_f32_32x32x2f32(w, a, adv, 0, 0, 0);
      }
    }
  }
  return adv;
}

template <typename T, int KIND>
__device__ __forceinline__ void epi_tile_store(const EpiParams& ep, const f32x16_t& acc, int row,
                                               int n32, int M, int N, int vec_epi, int half,
                                               int l32, const uint32_t* act0, const QuadIn (&in)[4],
                                               const uint32_t* u0 = nullptr) {
  const int nb = n32 + half * 4;
  const f32x16_t adv = epi_adapter<T, KIND>(ep, row, n32, M, N, half, l32, act0, u0);
  if (row < M) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = nb + g * 8;
      if (col < N) {
        const float a4[4] = {acc[g * 4 + 0], acc[g * 4 + 1], acc[g * 4 + 2], acc[g * 4 + 3]};
        const float d4[4] = {adv[g * 4 + 0], adv[g * 4 + 1], adv[g * 4 + 2], adv[g * 4 + 3]};
        epi_quad<T, KIND>(ep, row, col, N, vec_epi && col + 3 < N, a4, d4, in[g]);
      }
    }
  }
}

// The epilogue of one 32 x 32 tile of the tiled kernel through the wave's
// 12 KB of LDS `ebuf` (16-byte aligned operand rows, N % 4 == 0, no tap).
// In the accumulator layout a lane holds one row and four 4-column quads, so
// its row-operand loads and its stores would each cover 32 rows x 16 bytes
// per instruction.  Here the row operands (z_raw: y and the gate; add-aux:
// aux; residual: z_raw and the running sum) arrive by direct-to-LDS loads of
// eight whole 128-byte row segments each, every lane reads its quads from
// LDS, and the values go back to LDS and leave as eight whole 128-byte fp32
// (64-byte bf16) row segments per store.  LDS holds [32 rows][8 chunks] of
// 16 bytes with chunk c of row r at slot c ^ (r & 7), so the eight lanes of
// a 16-byte access phase hit eight distinct bank groups.  Rows past M and
// chunks past N load from clamped in-range addresses and are not stored.
// The arithmetic is epi_value's, as in epi_quad.
template <int KIND>
__device__ __forceinline__ void epi_tile_staged(const EpiParams& ep, const f32x16_t& acc, int r0, int n32,
                                                int M, int N, int lane, int half, int l32,
                                                const uint32_t* act0, float* ebuf) {
  constexpr bool reads = epi_reads(KIND);
  const bool has_q = KIND == EPI_ZRAW || (KIND == EPI_RESIDUAL && !ep.first);
  float* pb = ebuf;         // y, aux or the z_raw operand
  float* qb = ebuf + 1024;  // the gate or the running sum
  float* sb = ebuf + 2048;  // the values
  if constexpr (reads) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = i * 8 + (lane >> 3), c = (lane & 7) ^ (r & 7);
      const size_t row = (size_t)min(r0 + r, M - 1);
      const int col = min(n32 + 4 * c, N - 4);
      const float* ps = KIND == EPI_ZRAW ? ep.y + row * ep.ld_y + col : ep.aux + row * ep.ld_aux + col;
      __builtin_amdgcn_global_load_lds((const void*)ps,
                                       (__attribute__((address_space(3))) void*)(pb + 256 * i), 16, 0, 0);
      if (has_q) {
        const float* qs = KIND == EPI_ZRAW ? ep.g + row * ep.ld_g + col : ep.out32 + row * ep.ld32 + col;
        __builtin_amdgcn_global_load_lds((const void*)qs,
                                         (__attribute__((address_space(3))) void*)(qb + 256 * i), 16, 0, 0);
      }
    }
  }
  const f32x16_t adv = epi_adapter<uint16_t, KIND>(ep, r0 + l32, n32, M, N, half, l32, act0, nullptr);
  if constexpr (reads) {
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int pos = 4 * (l32 * 8 + ((half + 2 * g) ^ (l32 & 7)));
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f), q = p;
    if constexpr (reads) {
      p = *reinterpret_cast<const float4*>(pb + pos);
      if (has_q) q = *reinterpret_cast<const float4*>(qb + pos);
    }
    const float p4[4] = {p.x, p.y, p.z, p.w}, q4[4] = {q.x, q.y, q.z, q.w};
    float v[4], tp;
    // Segments: the launch stages a segment epilogue only when every segment
    // boundary falls on a 32-column edge, so the block's first column names
    // the segment of all 32 (a uniform branch, no per-element compare).
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = epi_value<KIND>(ep, acc[g * 4 + e], p4[e], q4[e], adv[g * 4 + e],
                             KIND == EPI_SEGMENTS ? n32 : n32 + half * 4 + g * 8 + e, tp);
    *reinterpret_cast<float4*>(sb + pos) = make_float4(v[0], v[1], v[2], v[3]);
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = i * 8 + (lane >> 3), cs = lane & 7, c = cs ^ (r & 7);
    const float4 v = *reinterpret_cast<const float4*>(sb + 4 * (r * 8 + cs));
    const size_t row = (size_t)(r0 + r);
    if (r0 + r < M && n32 + 4 * c < N) {
      if (ep.out32) *reinterpret_cast<float4*>(ep.out32 + row * ep.ld32 + n32 + 4 * c) = v;
      if (ep.out16)
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(ep.out16) + row * ep.ld16 + n32 + 4 * c) =
            make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    }
  }
  __builtin_amdgcn_wave_barrier();
}

template <typename T, int KIND, bool CLAMP = true>
__device__ __forceinline__ void epilogue_32x32(const EpiParams& ep, const f32x16_t& acc, int row,
                                               int n32, int M, int N, int vec_epi, int half,
                                               int l32, const uint32_t* act0 = nullptr) {
  QuadIn in[4];
  epi_tile_load<KIND, CLAMP>(ep, row, n32, M, N, vec_epi, half, in);
  epi_tile_store<T, KIND>(ep, acc, row, n32, M, N, vec_epi, half, l32, act0, in);
}

template <typename T, int KIND>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(const T* __restrict__ A, int lda,
                                                  const T* __restrict__ B, int ldb, int M, int N,
                                                  int K, int vec_load, int vec_epi, EpiParams ep) {
  constexpr int BK = Op<T>::BK, LD = Op<T>::LD, VE = Op<T>::VE;
  constexpr int CPR = BK / VE;         // 16-byte chunks per slab row
  constexpr int NV = BM * CPR / NT;    // chunks per thread per operand
  static_assert(BM == BN, "both operands share the staging map");
  __shared__ __attribute__((aligned(16))) T sA[BM * LD];
  __shared__ __attribute__((aligned(16))) T sB[BN * LD];

  const int tilesN = (N + BN - 1) / BN, tilesM = (M + BM - 1) / BM;
  const int tile = xcd_tile(blockIdx.x, tilesM * tilesN);
  const int m0 = (tile / tilesN) * BM, n0 = (tile % tilesN) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, l32 = lane & 31;

  float4 ra[NV], rb[NV];
  auto load_slab = [&](int k0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = tid + NT * i;
      const int r = v / CPR, c = (v % CPR) * VE;
      const int gk = k0 + c;
      const int gm = m0 + r, gn = n0 + r;
      if (vec_load) {
        ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const float4*>(A + (size_t)gm * lda + gk)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const float4*>(B + (size_t)gn * ldb + gk)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        T ta[VE], tb[VE];
#pragma unroll
        for (int q = 0; q < VE; ++q) {
          const bool kin = gk + q < K;
          ta[q] = (gm < M && kin) ? A[(size_t)gm * lda + gk + q] : T(0);
          tb[q] = (gn < N && kin) ? B[(size_t)gn * ldb + gk + q] : T(0);
        }
        __builtin_memcpy(&ra[i], ta, 16);
        __builtin_memcpy(&rb[i], tb, 16);
      }
    }
  };
  auto store_slab = [&]() {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = tid + NT * i;
      const int r = v / CPR, c = (v % CPR) * VE;
      *reinterpret_cast<float4*>(&sA[r * LD + c]) = ra[i];
      *reinterpret_cast<float4*>(&sB[r * LD + c]) = rb[i];
    }
  };

  f32x16_t acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][u][i] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  load_slab(0);
  store_slab();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_slab((kt + 1) * BK);
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8_t fa[2], fb[4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
          fa[t] = *reinterpret_cast<const bf16x8_t*>(&sA[(wave * 64 + t * 32 + l32) * LD + kk * 16 + half * 8]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          fb[u] = *reinterpret_cast<const bf16x8_t*>(&sB[(u * 32 + l32) * LD + kk * 16 + half * 8]);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[u], fa[t], acc[t][u], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < BK / 8; ++kk) {
        float4 fa[2], fb[4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
          fa[t] = *reinterpret_cast<const float4*>(&sA[(wave * 64 + t * 32 + l32) * LD + kk * 8 + half * 4]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          fb[u] = *reinterpret_cast<const float4*>(&sB[(u * 32 + l32) * LD + kk * 8 + half * 4]);
        // MFMA q reads k = kk*8 + 4*half + q from lane half `half` of both
        // operands, so the four products cover k = kk*8 .. kk*8+7.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u].x, fa[t].x, acc[t][u], 0, 0, 0);
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u].y, fa[t].y, acc[t][u], 0, 0, 0);
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u].z, fa[t].z, acc[t][u], 0, 0, 0);
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u].w, fa[t].w, acc[t][u], 0, 0, 0);
          }
      }
    }
    __syncthreads();
    if (kt + 1 < nk) {
      store_slab();
      __syncthreads();
    }
  }

  // ---- epilogue ----
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      epilogue_32x32<T, KIND>(ep, acc[t][u], m0 + wave * 64 + t * 32 + l32, n0 + u * 32, M, N, vec_epi,
                              half, l32);
}

// ---------------------------------------------------------------------------
// bf16 GEMM with a direct-to-LDS pipeline (the production path for the model).
//
// A 256-thread workgroup (2x2 waves) computes a 128 x (64*NW) tile; each wave
// owns 64 token rows x 32*NW weight rows.  Operand slabs of 32 K-elements
// move global -> LDS with global_load_lds_dwordx4 (no register staging)
// through a ring of LDS_STAGES slabs, so two slabs are in flight while a
// third feeds the matrix cores.  Slab rows are 64 bytes with the 16-byte
// chunk index XOR-swizzled by ((r>>1) ^ (r>>3)) & 3 (r = row mod 16), which
// keeps the fragment reads bank-conflict free.  Each wave waits for its own
// loads of the slab it is about to read (s_waitcnt vmcnt) and the workgroup
// then meets at a plain s_barrier; the slot refilled next was last read
// before that barrier.  Rows past M or N load a clamped in-range row and
// their results are discarded; K must be a multiple of 32.
constexpr int LDS_BK = 32, LDS_STAGES = 3;

__device__ __forceinline__ int slab_swizzle(int r) { return (((r & 15) >> 1) ^ ((r & 15) >> 3)) & 3; }

template <int KIND, int NW, bool STG = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_lds_kernel(
    const uint16_t* __restrict__ A, int lda, const uint16_t* __restrict__ B, int ldb, int M, int N,
    int K, int vec_epi, EpiParams ep) {
  constexpr int BK = LDS_BK, S = LDS_STAGES;
  constexpr int MT = 2;                 // 32-row MFMA tiles per wave along M
  constexpr int BMt = 64 * MT, BNt = 64 * NW, R = BMt + BNt;
  constexpr int RPI = 16;               // slab rows per DMA instruction (64 lanes x 16 B)
  constexpr int BPW = R / RPI / 4;      // DMA instructions per wave per slab
  static_assert((R / RPI) % 4 == 0, "slab rows must split over four waves");
  // The slab ring is dynamic LDS (gemm_lds_bytes): with a static array the
  // compiler derives an LDS-bound occupancy and pads the VGPR count up to it
  // (100 -> 129), which keeps the tile from sharing a SIMD with a scan.
  extern __shared__ __attribute__((aligned(1024))) uint16_t gemm_lds_smem[];
  auto sm = reinterpret_cast<uint16_t(*)[R * BK]>(gemm_lds_smem);

  const int tilesN = (N + BNt - 1) / BNt, tilesM = (M + BMt - 1) / BMt;
  const int tile = xcd_tile(blockIdx.x, tilesM * tilesN);
  int mt, nt;
  tile_coords(tile, tilesM, tilesN, mt, nt);
  const int m0 = mt * BMt, n0 = nt * BNt;
  // The wave index as a uniform value: the LDS slab addresses and the
  // operand panel bases below are then scalar.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;

  // Source rows of this wave's DMA instructions (row-major slab: A rows then
  // B rows), as a 32-bit byte offset per lane from the tile's row panel in A
  // or weight panel in B (a panel spans at most 128 rows), so that a slab's
  // loads add K to a scalar base and read at a fixed per-lane offset.
  const int lr = lane >> 2, pc = lane & 3;
  const char* const pa = reinterpret_cast<const char*>(A + (size_t)m0 * lda);
  const char* const pb = reinterpret_cast<const char*>(B + (size_t)n0 * ldb);
  uint32_t src_off[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int row = (wave + 4 * i) * RPI + lr;
    const int lc = pc ^ slab_swizzle(row);
    if (row < BMt)
      src_off[i] = (uint32_t)(((size_t)(min(m0 + row, M - 1) - m0) * lda + lc * 8) * 2);
    else
      src_off[i] = (uint32_t)(((size_t)(min(n0 + row - BMt, N - 1) - n0) * ldb + lc * 8) * 2);
  }
  auto issue = [&](int slot, int k0) {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      // Rows below BMt belong to A (wave + 4 i is uniform, so is the choice).
      const char* base = ((wave + 4 * i) * RPI < BMt ? pa : pb) + 2 * (size_t)k0;
      __builtin_amdgcn_global_load_lds(
          (const void*)(base + src_off[i]),
          (__attribute__((address_space(3))) void*)(&sm[slot][((wave + 4 * i) * RPI) * BK]), 16, 0, 0);
    }
  };

  f32x16_t acc[MT][NW];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NW; ++u)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][u][i] = 0.0f;

  const int nk = K / BK;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nk) issue(st, st * BK);
  const int fr = slab_swizzle(l32);
  // The ring slot of slab kt is kt % S: stepping S slabs per outer iteration
  // makes it a constant of each unrolled step, so every fragment address is
  // a per-lane offset plus an immediate.
  for (int kt0 = 0; kt0 < nk; kt0 += S) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int kt = kt0 + j;
      if (kt >= nk) break;
      // Slab kt is complete once at most the slabs issued after it are in flight.
      static_assert(S == 3, "the wait below assumes one slab issued after the current one");
      if (kt + 1 < nk)
        __builtin_amdgcn_s_waitcnt(BPW | (0x7 << 4) | (0xF << 8));  // vmcnt(BPW)
      else
        __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));        // vmcnt(0)
      __builtin_amdgcn_s_barrier();
      if (kt + S - 1 < nk) issue((j + S - 1) % S, (kt + S - 1) * BK);
      const uint16_t* a = sm[j];
      const uint16_t* b = sm[j] + BMt * BK;
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int ch = (kk * 2 + half) ^ fr;
        bf16x8_t fa[MT], fb[NW];
#pragma unroll
        for (int t = 0; t < MT; ++t)
          fa[t] = *reinterpret_cast<const bf16x8_t*>(a + (wm * MT * 32 + t * 32 + l32) * BK + ch * 8);
#pragma unroll
        for (int u = 0; u < NW; ++u)
          fb[u] = *reinterpret_cast<const bf16x8_t*>(b + (wn * NW * 32 + u * 32 + l32) * BK + ch * 8);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int u = 0; u < NW; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[u], fa[t], acc[t][u], 0, 0, 0);
      }
    }
  }

  if constexpr (STG) {
    // Whole tiles: once every wave has read the last slab, each wave stages
    // its tiles' epilogues in its own 12 KB of the ring.
    static_assert(4 * 3 * 1024 * 4 <= S * R * BK * 2, "four 12 KB staging areas fit the ring");
    __syncthreads();
    float* ebuf = reinterpret_cast<float*>(gemm_lds_smem) + wave * 3 * 1024;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r0 = m0 + wm * MT * 32 + t * 32;
      uint32_t act0[4] = {0u, 0u, 0u, 0u};
      if constexpr (KIND == EPI_ZRAW) adapter_act_frag(ep, r0 + l32, M, 0, half, act0);
#pragma unroll
      for (int u = 0; u < NW; ++u)
        epi_tile_staged<KIND>(ep, acc[t][u], r0, n0 + wn * NW * 32 + u * 32, M, N, lane, half, l32, act0, ebuf);
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int row = m0 + wm * MT * 32 + t * 32 + l32;
    uint32_t act0[4] = {0u, 0u, 0u, 0u};
    if constexpr (KIND == EPI_ZRAW) adapter_act_frag(ep, row, M, 0, half, act0);
    // One column tile's operands in flight at a time: loading both tiles'
    // before either stores lifts the z_raw kernel to 186 VGPRs, and the
    // prefill, where a scan workgroup shares the CU, then runs slower.
#pragma unroll
    for (int u = 0; u < NW; ++u)
      epilogue_32x32<uint16_t, KIND, KIND == EPI_ZRAW>(ep, acc[t][u], row, n0 + wn * NW * 32 + u * 32, M, N,
                                                        vec_epi, half, l32, KIND == EPI_ZRAW ? act0 : nullptr);
  }
}

// ---------------------------------------------------------------------------
// bf16 GEMM for few token rows (decode steps, small batches): one wave per
// 32*MT token rows x 32 weight rows, no LDS.  The operand fragments come
// straight from global memory (L2) through a register ring RING K-steps
// deep.  Each output element accumulates its 16-wide K-steps in increasing
// order on the same MFMA as the tiled kernels, so every result is bit-for-bit
// the one those produce; only the tile shape differs, which gives
// (N/32) x (M/(32*MT)) independent waves instead of a handful of 128 x 256
// tiles.  With fp32 activations (TA = float) each fragment is rounded to
// bf16 (nearest even, as launch_to_bf16) in registers when it is consumed, so
// the product equals the one over a separately converted copy.

template <typename TA>
struct SkFrag {  // one lane's 8 K-elements of one token row
  static constexpr int V = sizeof(TA) == 2 ? 1 : 2;  // 16-byte loads
  uint4 v[V];
  __device__ __forceinline__ bf16x8_t bf16() const {
    bf16x8_t f;
    if constexpr (V == 1) {
      __builtin_memcpy(&f, &v[0], 16);
    } else {
      const uint32_t w[4] = {pack_bf16x2(__uint_as_float(v[0].x), __uint_as_float(v[0].y)),
                             pack_bf16x2(__uint_as_float(v[0].z), __uint_as_float(v[0].w)),
                             pack_bf16x2(__uint_as_float(v[1].x), __uint_as_float(v[1].y)),
                             pack_bf16x2(__uint_as_float(v[1].z), __uint_as_float(v[1].w))};
      __builtin_memcpy(&f, w, 16);
    }
    return f;
  }
};

template <int KIND, typename TA, int MT, int RING>
__global__ __launch_bounds__(64) void gemm_skinny_kernel(const TA* __restrict__ A, int lda,
                                                         const uint16_t* __restrict__ B, int ldb, int M,
                                                         int N, int K, int vec_epi, EpiParams ep) {
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32 * MT;
  const TA* pa[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) pa[t] = A + (size_t)min(m0 + 32 * t + l32, M - 1) * lda + 8 * half;
  const uint16_t* pb = B + (size_t)min(n0 + l32, N - 1) * ldb + 8 * half;
  // K % 16 == 0.  The loop is branch-free (prefetches past the end reload
  // the last step and go unused), so the compiler's wait counts stay exact
  // and RING steps of loads remain in flight.
  const int nk = K / 16;
  SkFrag<TA> ra[RING][MT];
  uint4 rb[RING];
  auto fetch = [&](int kt, int slot) {
    const int ko = min(kt, nk - 1) * 16;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int v = 0; v < SkFrag<TA>::V; ++v)
        ra[slot][t].v[v] = *reinterpret_cast<const uint4*>(pa[t] + ko + v * (16 / sizeof(TA)));
    rb[slot] = *reinterpret_cast<const uint4*>(pb + ko);
  };
  f32x16_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  auto step = [&](int q) {
    bf16x8_t fb;
    __builtin_memcpy(&fb, &rb[q], 16);
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb, ra[q][t].bf16(), acc[t], 0, 0, 0);
  };
#pragma unroll
  for (int q = 0; q < RING; ++q) fetch(q, q);
  int k0 = 0;
  for (; k0 + RING <= nk; k0 += RING) {
#pragma unroll
    for (int q = 0; q < RING; ++q) {
      step(q);
      fetch(k0 + RING + q, q);
      // Each slot is refilled right after its MFMA.  Without the barrier the
      // scheduler sank all RING refills below the last step's vmcnt(0), and
      // every RING steps waited out a whole memory round trip.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // The remaining nk - k0 < RING steps are in slots 0 ..
#pragma unroll
  for (int q = 0; q < RING; ++q)
    if (q < nk - k0) step(q);
#pragma unroll
  for (int t = 0; t < MT; ++t)
    epilogue_32x32<uint16_t, KIND>(ep, acc[t], m0 + 32 * t + l32, n0, M, N, vec_epi, half, l32);
}

template <typename TA, int MT, int RING>
static void launch_skinny_kind(hipStream_t stream, int kind, dim3 grid, const TA* A, int lda,
                               const uint16_t* B, int ldb, int M, int N, int K, int ve,
                               const EpiParams& ep) {
#define PSSA_GEMM_SK_CASE(KD)                                                                      \
  case KD:                                                                                         \
    gemm_skinny_kernel<KD, TA, MT, RING><<<grid, 64, 0, stream>>>(A, lda, B, ldb, M, N, K, ve, ep); \
    break;
  switch (kind) {
    PSSA_GEMM_SK_CASE(EPI_STORE)
    PSSA_GEMM_SK_CASE(EPI_SEGMENTS)
    PSSA_GEMM_SK_CASE(EPI_ADD_AUX)
    PSSA_GEMM_SK_CASE(EPI_ZRAW)
    PSSA_GEMM_SK_CASE(EPI_SILU)
    PSSA_GEMM_SK_CASE(EPI_RESIDUAL)
    PSSA_GEMM_SK_CASE(EPI_SCALE)
    PSSA_GEMM_SK_CASE(EPI_SEGMENTS_TAP)
    default:
      break;
  }
#undef PSSA_GEMM_SK_CASE
}

// ---------------------------------------------------------------------------
// bf16 GEMM for few token rows through LDS (decode steps, small batches).
// A workgroup of WM x WN waves computes a (32*WM) x (32*WN) tile with one
// 32 x 32 MFMA tile per wave, so each wave runs a single K chain, as the
// skinny kernel's waves do.  Operand slabs of 64 K-elements (one 128-byte line
// per row) move global -> LDS with global_load_lds_dwordx4, eight lanes per
// row, through a ring of S slabs: every request reads a whole line, where the
// skinny kernel's fragment loads take 32 bytes of 32 lines per instruction.
// A slab row holds its eight 16-byte chunks with chunk c at position
// c ^ ((r >> 1) & 7) (r = slab row), so the 16 lanes of a fragment read that
// share a chunk index fall in distinct banks.  Each output element
// accumulates its 16-wide K-steps in increasing order on
// v_mfma_f32_32x32x16_bf16 with the operands placed as in the tiled kernels,
// so the bits are theirs.  K % 64 == 0; rows past M or N load a clamped
// in-range row and their results are discarded.  The shape: one wave per
// workgroup and four slabs (32 KB, five workgroups per CU) measured fastest
// at 256 rows against 2 x 2, 1 x 2, 2 x 1, 1 x 4 and 4 x 1 waves and 3 or 8
// slabs.
#ifndef PSSA_FEW_WM
#define PSSA_FEW_WM 1
#endif
#ifndef PSSA_FEW_WN
#define PSSA_FEW_WN 1
#endif
#ifndef PSSA_FEW_S
#define PSSA_FEW_S 4
#endif
constexpr int FEW_WM = PSSA_FEW_WM, FEW_WN = PSSA_FEW_WN, FEW_S = PSSA_FEW_S;
constexpr size_t gemm_few_bytes() { return (size_t)FEW_S * 32 * (FEW_WM + FEW_WN) * 128; }

template <int KIND, int WM, int WN, int S>
__global__ __launch_bounds__(64 * WM * WN) void gemm_few_kernel(const uint16_t* __restrict__ A, int lda,
                                                                const uint16_t* __restrict__ B, int ldb,
                                                                int M, int N, int K, int vec_epi,
                                                                EpiParams ep) {
  constexpr int NWV = WM * WN, BMt = 32 * WM, BNt = 32 * WN, R = BMt + BNt;
  constexpr int SLAB = R * 64;      // bf16 elements per slab
  constexpr int BPW = R / 8 / NWV;  // DMA instructions per wave per slab, eight rows each
  static_assert(R % (8 * NWV) == 0, "slab rows must split evenly over the waves");
  // Few-row products are latency-bound chains; in a decode step they share
  // the SIMDs with another lane group's HBM-bound carry update, whose waves
  // keep the default priority (graph replay 1.77 -> 1.75 ms per step).
  __builtin_amdgcn_s_setprio(2);
  static_assert(S >= 2 && (S - 2) * BPW <= 63, "vmcnt holds at most 63");
  extern __shared__ __attribute__((aligned(1024))) uint16_t gemm_few_smem[];

  const int tilesM = (M + BMt - 1) / BMt, tilesN = (N + BNt - 1) / BNt;
  int mt, nt;
  tile_coords(xcd_tile(blockIdx.x, tilesM * tilesN), tilesM, tilesN, mt, nt);
  const int m0 = mt * BMt, n0 = nt * BNt;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int wm = wave / WN, wn = wave % WN;

  // Instruction i of this wave fills slab rows (wave + NWV*i)*8 .. +7: lane L
  // writes position L % 8 of row L / 8 of those, so it loads that row's
  // chunk (L % 8) ^ swizzle.
  // As 32-bit byte offsets from the tile's row panel in A or weight panel
  // in B, so that a slab's loads add K to a scalar base.
  const char* const pa = reinterpret_cast<const char*>(A + (size_t)m0 * lda);
  const char* const pb = reinterpret_cast<const char*>(B + (size_t)n0 * ldb);
  uint32_t src_off[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int row = (wave + NWV * i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    src_off[i] = (uint32_t)(2 * ((row < BMt ? (size_t)(min(m0 + row, M - 1) - m0) * lda
                                            : (size_t)(min(n0 + row - BMt, N - 1) - n0) * ldb) + c * 8));
  }
  const int nk = K / 64;
  // Slabs past the end reload the last one into the slot just read, which
  // no later step reads, so every step waits for the same count.  `slot` is
  // kt % S, a constant at every call.
  auto issue = [&](int kt, int slot) {
    const int k0 = min(kt, nk - 1) * 64;
    uint16_t* dst = gemm_few_smem + slot * SLAB + wave * 8 * 64;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      // Whether instruction i fills A or B rows is the same for every lane.
      const char* base = ((wave + NWV * i) * 8 < BMt ? pa : pb) + 2 * (size_t)k0;
      __builtin_amdgcn_global_load_lds((const void*)(base + src_off[i]),
                                       (__attribute__((address_space(3))) void*)(dst + NWV * i * 8 * 64), 16,
                                       0, 0);
    }
  };

  f32x16_t acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int kt = 0; kt < S - 1; ++kt) issue(kt, kt);
  // The epilogue's row operands (and the z_raw adapter's first fragments)
  // load now, behind the first slabs, rather than after the products.
  const int row = m0 + wm * 32 + l32, n32 = n0 + wn * 32;
  QuadIn in[4];
  epi_tile_load<KIND, true>(ep, row, n32, M, N, vec_epi, half, in);
  uint32_t act0[4] = {0u, 0u, 0u, 0u}, u0[4] = {0u, 0u, 0u, 0u};
  if constexpr (KIND == EPI_ZRAW) {
    adapter_act_frag(ep, row, M, 0, half, act0);
    adapter_u_frag(ep, n32 + l32, N, 0, half, u0);
  }
  const int ra = wm * 32 + l32, rb = BMt + wn * 32 + l32;  // slab rows of this lane's fragments
  const int sa = (ra >> 1) & 7, sb = (rb >> 1) & 7;
  // S slabs per outer step, so each step's ring slot is a constant.
  for (int kt0 = 0; kt0 < nk; kt0 += S) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int kt = kt0 + j;
      if (kt >= nk) break;
      // This wave's part of slab kt has landed once at most the S - 2 slabs
      // issued after it are in flight; the barrier then covers every wave's
      // part, and every wave has finished reading the slot refilled next.
      __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 2) * BPW));
      __builtin_amdgcn_s_barrier();
      issue(kt + S - 1, (j + S - 1) % S);
      const uint16_t* sl = gemm_few_smem + j * SLAB;
      // All eight fragments of the slab are read before the first product,
      // so one LDS round trip precedes the four dependent MFMAs rather than
      // each.
      bf16x8_t fa[4], fb[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int c = 2 * kk + half;
        fa[kk] = *reinterpret_cast<const bf16x8_t*>(sl + ra * 64 + (c ^ sa) * 8);
        fb[kk] = *reinterpret_cast<const bf16x8_t*>(sl + rb * 64 + (c ^ sb) * 8);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[kk], fa[kk], acc, 0, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // the reloads past the end
  epi_tile_store<uint16_t, KIND>(ep, acc, row, n32, M, N, vec_epi, half, l32,
                                 KIND == EPI_ZRAW ? act0 : nullptr, in, KIND == EPI_ZRAW ? u0 : nullptr);
}

static void launch_few_kind(hipStream_t stream, int kind, unsigned blocks, const uint16_t* A, int lda,
                            const uint16_t* B, int ldb, int M, int N, int K, int ve, const EpiParams& ep) {
#define PSSA_GEMM_FEW_CASE(KD)                                                                 \
  case KD:                                                                                     \
    gemm_few_kernel<KD, FEW_WM, FEW_WN, FEW_S>                                                 \
        <<<blocks, 64 * FEW_WM * FEW_WN, gemm_few_bytes(), stream>>>(A, lda, B, ldb, M, N, K, ve, ep); \
    break;
  switch (kind) {
    PSSA_GEMM_FEW_CASE(EPI_STORE)
    PSSA_GEMM_FEW_CASE(EPI_SEGMENTS)
    PSSA_GEMM_FEW_CASE(EPI_ADD_AUX)
    PSSA_GEMM_FEW_CASE(EPI_ZRAW)
    PSSA_GEMM_FEW_CASE(EPI_SILU)
    PSSA_GEMM_FEW_CASE(EPI_RESIDUAL)
    PSSA_GEMM_FEW_CASE(EPI_SCALE)
    PSSA_GEMM_FEW_CASE(EPI_SEGMENTS_TAP)
    default:
      break;
  }
#undef PSSA_GEMM_FEW_CASE
}

// fp32 GEMM for few token rows: one wave per 32*MT token rows x 32 weight
// rows, operand fragments straight from global memory through a register
// ring of RING 8-deep K steps.  A lane holds the four K values
// k0 + 4*half .. +3 of its row of each operand, and MFMA q of a step sums the
// pair (k0 + q, k0 + 4 + q): the v_mfma_f32_32x32x2f32 sequence of
// gemm_kernel<float> for every output element, so both give the same bits
// (K % 16 == 0: the tiled kernel's zero-padded last slab adds nothing).
template <int KIND, int MT, int RING>
__global__ __launch_bounds__(64) void gemm_skinny_f32_kernel(const float* __restrict__ A, int lda,
                                                             const float* __restrict__ B, int ldb, int M, int N,
                                                             int K, int vec_epi, EpiParams ep) {
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32 * MT;
  const float* pa[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) pa[t] = A + (size_t)min(m0 + 32 * t + l32, M - 1) * lda + 4 * half;
  const float* pb = B + (size_t)min(n0 + l32, N - 1) * ldb + 4 * half;
  // Branch-free loop: prefetches past the end reload the last step and go
  // unused, so the compiler's wait counts stay partial.
  const int nk = K / 8;
  float4 ra[RING][MT], rb[RING];
  auto fetch = [&](int kt, int slot) {
    const int ko = min(kt, nk - 1) * 8;
#pragma unroll
    for (int t = 0; t < MT; ++t) ra[slot][t] = *reinterpret_cast<const float4*>(pa[t] + ko);
    rb[slot] = *reinterpret_cast<const float4*>(pb + ko);
  };
  f32x16_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
  auto step = [&](int q) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(rb[q].x, ra[q][t].x, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(rb[q].y, ra[q][t].y, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(rb[q].z, ra[q][t].z, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(rb[q].w, ra[q][t].w, acc[t], 0, 0, 0);
    }
  };
#pragma unroll
  for (int q = 0; q < RING; ++q) fetch(q, q);
  int k0 = 0;
  for (; k0 + RING <= nk; k0 += RING) {
#pragma unroll
    for (int q = 0; q < RING; ++q) {
      step(q);
      fetch(k0 + RING + q, q);
      __builtin_amdgcn_sched_barrier(0);  // refill right after the step, as above
    }
  }
#pragma unroll
  for (int q = 0; q < RING; ++q)
    if (q < nk - k0) step(q);
#pragma unroll
  for (int t = 0; t < MT; ++t)
    epilogue_32x32<float, KIND>(ep, acc[t], m0 + 32 * t + l32, n0, M, N, vec_epi, half, l32);
}

template <int MT, int RING>
static void launch_skinny_f32_kind(hipStream_t stream, int kind, dim3 grid, const float* A, int lda,
                                   const float* B, int ldb, int M, int N, int K, int ve, const EpiParams& ep) {
#define PSSA_GEMM_SKF_CASE(KD)                                                                    \
  case KD:                                                                                        \
    gemm_skinny_f32_kernel<KD, MT, RING><<<grid, 64, 0, stream>>>(A, lda, B, ldb, M, N, K, ve, ep); \
    break;
  switch (kind) {
    PSSA_GEMM_SKF_CASE(EPI_STORE)
    PSSA_GEMM_SKF_CASE(EPI_SEGMENTS)
    PSSA_GEMM_SKF_CASE(EPI_ADD_AUX)
    PSSA_GEMM_SKF_CASE(EPI_ZRAW)
    PSSA_GEMM_SKF_CASE(EPI_SILU)
    PSSA_GEMM_SKF_CASE(EPI_RESIDUAL)
    PSSA_GEMM_SKF_CASE(EPI_SCALE)
    PSSA_GEMM_SKF_CASE(EPI_SEGMENTS_TAP)
    default:
      break;
  }
#undef PSSA_GEMM_SKF_CASE
}

template <typename T>
static void launch_kind(hipStream_t stream, int kind, dim3 grid, const T* A, int lda, const T* B,
                        int ldb, int M, int N, int K, int vl, int ve, const EpiParams& ep) {
#define PSSA_GEMM_CASE(KD)                                                                   \
  case KD:                                                                                   \
    gemm_kernel<T, KD><<<grid, NT, 0, stream>>>(A, lda, B, ldb, M, N, K, vl, ve, ep); \
    break;
  switch (kind) {
    PSSA_GEMM_CASE(EPI_STORE)
    PSSA_GEMM_CASE(EPI_SEGMENTS)
    PSSA_GEMM_CASE(EPI_ADD_AUX)
    PSSA_GEMM_CASE(EPI_ZRAW)
    PSSA_GEMM_CASE(EPI_SILU)
    PSSA_GEMM_CASE(EPI_RESIDUAL)
    PSSA_GEMM_CASE(EPI_SCALE)
    PSSA_GEMM_CASE(EPI_SEGMENTS_TAP)
    default:
      break;
  }
#undef PSSA_GEMM_CASE
}

// Bytes of the slab ring of a gemm_lds_kernel<*, NW> workgroup.
constexpr size_t gemm_lds_bytes(int nw) { return (size_t)LDS_STAGES * (128 + 64 * nw) * LDS_BK * 2; }

template <int NW>
static void launch_lds_kind(hipStream_t stream, int kind, dim3 grid, const uint16_t* A, int lda,
                            const uint16_t* B, int ldb, int M, int N, int K, int ve,
                            const EpiParams& ep) {
  constexpr size_t lds = gemm_lds_bytes(NW);
  static_assert(lds <= 64 * 1024, "the ring fits the default dynamic LDS limit");
  // 128 x 128 tiles stage their epilogues through LDS (epi_tile_staged):
  // vector operands, N % 4 == 0, no tap, and segment boundaries on 32-column
  // edges (or at N and past it).
  bool seg32 = true;
  for (int i = 0; i < 4; ++i) seg32 = seg32 && (ep.seg[i] % 32 == 0 || ep.seg[i] >= N);
  const bool stg = NW == 2 && ve && N % 4 == 0 && !ep.tap && (kind != EPI_SEGMENTS || seg32);
#define PSSA_GEMM_LDS_CASE(KD)                                                                        \
  case KD:                                                                                            \
    if (stg && KD != EPI_SEGMENTS_TAP)                                                                \
      gemm_lds_kernel<KD, NW, NW == 2 && KD != EPI_SEGMENTS_TAP><<<grid, 256, lds, stream>>>(         \
          A, lda, B, ldb, M, N, K, ve, ep);                                                           \
    else                                                                                              \
      gemm_lds_kernel<KD, NW><<<grid, 256, lds, stream>>>(A, lda, B, ldb, M, N, K, ve, ep);          \
    break;
  switch (kind) {
    PSSA_GEMM_LDS_CASE(EPI_STORE)
    PSSA_GEMM_LDS_CASE(EPI_SEGMENTS)
    PSSA_GEMM_LDS_CASE(EPI_ADD_AUX)
    PSSA_GEMM_LDS_CASE(EPI_ZRAW)
    PSSA_GEMM_LDS_CASE(EPI_SILU)
    PSSA_GEMM_LDS_CASE(EPI_RESIDUAL)
    PSSA_GEMM_LDS_CASE(EPI_SCALE)
    PSSA_GEMM_LDS_CASE(EPI_SEGMENTS_TAP)
    default:
      break;
  }
#undef PSSA_GEMM_LDS_CASE
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Checks the epilogue operands; `vec_epi` tells whether every row operand is
// 16-byte aligned at multiples of 4 columns (vector epilogue).
static Status check_epilogue(const EpiParams& ep, bool bf16, int& vec_epi) {
  if (ep.kind < 0 || ep.kind >= EPI_KINDS) return Status::Invalid("gemm: unknown epilogue");
  if (!ep.out32 && !ep.out16) return Status::Invalid("gemm: no output");
  if (ep.kind == EPI_RESIDUAL && !ep.out32) return Status::Invalid("gemm: residual needs the fp32 output");
  if (ep.kind == EPI_ZRAW && (!ep.y || !ep.g || (ep.rank > 0 && (!ep.act || !ep.U))))
    return Status::Invalid("gemm: z_raw epilogue operands missing");
  bool v = true;
  auto chk32 = [&](const float* p, int ld) {
    if (p) v = v && al16(p) && ld % 4 == 0;
  };
  chk32(ep.out32, ep.ld32);
  chk32(ep.aux, ep.ld_aux);
  chk32(ep.y, ep.ld_y);
  chk32(ep.g, ep.ld_g);
  chk32(ep.tap, ep.ld_tap);
  if (ep.out16) v = v && ((uintptr_t)ep.out16 % (bf16 ? 8 : 16) == 0) && ep.ld16 % 4 == 0;
  vec_epi = v ? 1 : 0;
  return Status::Ok();
}

// ---------------------------------------------------------------------------
// The decode step's input product with the block's RMSNorm folded in: a
// workgroup of four waves owns 32 token rows x 128 weight rows.  Each wave
// normalises 8 of the rows (rms_inv_v4 / rms_apply, the standalone norm's
// arithmetic), writes their bf16 values into an LDS panel of the 32 whole
// rows (chunk c of row r at c ^ (r & 15), conflict-free fragment reads) and,
// in the first column tile, the fp32 rows to XN for the scan; the weight
// slabs stream through the few-row kernel's direct-to-LDS ring meanwhile.
// Each wave then runs one 32 x 32 tile's K chain (the tiled kernels' MFMA
// order), so the result equals rmsnorm followed by the product bit for bit.
// d % 128 == 0, d <= 256 * RMS_V4.
constexpr int NORM_BN = 128;
size_t gemm_norm_bytes(int d) { return (size_t)FEW_S * NORM_BN * 128 + (size_t)32 * d * 2; }

template <int KIND>
__global__ __launch_bounds__(256) void gemm_norm_kernel(const float* __restrict__ X, int d,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, float* __restrict__ XN,
                                                        const uint16_t* __restrict__ B, int ldb, int M, int N,
                                                        int vec_epi, EpiParams ep) {
  constexpr int NWV = 4, S = FEW_S, SLAB = NORM_BN * 64, BPW = NORM_BN / 8 / NWV;
  static_assert(S >= 2 && (S - 2) * BPW <= 63, "vmcnt holds at most 63");
  extern __shared__ __attribute__((aligned(1024))) uint16_t gemm_norm_smem[];
  __builtin_amdgcn_s_setprio(2);  // as gemm_few_kernel: a decode-step product
  uint16_t* panel = gemm_norm_smem + S * SLAB;  // [32][d] bf16, swizzled

  const int tilesM = (M + 31) / 32, tilesN = (N + NORM_BN - 1) / NORM_BN;
  int mt, nt;
  tile_coords(xcd_tile(blockIdx.x, tilesM * tilesN), tilesM, tilesN, mt, nt);
  const int m0 = mt * 32, n0 = nt * NORM_BN;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, l32 = lane & 31;

  // Weight rows as 32-bit byte offsets from the tile's weight panel, so that
  // a slab's loads add K to a scalar base; `slot` is kt % S, a constant at
  // every call.
  const char* const pb = reinterpret_cast<const char*>(B + (size_t)n0 * ldb);
  uint32_t src_off[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int row = (wave + NWV * i) * 8 + (lane >> 3);
    src_off[i] = (uint32_t)(2 * ((size_t)(min(n0 + row, N - 1) - n0) * ldb + ((lane & 7) ^ ((row >> 1) & 7)) * 8));
  }
  const int nk = d / 64;
  auto issue = [&](int kt, int slot) {
    const int k0 = min(kt, nk - 1) * 64;
    uint16_t* dst = gemm_norm_smem + slot * SLAB + wave * 8 * 64;
#pragma unroll
    for (int i = 0; i < BPW; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pb + 2 * (size_t)k0 + src_off[i]),
                                       (__attribute__((address_space(3))) void*)(dst + NWV * i * 8 * 64), 16,
                                       0, 0);
  };
#pragma unroll
  for (int kt = 0; kt < S - 1; ++kt) issue(kt, kt);

  // The normalised rows: wave w takes tile rows 8w .. 8w + 7.
  float4 g[RMS_V4], bt[RMS_V4];
#pragma unroll
  for (int k = 0; k < RMS_V4; ++k) {
    const int i = 4 * lane + 256 * k;
    g[k] = i < d ? *reinterpret_cast<const float4*>(gamma + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    bt[k] = i < d ? *reinterpret_cast<const float4*>(beta + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // All eight rows' loads are in flight together (one round trip); the
  // workgroup's LDS holds one workgroup per CU, so the registers are there.
  {
    constexpr int r0 = 0;
    float4 xv[8][RMS_V4];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      rms_load_v4(X + (size_t)min(m0 + wave * 8 + r0 + q, M - 1) * d, d, lane, xv[q]);
    float inv8[8];
    rms_inv_v4<8>(xv, d, inv8);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int r = wave * 8 + r0 + q;
      const float inv = inv8[q];
#pragma unroll
      for (int k = 0; k < RMS_V4; ++k) {
        const int i = 4 * lane + 256 * k;
        if (i < d) {
          const float4 x4 = xv[q][k];
          const float4 v =
              make_float4(rms_apply(x4.x, inv, g[k].x, bt[k].x), rms_apply(x4.y, inv, g[k].y, bt[k].y),
                          rms_apply(x4.z, inv, g[k].z, bt[k].z), rms_apply(x4.w, inv, g[k].w, bt[k].w));
          if (nt == 0 && m0 + r < M) *reinterpret_cast<float4*>(XN + (size_t)(m0 + r) * d + i) = v;
          const int c = i >> 3;
          *reinterpret_cast<uint2*>(panel + (size_t)r * d + (c ^ (r & 15)) * 8 + (i & 4)) =
              make_uint2(bf16x2_bits(v.x, v.y), bf16x2_bits(v.z, v.w));
        }
      }
    }
  }
  __syncthreads();

  f32x16_t acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  const uint16_t* prow = panel + (size_t)l32 * d;
  const int sp = l32 & 15, rb = wave * 32 + l32, sb = (rb >> 1) & 7;
  // S slabs per outer step, so each step's ring slot is a constant.
  for (int kt0 = 0; kt0 < nk; kt0 += S) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int kt = kt0 + j;
      if (kt >= nk) break;
      __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 2) * BPW));
      __builtin_amdgcn_s_barrier();
      issue(kt + S - 1, (j + S - 1) % S);
      const uint16_t* sl = gemm_norm_smem + j * SLAB;
      bf16x8_t fa[4], fb[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int c = 2 * kk + half;
        fa[kk] = *reinterpret_cast<const bf16x8_t*>(prow + ((kt * 8 + c) ^ sp) * 8);
        fb[kk] = *reinterpret_cast<const bf16x8_t*>(sl + rb * 64 + (c ^ sb) * 8);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[kk], fa[kk], acc, 0, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // the reloads past the end
  epilogue_32x32<uint16_t, KIND>(ep, acc, m0 + l32, n0 + wave * 32, M, N, vec_epi, half, l32);
}

bool gemm_norm_fits(int d) { return d > 0 && d % 128 == 0 && d <= 256 * RMS_V4; }

Status launch_gemm_norm(hipStream_t stream, const float* X, const float* gamma, const float* beta, float* XN,
                        const uint16_t* B, int ldb, int M, int N, int d, const EpiParams& ep) {
  if (M <= 0 || N <= 0) return Status::Invalid("gemm: dimensions must be positive");
  if (!gemm_norm_fits(d)) return Status::Invalid("gemm: the folded norm needs d % 128 == 0 and d <= 1024");
  if (ep.kind != EPI_SEGMENTS && ep.kind != EPI_SEGMENTS_TAP)
    return Status::Invalid("gemm: the folded norm serves the input projection");
  if (ldb % 8 != 0 || !al16(B) || !al16(X) || !al16(XN) || !al16(gamma) || !al16(beta))
    return Status::Invalid("gemm: the folded norm needs 16-byte aligned rows");
  int vec_epi = 0;
  PSSA_RETURN_IF(check_epilogue(ep, true, vec_epi));
  const long tiles = (long)((M + 31) / 32) * ((N + NORM_BN - 1) / NORM_BN);
  if (tiles > 0x7fffffffL) return Status::Invalid("gemm: too many tiles");
  if (ep.kind == EPI_SEGMENTS)
    gemm_norm_kernel<EPI_SEGMENTS><<<(unsigned)tiles, 256, gemm_norm_bytes(d), stream>>>(
        X, d, gamma, beta, XN, B, ldb, M, N, vec_epi, ep);
  else
    gemm_norm_kernel<EPI_SEGMENTS_TAP><<<(unsigned)tiles, 256, gemm_norm_bytes(d), stream>>>(
        X, d, gamma, beta, XN, B, ldb, M, N, vec_epi, ep);
  PSSA_LAUNCH_CHECK("gemm_norm");
  return Status::Ok();
}

Status launch_gemm_f32a(hipStream_t stream, const float* A, int lda, const uint16_t* B, int ldb, int M,
                        int N, int K, const EpiParams& ep) {
  if (M <= 0 || N <= 0 || K <= 0) return Status::Invalid("gemm: dimensions must be positive");
  if (K % 16 != 0 || lda % 4 != 0 || ldb % 8 != 0 || !al16(A) || !al16(B))
    return Status::Invalid("gemm: fp32-activation product needs K % 16 == 0 and 16-byte rows");
  int vec_epi = 0;
  PSSA_RETURN_IF(check_epilogue(ep, true, vec_epi));
  const dim3 grid((N + 31) / 32, (M + 31) / 32);
  if (grid.y > 65535) return Status::Invalid("gemm: too many row groups");
  launch_skinny_kind<float, 1, 8>(stream, ep.kind, grid, A, lda, B, ldb, M, N, K, vec_epi, ep);
  PSSA_LAUNCH_CHECK("gemm_skinny_f32a");
  return Status::Ok();
}

Status launch_gemm(hipStream_t stream, int dtype, const void* A, int lda, const void* B, int ldb,
                   int M, int N, int K, const EpiParams& ep) {
  if (M <= 0 || N <= 0 || K <= 0) return Status::Invalid("gemm: dimensions must be positive");
  const bool bf16 = dtype == PSSA_HIP_BF16;
  int vec_epi = 0;
  PSSA_RETURN_IF(check_epilogue(ep, bf16, vec_epi));
  const int ve = bf16 ? 8 : 4;
  const int vec_load = (K % ve == 0) && (lda % ve == 0) && (ldb % ve == 0) && al16(A) && al16(B);
  const bool vec_bf16 = bf16 && lda % 8 == 0 && ldb % 8 == 0 && al16(A) && al16(B);
  // Few token rows: the 128 x 256 tiling would leave most CUs idle.  One
  // 32-row tile per wave up to 4096 output columns: at 256 rows that gives
  // (N/32) x 8 waves, about one per CU or more.  Wider products (a vocabulary
  // head) keep the tiled kernel: 128 rows x 16384 columns took 93 us as 2048
  // one-wave tiles, each re-reading the rows, and 15 us as 128 tiled ones.
  if (vec_bf16 && K % 16 == 0 && N <= 4096 && (long)((M + 127) / 128) * ((N + 255) / 256) < 128) {
    const auto* a16 = static_cast<const uint16_t*>(A);
    const auto* b16 = static_cast<const uint16_t*>(B);
#ifndef PSSA_FEW_OFF
    if (K % 64 == 0) {
      const long tiles = (long)((M + 32 * FEW_WM - 1) / (32 * FEW_WM)) * ((N + 32 * FEW_WN - 1) / (32 * FEW_WN));
      if (tiles > 0x7fffffffL) return Status::Invalid("gemm: too many tiles");
      launch_few_kind(stream, ep.kind, (unsigned)tiles, a16, lda, b16, ldb, M, N, K, vec_epi, ep);
      PSSA_LAUNCH_CHECK("gemm_few");
      return Status::Ok();
    }
#endif
    const dim3 grid((N + 31) / 32, (M + 31) / 32);
    if (grid.y > 65535) return Status::Invalid("gemm: too many row groups");
    launch_skinny_kind<uint16_t, 1, 16>(stream, ep.kind, grid, a16, lda, b16, ldb, M, N, K, vec_epi, ep);
    PSSA_LAUNCH_CHECK("gemm_skinny");
    return Status::Ok();
  }
  if (!bf16 && vec_load && K % 16 == 0 && (long)((M + 127) / 128) * ((N + 127) / 128) < 128) {
    // fp32 with few token rows: the 128 x 128 tiles would leave most CUs
    // idle (a 512-row product has 4 to 20 of them); one wave per 32 x 32
    // tile instead (64 x 32 past 768 output columns).
    const auto* a32 = static_cast<const float*>(A);
    const auto* b32 = static_cast<const float*>(B);
    if (N <= 768) {
      const dim3 grid((N + 31) / 32, (M + 31) / 32);
      if (grid.y > 65535) return Status::Invalid("gemm: too many row groups");
      launch_skinny_f32_kind<1, 8>(stream, ep.kind, grid, a32, lda, b32, ldb, M, N, K, vec_epi, ep);
    } else {
      const dim3 grid((N + 31) / 32, (M + 63) / 64);
      if (grid.y > 65535) return Status::Invalid("gemm: too many row groups");
      launch_skinny_f32_kind<2, 8>(stream, ep.kind, grid, a32, lda, b32, ldb, M, N, K, vec_epi, ep);
    }
    PSSA_LAUNCH_CHECK("gemm_skinny_f32");
    return Status::Ok();
  }
  if (vec_bf16 && K % LDS_BK == 0) {
    // Direct-to-LDS pipeline; 128 x 128 tiles, narrow outputs 128 x 64.
    // The 128-column tile needs about 100 VGPRs (256 columns: 176), so two
    // of its workgroups fit beside a workgroup of the concurrent lane
    // group's scan on one CU; the prefill measures 2-4% faster with it,
    // although each GEMM alone runs about as fast with either width.
    const int nw = N <= 64 ? 1 : 2;
    const long tiles = (long)((M + 127) / 128) * ((N + 64 * nw - 1) / (64 * nw));
    if (tiles > INT32_MAX) return Status::Invalid("gemm: too many tiles");
    const auto* a16 = static_cast<const uint16_t*>(A);
    const auto* b16 = static_cast<const uint16_t*>(B);
    if (nw == 1)
      launch_lds_kind<1>(stream, ep.kind, dim3((unsigned)tiles), a16, lda, b16, ldb, M, N, K, vec_epi, ep);
    else
      launch_lds_kind<2>(stream, ep.kind, dim3((unsigned)tiles), a16, lda, b16, ldb, M, N, K, vec_epi, ep);
    PSSA_LAUNCH_CHECK("gemm_lds");
    return Status::Ok();
  }
  const long tiles = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > INT32_MAX) return Status::Invalid("gemm: too many tiles");
  dim3 grid((unsigned)tiles);
  if (bf16)
    launch_kind<uint16_t>(stream, ep.kind, grid, static_cast<const uint16_t*>(A), lda,
                          static_cast<const uint16_t*>(B), ldb, M, N, K, vec_load, vec_epi, ep);
  else
    launch_kind<float>(stream, ep.kind, grid, static_cast<const float*>(A), lda,
                       static_cast<const float*>(B), ldb, M, N, K, vec_load, vec_epi, ep);
  PSSA_LAUNCH_CHECK("gemm");
  return Status::Ok();
}

__global__ void to_bf16_kernel(const float* __restrict__ in, int ld_in, uint16_t* __restrict__ out,
                               int ld_out, size_t rows, int cols) {
  const size_t n = rows * (size_t)cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / cols, c = i % cols;
    out[r * ld_out + c] = (uint16_t)f32_to_bf16_bits(in[r * ld_in + c]);
  }
}

Status launch_to_bf16(hipStream_t stream, const float* in, int ld_in, uint16_t* out, int ld_out,
                      size_t rows, int cols) {
  const size_t n = rows * (size_t)cols;
  if (!n) return Status::Ok();
  size_t g = (n + 255) / 256;
  if (g > 16384) g = 16384;
  to_bf16_kernel<<<(unsigned)g, 256, 0, stream>>>(in, ld_in, out, ld_out, rows, cols);
  PSSA_LAUNCH_CHECK("to_bf16");
  return Status::Ok();
}

Status init_gemm_attributes() {
  const void* few[] = {
#define PSSA_GEMM_FEW_FN(KD) reinterpret_cast<const void*>(&gemm_few_kernel<KD, FEW_WM, FEW_WN, FEW_S>),
      PSSA_GEMM_FEW_FN(EPI_STORE) PSSA_GEMM_FEW_FN(EPI_SEGMENTS) PSSA_GEMM_FEW_FN(EPI_ADD_AUX)
      PSSA_GEMM_FEW_FN(EPI_ZRAW) PSSA_GEMM_FEW_FN(EPI_SILU) PSSA_GEMM_FEW_FN(EPI_RESIDUAL)
      PSSA_GEMM_FEW_FN(EPI_SCALE) PSSA_GEMM_FEW_FN(EPI_SEGMENTS_TAP)
#undef PSSA_GEMM_FEW_FN
  };
  for (const void* f : few)
    PSSA_HIP_TRY(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_few_bytes()));
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_norm_kernel<EPI_SEGMENTS>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_norm_bytes(256 * RMS_V4)));
  PSSA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_norm_kernel<EPI_SEGMENTS_TAP>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_norm_bytes(256 * RMS_V4)));
  return Status::Ok();
}

}  // namespace pssa

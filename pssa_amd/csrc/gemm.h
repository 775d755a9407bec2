// MFMA GEMM C = epilogue(A * B^T) and the epilogues the PSSA block fuses.
#pragma once
#include "common.h"

namespace pssa {

enum EpiKind : int {
  EPI_STORE = 0,     // r = acc
  EPI_SEGMENTS = 1,  // column ranges: [0,seg0) softplus, [seg0,seg1) identity,
                     // [seg1,seg2) sigmoid, [seg2,seg3) SiLU, rest identity
  EPI_ADD_AUX = 2,   // r = acc + aux[row, col]
  EPI_ZRAW = 3,      // r = (y*scale + g*acc) + sum_q U[col,q]*act[row,q]
  EPI_SILU = 4,      // r = SiLU(acc)
  EPI_RESIDUAL = 5,  // zf = aux + acc; r = first ? zf : out32 + scale*zf
  EPI_SCALE = 6,     // r = acc * scale
  EPI_SEGMENTS_TAP = 7,  // SEGMENTS, and the SiLU segment also to `tap`
  EPI_KINDS = 8,
};

// Every GEMM writes r to out32 (fp32) and/or out16 (the operand type of the
// GEMM: bf16 bits for bf16 GEMMs, fp32 for fp32 GEMMs); either may be null.
struct EpiParams {
  int kind = EPI_STORE;
  int seg[4] = {0, 0, 0, 0};
  const float* aux = nullptr;  // ADD_AUX operand, RESIDUAL's z_raw
  int ld_aux = 0;
  const float* y = nullptr;    // ZRAW: SSM readout
  int ld_y = 0;
  const float* g = nullptr;    // ZRAW: memory gate
  int ld_g = 0;
  const float* act = nullptr;  // ZRAW: adapter activations [rows, rank] (fp32)
  int ld_act = 0;
  const void* U = nullptr;     // ZRAW: adapter up-projection [N, rank] in the operand type
  int rank = 0;
  float scale = 1.0f;
  int first = 1;
  float* out32 = nullptr;
  int ld32 = 0;
  void* out16 = nullptr;
  int ld16 = 0;
  // Optional fp32 tap: ZRAW writes the adapter output, RESIDUAL writes
  // z_final (before the residual scaling), SEGMENTS_TAP writes the columns
  // [seg[2], seg[3]) (the SiLU segment) to tap[row, col - seg[2]].
  float* tap = nullptr;
  int ld_tap = 0;
};

// A: activations [M, lda], B: weights [N, ldb], both K-contiguous and of the
// same type (dtype PSSA_HIP_BF16: bf16 bit patterns; PSSA_HIP_F32: fp32).
// Accumulation is fp32.
Status launch_gemm(hipStream_t stream, int dtype, const void* A, int lda, const void* B, int ldb,
                   int M, int N, int K, const EpiParams& ep);

// Same product for bf16 weights B and fp32 activations A, each activation
// rounded to bf16 (nearest even) inside the kernel: the result equals
// launch_gemm over a launch_to_bf16 copy of A, bit for bit.  K % 16 == 0,
// lda % 4 == 0, ldb % 8 == 0, 16-byte aligned operands.
Status launch_gemm_f32a(hipStream_t stream, const float* A, int lda, const uint16_t* B, int ldb, int M,
                        int N, int K, const EpiParams& ep);

// fp32 -> bf16 (round to nearest even) copy of a [rows, cols] matrix with
// leading dimensions ld_in / ld_out.
Status launch_to_bf16(hipStream_t stream, const float* in, int ld_in, uint16_t* out, int ld_out,
                      size_t rows, int cols);

// The input projection with the block's RMSNorm folded in (decode steps):
// XN[m] = rmsnorm(X[m]; gamma, beta) (fp32, as the standalone norm writes it)
// and out = bf16(XN) B^T with ep's column-segment epilogue, bit for bit the
// norm followed by launch_gemm.  Needs gemm_norm_fits(d), K = d, bf16 B.
bool gemm_norm_fits(int d);
Status launch_gemm_norm(hipStream_t stream, const float* X, const float* gamma, const float* beta, float* XN,
                        const uint16_t* B, int ldb, int M, int N, int d, const EpiParams& ep);

// Per-device set-up of the GEMM kernels (their dynamic LDS limits).
Status init_gemm_attributes();

}  // namespace pssa

// MFMA GEMM C = epilogue(A * B^T) and the epilogues the PSSA block fuses.
#pragma once
#include "common.h"

namespace pssa {

enum EpiKind : int {
  EPI_STORE = 0,     // C = acc
  EPI_SEGMENTS = 1,  // column ranges: [0,seg0) softplus, [seg0,seg1) identity,
                     // [seg1,seg2) sigmoid, [seg2,seg3) SiLU, rest identity
  EPI_ADD_AUX = 2,   // C = acc + aux[row, col]
  EPI_ZRAW = 3,      // C = y*scale + g*acc + sum_r U[col,r]*act[row,r]
  EPI_SILU = 4,      // C = SiLU(acc)
  EPI_RESIDUAL = 5,  // zf = zraw + acc; C = first ? zf : C + scale*zf
  EPI_SCALE = 6,     // C = acc * scale
};

struct EpiParams {
  int kind = EPI_STORE;
  int seg[4] = {0, 0, 0, 0};
  const float* aux = nullptr;
  int ld_aux = 0;
  const float* y = nullptr;
  int ld_y = 0;
  const float* g = nullptr;
  int ld_g = 0;
  const float* act = nullptr;
  int ld_act = 0;
  const float* U = nullptr;
  int rank = 0;
  float scale = 1.0f;
  const float* zraw = nullptr;
  int ld_zraw = 0;
  int first = 1;
};

// A: fp32 [M, lda]; B: [N, ldb] fp32 or bf16 bits (b_dtype); C: fp32 [M, ldc].
Status launch_gemm_xwt(hipStream_t stream, const float* A, int lda, const void* B, int ldb,
                       int b_dtype, float* C, int ldc, int M, int N, int K, const EpiParams& ep);

}  // namespace pssa

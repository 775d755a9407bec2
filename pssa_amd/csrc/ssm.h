// Fused diagonal SSM scan (prepare + recurrence + readout) for independent lanes.
#pragma once
#include "common.h"

namespace pssa {

struct SsmArgs {
  const float* delta = nullptr;  // softplus'd step sizes, row r at delta + r*ld_delta
  int ld_delta = 0;
  const float* bproj = nullptr;  // B_t, [rows, s]
  int ld_b = 0;
  const float* cproj = nullptr;  // C_t, [rows, s]
  int ld_c = 0;
  const float* xn = nullptr;     // normalised input x_t, [rows, d]
  int ld_x = 0;
  const float* rates2 = nullptr; // -softplus(a_raw) * log2(e), [d*s]
  float* carry = nullptr;        // h, lane b at carry + b*carry_stride, [d*s]; read, then overwritten
  long carry_stride = 0;
  float* y = nullptr;            // readout, [rows, d]
  int ld_y = 0;
  int T = 0, d = 0, s = 0;
  int lanes = 0;
  // Optional materialisation (stage API): per lane b, bar_a/bar_b at
  // + b*T*d*s, states at + b*(T+1)*d*s.  All three or none.
  float* bar_a = nullptr;
  float* bar_b = nullptr;
  float* states = nullptr;
};

// Rows of lane b are b*T .. b*T+T-1.  y must be zero-filled by the caller
// when s exceeds one workgroup's j-range (several workgroups then add their
// partial sums); ssm_needs_zeroed_y() says when.
bool ssm_needs_zeroed_y(int s);
Status launch_ssm_scan(hipStream_t stream, const SsmArgs& a);

// rates2[i] = rates[i] * log2(e) (stage API receives -softplus(a_raw)).
Status launch_scale(hipStream_t stream, const float* in, float* out, size_t n, float scale);

}  // namespace pssa

// Fused diagonal SSM scan (prepare + recurrence + readout) for independent lanes.
#pragma once
#include "common.h"

namespace pssa {

// Position of state j of channel i in one lane's carry: channel blocks of
// 64 (the last one d % 64 wide), each state-major, so the 64 channels x all
// states a step workgroup updates are one contiguous run.
__host__ __device__ __forceinline__ size_t carry_at(int j, int i, int d, int s) {
  const int i0 = i & ~63, w = d - i0 < 64 ? d - i0 : 64;
  return (size_t)i0 * s + (size_t)j * w + (i - i0);
}

// The states jw, jw + 1, ... of channel i in one lane's carry: state jw + q
// at base + q * stride (one base and a uniform stride instead of a 64-bit
// address per state, which the scan would otherwise keep live until its
// final stores, spilling).  The decode step keeps carry_at: with this form
// its code grew by a thousand moves and the carry update took 109 us
// instead of 80.
struct CarryCol {
  size_t base;
  int stride;
};
__host__ __device__ __forceinline__ CarryCol carry_col(int jw, int i, int d, int s) {
  const int i0 = i & ~63, w = d - i0 < 64 ? d - i0 : 64;
  return CarryCol{(size_t)i0 * s + (size_t)jw * w + (i - i0), w};
}

struct SsmArgs {
  const float* delta = nullptr;  // softplus'd step sizes, row r at delta + r*ld_delta
  int ld_delta = 0;
  const float* bproj = nullptr;  // B_t, [rows, s]
  int ld_b = 0;
  const float* cproj = nullptr;  // C_t, [rows, s]
  int ld_c = 0;
  const float* xn = nullptr;     // normalised input x_t, [rows, d]
  int ld_x = 0;
  // State-major layouts (channel contiguous), so that the 64 channels of a
  // wave read and write 256 contiguous bytes per state.
  const float* rates2 = nullptr; // -softplus(a_raw) * log2(e), [s, d]
  float* carry = nullptr;        // h, lane b at carry + b*carry_stride, channel-blocked (carry_at); read, then overwritten
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
  // Partial readouts [state blocks, lanes*T, d], required when
  // ssm_state_blocks(s) > 2 (the blocks are then summed in a fixed order).
  float* y_part = nullptr;
  size_t rows = 0;  // set by launch_ssm_scan
  // Optional bf16 copy of y, written by the single-step kernel when
  // ssm_step_writes_y (other paths leave it untouched).
  uint16_t* y16 = nullptr;
  int ld_y16 = 0;
  // Set when another lane group's kernels share the CUs with this scan: the
  // four-wave variant then runs at any grid size (the eight-wave one is the
  // faster scan alone on small grids, but leaves those kernels less room).
  int concurrent = 0;
};

// Rows of lane b are b*T .. b*T+T-1.  The states of a channel are split into
// ssm_state_blocks(s) workgroups.  With two blocks both add their partial
// readouts into y, which the caller zero-fills first (ssm_needs_zeroed_y; two
// addends onto zero give the same sum in either order); with more, the
// caller provides y_part and the blocks are summed in a fixed order.
int ssm_state_blocks(int s);
bool ssm_needs_zeroed_y(int s);
// A single time step (T == 1) with at most two state blocks stores y (and
// y16) directly: no zero-fill of y is needed and y16 is written.
bool ssm_step_writes_y(int T, int s);
Status launch_ssm_scan(hipStream_t stream, const SsmArgs& a);

// rates2[i] = rates[i] * log2(e) (stage API receives -softplus(a_raw)).
Status launch_scale(hipStream_t stream, const float* in, float* out, size_t n, float scale);

// out[c, r] = in[r, c] for `count` consecutive [rows, cols] matrices (the
// reference's [d, s] state layout <-> the scan's [s, d]), scaled by `scale`.
// Carries of `count` matrices between the reference's [d, s] layout
// (to_device) and the device's channel-blocked one (carry_at), or back.
Status launch_carry_convert(hipStream_t stream, const float* in, float* out, size_t count, int d, int s,
                            bool to_device);
Status launch_transpose(hipStream_t stream, const float* in, float* out, size_t count, int rows,
                        int cols, float scale);

}  // namespace pssa

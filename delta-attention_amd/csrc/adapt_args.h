// Argument blocks of the drift-cosine and adaptive-stride kernels
// (anchor_cos.hip), shared with the library's adaptive chunk loop
// (adapt_loop.hip), which fills them itself.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace da {

struct CosArgs {
  const void* a;           // dense anchor rows or deltas [B, n, H, D]
  int64_t a_b, a_n, a_h;
  const void* s;           // key-sparse output [B, rows, H, D] or nullptr
  int64_t s_b, s_r, s_h;
  const int64_t* rows;     // anchor row of each delta in `s` (nullptr: row i)
  int64_t n_rows;          // rows of `s` (indices are clamped into it)
  float* cos;              // [B, n - 1, H]
  int* hist;               // [bins] or nullptr
  int bins;
  float lo, hi;
  int B, n, H, D;
  const int* n_dev;        // set: the delta count is min(*n_dev, n), read on the device
  // set: {slot0, step} on the device. slot0 >= 0: delta i's dense row is slot
  // slot0 + i * step of `a`; slot0 < 0: row i of a_alt (strides alt_*)
  const int* sel;
  const void* a_alt;
  int64_t alt_b, alt_n, alt_h;
};

struct AdaptArgs {
  const float* cos;        // [B, n - 1, H] of this chunk
  int B, H;
  int* state;              // {gamma, n} of this chunk; overwritten with the next chunk's
  int chunk;               // this chunk's index into the logs
  int next_start, next_end, max_n;
  int64_t* rows_next;      // [max_n] or nullptr
  int trigger;             // 0 absolute, 1 relative
  double threshold, margin, k;
  int gamma_min, gamma_max;
  double* log_mean;
  float* log_min;
  int* log_gamma;
  int* log_n;
  // full_state: state holds 5 ints {gamma, n, n_recompute, slot0, step}, all
  // written for the next chunk. spec_gamma > 0: the dense rows at multiples of
  // spec_gamma are computed ahead; a next chunk whose anchors are all such
  // rows (stride and start multiples of spec_gamma) reads them at slots
  // slot0 + j * step and recomputes none; any other chunk (every chunk with
  // spec_gamma 0) gets slot0 = -1 and recomputes its n anchors.
  // sel_log[2 c .. 2 c + 1] logs this chunk's {slot0, step}.
  bool full_state;
  int spec_gamma;
  int* sel_log;
};

int adapt_step_launch(const CosArgs& c, const AdaptArgs& a, int n_grid, int dtype, hipStream_t st);

}  // namespace da

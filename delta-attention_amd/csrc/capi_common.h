// Argument checks shared by the C entry points.
#pragma once

#include <stdint.h>

#include "delta_attn.h"

namespace da {

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Element strides of a bf16/fp16 row must keep 16-byte row alignment.
inline bool strides8(const int64_t s[3]) { return s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }

// Head dims of the forward kernels (the training backward takes 32, 64, 128).
inline bool head_dim_ok(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }

inline int check_common(int B, int Hq, int Hkv, int D, int dtype) {
  if (dtype != DA_BF16 && dtype != DA_FP16) return DA_ERR_DTYPE;
  if (!head_dim_ok(D)) return DA_ERR_HEAD_DIM;
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return DA_ERR_INVALID_ARG;
  return DA_OK;
}

}  // namespace da

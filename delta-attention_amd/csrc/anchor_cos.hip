// Consecutive-anchor delta cosine: the drift signal of the delta correction.
//
// For anchor deltas d_0 .. d_{n-1} (per batch and head, d_i in R^D) it writes
//   cos[b, i, h] = <d_i, d_{i+1}> / (max(|d_i|, eps) * max(|d_{i+1}|, eps)),
// i = 0 .. n-2, eps = 1e-8, the per-vector clamped form of
// torch.nn.functional.cosine_similarity over the last dim (what
// stride.py:43-52 interanchor_cos and drift.py:23-49 drift_summary take over
// [b, n-1, h]), in fp32 from the stored bf16/fp16 values.
//   * The deltas are read from a delta buffer, or formed on the fly from the
//     dense anchor rows and the key-sparse output at the anchor rows with one
//     rounding to the element type, rnd(dense - sparse), as the reference's
//     tensor subtraction does (llama.py:784-788: the adaptive stride's chunk
//     deltas, never written to memory here).
//   * Optionally every cosine is binned into an int32 histogram over
//     [lo, hi] with torch.histc's rule: bin = (int)((x - lo) * bins / (hi - lo)),
//     x == hi goes to the last bin, values outside [lo, hi] and NaN are
//     dropped (drift.py's 40 bins over [-1, 1]).
// One wave per (b, i, h) pair: lanes hold D / 64 elements of both deltas,
// dot product and squared norms are wave reductions. The deltas are tiny next
// to the attention passes (C3: 2046 x 32 rows of 256 B), so the kernel is
// latency-bound; it replaces a subtract, a cosine and reductions of torch ops.
#include "device_common.h"
#include "capi_common.h"

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
};

template <typename T>
__device__ __forceinline__ void delta_pair(const CosArgs& a, int b, int i, int h, int e,
                                           float& x0, float& x1) {
  using E = Elt<T>;
  constexpr size_t esz = sizeof(T);
  const char* ap = (const char*)a.a + ((int64_t)b * a.a_b + (int64_t)i * a.a_n + (int64_t)h * a.a_h + e) * esz;
  const uint32_t v = *(const uint32_t*)ap;
  if (a.s) {
    int64_t r = a.rows ? a.rows[i] : i;
    r = r < 0 ? 0 : (r >= a.n_rows ? a.n_rows - 1 : r);
    const char* sp = (const char*)a.s + ((int64_t)b * a.s_b + r * a.s_r + (int64_t)h * a.s_h + e) * esz;
    const uint32_t w = *(const uint32_t*)sp;
    const uint32_t d = E::pack2(E::lo(v) - E::lo(w), E::hi(v) - E::hi(w));   // rnd(dense - sparse)
    x0 = E::lo(d);
    x1 = E::hi(d);
  } else {
    x0 = E::lo(v);
    x1 = E::hi(v);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void anchor_cos_kernel(CosArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t pairs = (int64_t)a.B * (a.n - 1) * a.H;
  if (p >= pairs) return;
  const int h = (int)(p % a.H);
  const int64_t t = p / a.H;
  const int i = (int)(t % (a.n - 1));
  const int b = (int)(t / (a.n - 1));
  float w12 = 0.f, w1 = 0.f, w2 = 0.f;
  for (int e = 2 * lane; e < a.D; e += 128) {
    float u0, u1, v0, v1;
    delta_pair<T>(a, b, i, h, e, u0, u1);
    delta_pair<T>(a, b, i + 1, h, e, v0, v1);
    w12 += u0 * v0 + u1 * v1;
    w1 += u0 * u0 + u1 * u1;
    w2 += v0 * v0 + v1 * v1;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    w12 += __shfl_xor(w12, off);
    w1 += __shfl_xor(w1, off);
    w2 += __shfl_xor(w2, off);
  }
  if (lane != 0) return;
  constexpr float EPS = 1e-8f;
  const float c = w12 / (fmaxf(sqrtf(w1), EPS) * fmaxf(sqrtf(w2), EPS));
  a.cos[p] = c;
  if (a.hist && c >= a.lo && c <= a.hi) {
    int bin = (int)((c - a.lo) * (float)a.bins / (a.hi - a.lo));
    if (bin >= a.bins) bin = a.bins - 1;
    atomicAdd(&a.hist[bin], 1);
  }
}

}  // namespace da

using namespace da;

extern "C" int da_anchor_delta_cos(const void* a, const int64_t a_str[3],
                                   const void* sparse, const int64_t s_str[3],
                                   const int64_t* rows, int64_t n_rows,
                                   int B, int n, int H, int D,
                                   float* cos_out, int* hist, int bins, float lo, float hi,
                                   int dtype, void* stream) {
  int rc;
  if ((rc = check_common(B, H, H, D, dtype)) != DA_OK) return rc;
  if (n < 0 || !a_str) return DA_ERR_INVALID_ARG;
  if (n < 2) return DA_OK;                        // no consecutive pair
  if (!a || !cos_out) return DA_ERR_INVALID_ARG;
  if (sparse && (!s_str || n_rows < 1)) return DA_ERR_INVALID_ARG;
  if (hist && (bins < 1 || !(hi > lo))) return DA_ERR_INVALID_ARG;
  // lanes read element pairs: 4-byte alignment of rows and elements
  if (((uintptr_t)a & 3u) || a_str[0] % 2 || a_str[1] % 2 || a_str[2] % 2) return DA_ERR_ALIGNMENT;
  if (sparse && (((uintptr_t)sparse & 3u) || s_str[0] % 2 || s_str[1] % 2 || s_str[2] % 2))
    return DA_ERR_ALIGNMENT;
  const int64_t pairs = (int64_t)B * (n - 1) * H;
  const int64_t grid = (pairs + 3) / 4;
  if (grid > 0x7fffffffLL) return DA_ERR_INVALID_ARG;
  CosArgs c = {};
  c.a = a; c.a_b = a_str[0]; c.a_n = a_str[1]; c.a_h = a_str[2];
  c.s = sparse;
  if (s_str) { c.s_b = s_str[0]; c.s_r = s_str[1]; c.s_h = s_str[2]; }
  c.rows = rows; c.n_rows = n_rows;
  c.cos = cos_out; c.hist = hist; c.bins = bins; c.lo = lo; c.hi = hi;
  c.B = B; c.n = n; c.H = H; c.D = D;
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  if (dtype == DA_BF16)
    hipLaunchKernelGGL((anchor_cos_kernel<__bf16>), dim3((unsigned)grid), dim3(256), 0, s, c);
  else
    hipLaunchKernelGGL((anchor_cos_kernel<_Float16>), dim3((unsigned)grid), dim3(256), 0, s, c);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

// Element-wise kernels of the decoder layer around the attention path, for the
// full-model prefill: residual add + RMSNorm, and the SwiGLU gate.
//
// Arithmetic follows the reference's torch ops element by element, one
// rounding to the element type per tensor op:
//   add + norm (delta_attention/llama.py:69-74, :968-979):
//       h = rnd(x + r);  y = rnd(w * rnd(h * rsqrt(mean(h^2) + eps)))   (fp32 inside)
//   SwiGLU (delta_attention/llama.py:212-213):
//       y = rnd(rnd(silu(g)) * u),  silu(g) = g / (1 + exp(-g))          (fp32 inside)
// Both are HBM-bound: each element is read once and written once with 16-byte
// accesses, non-temporal for large inputs (4-5 % faster than ordinary ones at
// the 8B model's prefill shapes) and ordinary below NT_MIN_BYTES (a decode
// step's single row is read by the next kernel from L2; streamed, it took 9.6
// us per norm instead of ~4). The norm weight is read with ordinary loads
// (every row reuses it). One wave owns one row of the norm (the sum of squares
// is a wave reduction, no LDS).
#include "device_common.h"
#include "capi_common.h"

namespace da {

// Inputs of at least this many bytes stream through non-temporal accesses.
constexpr int64_t NT_MIN_BYTES = 4 << 20;

template <bool NT>
__device__ __forceinline__ u32x4 ld4(const void* p) { return NT ? ld_nt4(p) : *(const u32x4*)p; }
template <bool NT>
__device__ __forceinline__ void st4(void* p, u32x4 v) {
  if constexpr (NT) st_nt4(p, v);
  else *(u32x4*)p = v;
}

struct NormArgs {
  const void* x;      // [rows, n] (row stride xs)
  const void* r;      // residual [rows, n] or nullptr
  void* h;            // x + r written here when r is given (may alias x or r)
  void* y;            // normalised output
  const void* w;      // [n]
  int64_t xs, rs, hs, ys;
  int64_t rows;
  int n;
  float eps;
};

// CH = 16-byte chunks per lane (n = 64 * 8 * CH elements)
template <typename T, int CH, bool NT>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(NormArgs a) {
  using E = Elt<T>;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  constexpr size_t esz = sizeof(T);
  const char* xp = (const char*)a.x + row * a.xs * esz;
  u32x4 v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) v[c] = ld4<NT>(xp + (c * 64 + lane) * 16);
  if (a.r) {
    const char* rp = (const char*)a.r + row * a.rs * esz;
    char* hp = (char*)a.h + row * a.hs * esz;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const u32x4 rv = ld4<NT>(rp + (c * 64 + lane) * 16);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[c][e] = E::pack2(E::lo(v[c][e]) + E::lo(rv[e]), E::hi(v[c][e]) + E::hi(rv[e]));
      st4<NT>(hp + (c * 64 + lane) * 16, v[c]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float l = E::lo(v[c][e]), h = E::hi(v[c][e]);
      ss += l * l + h * h;
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float rinv = rsqrtf(ss / (float)a.n + a.eps);
  const char* wp = (const char*)a.w;
  char* yp = (char*)a.y + row * a.ys * esz;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const u32x4 wv = *(const u32x4*)(wp + (c * 64 + lane) * 16);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t t = E::pack2(E::lo(v[c][e]) * rinv, E::hi(v[c][e]) * rinv);
      o[e] = E::pack2(E::lo(wv[e]) * E::lo(t), E::hi(wv[e]) * E::hi(t));
    }
    st4<NT>(yp + (c * 64 + lane) * 16, o);
  }
}

struct SwiGluArgs {
  const void* g;
  const void* u;
  void* y;
  int64_t gs, us, ys;   // row strides (elements)
  int64_t rows;
  int n;                // row length, multiple of 8
};

template <typename T, bool NT>
__global__ __launch_bounds__(256) void swiglu_kernel(SwiGluArgs a) {
  using E = Elt<T>;
  const int cpr = a.n / 8;   // 16-byte chunks per row
  const int64_t total = a.rows * cpr;
  constexpr size_t esz = sizeof(T);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cpr;
    const int c = (int)(i % cpr);
    const u32x4 gv = ld4<NT>((const char*)a.g + (row * a.gs + 8 * c) * esz);
    const u32x4 uv = ld4<NT>((const char*)a.u + (row * a.us + 8 * c) * esz);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float gl = E::lo(gv[e]), gh = E::hi(gv[e]);
      const uint32_t s = E::pack2(gl / (1.f + __expf(-gl)), gh / (1.f + __expf(-gh)));
      o[e] = E::pack2(E::lo(s) * E::lo(uv[e]), E::hi(s) * E::hi(uv[e]));
    }
    st4<NT>((char*)a.y + (row * a.ys + 8 * c) * esz, o);
  }
}

template <typename T, bool NT>
static void launch_norm_nt(const NormArgs& a, hipStream_t s) {
  const int grid = (int)((a.rows + 3) / 4);
  switch (a.n / 512) {
    case 4: hipLaunchKernelGGL((add_rmsnorm_kernel<T, 4, NT>), dim3(grid), dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((add_rmsnorm_kernel<T, 8, NT>), dim3(grid), dim3(256), 0, s, a); break;
    case 10: hipLaunchKernelGGL((add_rmsnorm_kernel<T, 10, NT>), dim3(grid), dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL((add_rmsnorm_kernel<T, 16, NT>), dim3(grid), dim3(256), 0, s, a); break;
    default: break;
  }
}

template <typename T>
static void launch_norm(const NormArgs& a, hipStream_t s) {
  if (a.rows * a.n * (int64_t)sizeof(T) >= NT_MIN_BYTES) launch_norm_nt<T, true>(a, s);
  else launch_norm_nt<T, false>(a, s);
}

}  // namespace da

using namespace da;

extern "C" int da_add_rmsnorm(const void* x, int64_t x_stride, const void* residual, int64_t r_stride,
                              void* h, int64_t h_stride, void* y, int64_t y_stride,
                              const void* weight, int64_t rows, int n, float eps,
                              int dtype, void* stream) {
  if (dtype != DA_BF16 && dtype != DA_FP16) return DA_ERR_DTYPE;
  if (rows < 0 || !(n == 2048 || n == 4096 || n == 5120 || n == 8192)) return DA_ERR_INVALID_ARG;
  if (rows == 0) return DA_OK;
  if (!x || !y || !weight || (residual && !h) || eps < 0.f) return DA_ERR_INVALID_ARG;
  if (x_stride < n || y_stride < n || (residual && (r_stride < n || h_stride < n)))
    return DA_ERR_INVALID_ARG;
  if ((rows + 3) / 4 > 0x7fffffffLL) return DA_ERR_INVALID_ARG;
  if (!aligned16(x) || !aligned16(y) || !aligned16(weight) || x_stride % 8 || y_stride % 8 ||
      (residual && (!aligned16(residual) || !aligned16(h) || r_stride % 8 || h_stride % 8)))
    return DA_ERR_ALIGNMENT;
  NormArgs a = {};
  a.x = x; a.r = residual; a.h = h; a.y = y; a.w = weight;
  a.xs = x_stride; a.rs = r_stride; a.hs = h_stride; a.ys = y_stride;
  a.rows = rows; a.n = n; a.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  if (dtype == DA_BF16) launch_norm<__bf16>(a, s);
  else launch_norm<_Float16>(a, s);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

extern "C" int da_swiglu(const void* gate, int64_t g_stride, const void* up, int64_t u_stride,
                         void* out, int64_t o_stride, int64_t rows, int n, int dtype, void* stream) {
  if (dtype != DA_BF16 && dtype != DA_FP16) return DA_ERR_DTYPE;
  if (rows < 0 || n < 0 || n % 8) return DA_ERR_INVALID_ARG;
  if (rows == 0 || n == 0) return DA_OK;
  if (!gate || !up || !out || g_stride < n || u_stride < n || o_stride < n) return DA_ERR_INVALID_ARG;
  if (!aligned16(gate) || !aligned16(up) || !aligned16(out) || g_stride % 8 || u_stride % 8 ||
      o_stride % 8)
    return DA_ERR_ALIGNMENT;
  SwiGluArgs a = {};
  a.g = gate; a.u = up; a.y = out; a.gs = g_stride; a.us = u_stride; a.ys = o_stride;
  a.rows = rows; a.n = n;
  const int64_t chunks = rows * (n / 8);
  const int64_t want = (chunks + 255) / 256;
  const int grid = (int)(want < 65536 ? want : 65536);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  const bool nt = rows * n * 2 >= NT_MIN_BYTES;   // both element types are 2 bytes
  if (dtype == DA_BF16) {
    if (nt) hipLaunchKernelGGL((swiglu_kernel<__bf16, true>), dim3(grid), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((swiglu_kernel<__bf16, false>), dim3(grid), dim3(256), 0, s, a);
  } else {
    if (nt) hipLaunchKernelGGL((swiglu_kernel<_Float16, true>), dim3(grid), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((swiglu_kernel<_Float16, false>), dim3(grid), dim3(256), 0, s, a);
  }
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

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
#include "adapt_args.h"

#include <algorithm>

namespace da {


template <typename T>
__device__ __forceinline__ void delta_pair(const CosArgs& a, int b, int i, int h, int e,
                                           float& x0, float& x1) {
  using E = Elt<T>;
  constexpr size_t esz = sizeof(T);
  const char* ap;
  if (a.sel && a.sel[0] < 0) {
    ap = (const char*)a.a_alt + ((int64_t)b * a.alt_b + (int64_t)i * a.alt_n + (int64_t)h * a.alt_h + e) * esz;
  } else {
    const int64_t slot = a.sel ? a.sel[0] + (int64_t)i * a.sel[1] : i;
    ap = (const char*)a.a + ((int64_t)b * a.a_b + slot * a.a_n + (int64_t)h * a.a_h + e) * esz;
  }
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

// Histograms of up to this many bins are binned in LDS first.
constexpr int LDS_BINS = 256;

// One wave per pair; the grid may be smaller than the pairs (sized for a
// device-held count's expected value, or capped when binning), and the waves
// then loop. Binning: each workgroup counts into an LDS histogram and adds its
// non-zero bins to the global one at the end (one global atomic per pair
// serialised on the few bin addresses: 0.75 ms for the 65K cosines of a 128K
// layer).
template <typename T>
__global__ __launch_bounds__(256) void anchor_cos_kernel(CosArgs a) {
  __shared__ int s_hist[LDS_BINS];
  const bool lds_hist = a.hist && a.bins <= LDS_BINS;
  if (lds_hist) {
    for (int i = threadIdx.x; i < a.bins; i += 256) s_hist[i] = 0;
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int n = a.n_dev ? min(max(*a.n_dev, 0), a.n) : a.n;
  const int64_t pairs = n >= 2 ? (int64_t)a.B * (n - 1) * a.H : 0;
  for (int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); p < pairs;
       p += (int64_t)gridDim.x * 4) {
    const int h = (int)(p % a.H);
    const int64_t t = p / a.H;
    const int i = (int)(t % (n - 1));
    const int b = (int)(t / (n - 1));
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
    if (lane == 0) {
      constexpr float EPS = 1e-8f;
      const float c = w12 / (fmaxf(sqrtf(w1), EPS) * fmaxf(sqrtf(w2), EPS));
      a.cos[p] = c;
      if (a.hist && c >= a.lo && c <= a.hi) {
        int bin = (int)((c - a.lo) * (float)a.bins / (a.hi - a.lo));
        if (bin >= a.bins) bin = a.bins - 1;
        if (lds_hist) atomicAdd(&s_hist[bin], 1);
        else atomicAdd(&a.hist[bin], 1);
      }
    }
  }
  if (lds_hist) {
    __syncthreads();
    for (int i = threadIdx.x; i < a.bins; i += 256)
      if (s_hist[i]) atomicAdd(&a.hist[i], s_hist[i]);
  }
}

// One chunk's decision of the adaptive stride (llama.py:784-805 with
// stride.py:55-86), on the device so that the host enqueues every chunk
// without reading anything back. One workgroup: the mean (fp64, fixed order)
// and min of the chunk's b x (n-1) x h delta cosines (fewer than two anchors:
// 1.0 and 1.0, as interanchor_cos returns), logged per chunk; the next stride
// by the absolute rule (halve below `threshold`, double above threshold +
// margin) or the relative one (halve below mu - k sd, double above mu + k sd
// of the earlier chunks' means, population sd, at least two of them), clamped
// to [gamma_min, gamma_max]; then the next chunk's anchor rows start + j *
// gamma for j < ceil((end - start) / gamma), -1 for the rest of the max_n
// slots (rows that the query-sparse kernel treats as empty).

__global__ __launch_bounds__(256) void adapt_next_kernel(AdaptArgs a) {
  __shared__ double s_sum[256];
  __shared__ float s_min[256];
  __shared__ int s_next[2];
  const int tid = threadIdx.x;
  const int gamma = a.state[0];
  const int n = a.state[1];
  const int64_t pairs = n >= 2 ? (int64_t)a.B * (n - 1) * a.H : 0;
  double sum = 0.0;
  float mn = INFINITY;
  for (int64_t p = tid; p < pairs; p += 256) {
    const float c = a.cos[p];
    sum += (double)c;
    mn = fminf(mn, c);
  }
  s_sum[tid] = sum;
  s_min[tid] = mn;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (tid < off) {
      s_sum[tid] += s_sum[tid + off];
      s_min[tid] = fminf(s_min[tid], s_min[tid + off]);
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (a.sel_log) {
      a.sel_log[2 * a.chunk] = a.state[3];
      a.sel_log[2 * a.chunk + 1] = a.state[4];
    }
    const double mean = pairs > 0 ? s_sum[0] / (double)pairs : 1.0;
    const float cmin = pairs > 0 ? s_min[0] : 1.0f;
    a.log_mean[a.chunk] = mean;
    a.log_min[a.chunk] = cmin;
    a.log_gamma[a.chunk] = gamma;
    a.log_n[a.chunk] = n;
    int g = gamma;
    if (a.trigger == 0) {
      if (mean < a.threshold) g = max(gamma / 2, a.gamma_min);
      else if (mean > a.threshold + a.margin) g = min(gamma * 2, a.gamma_max);
    } else if (a.chunk >= 2) {
      double mu = 0.0;
      for (int i = 0; i < a.chunk; ++i) mu += a.log_mean[i];
      mu /= (double)a.chunk;
      double var = 0.0;
      for (int i = 0; i < a.chunk; ++i) {
        const double d = a.log_mean[i] - mu;
        var += d * d;
      }
      const double sd = sqrt(var / (double)a.chunk);
      if (mean < mu - a.k * sd) g = max(gamma / 2, a.gamma_min);
      else if (mean > mu + a.k * sd) g = min(gamma * 2, a.gamma_max);
    }
    const int nn = a.next_end > a.next_start ? (a.next_end - a.next_start + g - 1) / g : 0;
    s_next[0] = g;
    s_next[1] = min(nn, a.max_n);
    a.state[0] = g;
    a.state[1] = min(nn, a.max_n);
    if (a.full_state) {
      const bool ahead = a.spec_gamma > 0 && g % a.spec_gamma == 0 &&
                         a.next_start % a.spec_gamma == 0;
      a.state[2] = ahead ? 0 : min(nn, a.max_n);
      a.state[3] = ahead ? a.next_start / a.spec_gamma : -1;
      a.state[4] = ahead ? g / a.spec_gamma : 1;
    }
  }
  __syncthreads();
  if (a.rows_next) {
    const int g = s_next[0], nn = s_next[1];
    for (int j = tid; j < a.max_n; j += 256)
      a.rows_next[j] = j < nn ? (int64_t)a.next_start + (int64_t)j * g : (int64_t)-1;
  }
}

// The two launches of one chunk step (the library's own chunk loop); the
// cosine grid is sized for n_grid deltas (c.n_dev holds the count).
int adapt_step_launch(const CosArgs& c, const AdaptArgs& a, int n_grid, int dtype, hipStream_t st) {
  const int ng = std::min(std::max(n_grid, 2), c.n > 1 ? c.n : 2);
  const int64_t grid = ((int64_t)c.B * (ng - 1) * c.H + 3) / 4;
  if (grid > 0x7fffffffLL) return DA_ERR_INVALID_ARG;
  (void)hipGetLastError();
  if (dtype == DA_BF16)
    hipLaunchKernelGGL((anchor_cos_kernel<__bf16>), dim3((unsigned)grid), dim3(256), 0, st, c);
  else
    hipLaunchKernelGGL((anchor_cos_kernel<_Float16>), dim3((unsigned)grid), dim3(256), 0, st, c);
  hipLaunchKernelGGL(adapt_next_kernel, dim3(1), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
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
  int64_t grid = (pairs + 3) / 4;
  if (grid > 0x7fffffffLL) return DA_ERR_INVALID_ARG;
  // binning: a few hundred workgroups, each looping over many pairs
  if (hist) grid = std::min<int64_t>(grid, 512);
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

extern "C" int da_adapt_chunk_step(const void* dense, const int64_t d_str[3],
                                   const void* sparse, const int64_t s_str[3], int64_t n_rows,
                                   const int64_t* rows, int B, int H, int D, int max_n,
                                   int* state, float* cos_work, int chunk,
                                   int next_start, int next_end, int64_t* rows_next,
                                   int trigger, double threshold, double margin, double k,
                                   int gamma_min, int gamma_max,
                                   double* log_mean, float* log_min, int* log_gamma, int* log_n,
                                   int dtype, void* stream) {
  int rc;
  if ((rc = check_common(B, H, H, D, dtype)) != DA_OK) return rc;
  if (!dense || !d_str || !sparse || !s_str || n_rows < 1 || !rows || !state || !cos_work)
    return DA_ERR_INVALID_ARG;
  if (!log_mean || !log_min || !log_gamma || !log_n || chunk < 0) return DA_ERR_INVALID_ARG;
  if (max_n < 1 || (trigger != 0 && trigger != 1) || gamma_min < 1 || gamma_max < gamma_min)
    return DA_ERR_INVALID_ARG;
  if (next_end > next_start && (next_start < 0 || !rows_next)) return DA_ERR_INVALID_ARG;
  if (((uintptr_t)dense & 3u) || d_str[0] % 2 || d_str[1] % 2 || d_str[2] % 2) return DA_ERR_ALIGNMENT;
  if (((uintptr_t)sparse & 3u) || s_str[0] % 2 || s_str[1] % 2 || s_str[2] % 2) return DA_ERR_ALIGNMENT;
  const int64_t grid = ((int64_t)B * (max_n > 1 ? max_n - 1 : 1) * H + 3) / 4;
  if (grid > 0x7fffffffLL) return DA_ERR_INVALID_ARG;
  CosArgs c = {};
  c.a = dense; c.a_b = d_str[0]; c.a_n = d_str[1]; c.a_h = d_str[2];
  c.s = sparse; c.s_b = s_str[0]; c.s_r = s_str[1]; c.s_h = s_str[2];
  c.rows = rows; c.n_rows = n_rows;
  c.cos = cos_work; c.B = B; c.n = max_n; c.H = H; c.D = D;
  c.n_dev = state + 1;
  AdaptArgs a = {};
  a.cos = cos_work; a.B = B; a.H = H; a.state = state; a.chunk = chunk;
  a.next_start = next_start; a.next_end = next_end; a.max_n = max_n;
  a.rows_next = next_end > next_start ? rows_next : nullptr;
  a.trigger = trigger; a.threshold = threshold; a.margin = margin; a.k = k;
  a.gamma_min = gamma_min; a.gamma_max = gamma_max;
  a.log_mean = log_mean; a.log_min = log_min; a.log_gamma = log_gamma; a.log_n = log_n;
  hipStream_t st = (hipStream_t)stream;
  (void)hipGetLastError();
  if (dtype == DA_BF16)
    hipLaunchKernelGGL((anchor_cos_kernel<__bf16>), dim3((unsigned)grid), dim3(256), 0, st, c);
  else
    hipLaunchKernelGGL((anchor_cos_kernel<_Float16>), dim3((unsigned)grid), dim3(256), 0, st, c);
  hipLaunchKernelGGL(adapt_next_kernel, dim3(1), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

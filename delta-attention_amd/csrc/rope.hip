// Fused attention prologue: optional per-head RMSNorm (Qwen3) and rotary
// position embedding, in place on the q and k projection outputs, in the
// layout the attention kernels read directly ([B, S, H, D] storage).
//
// Arithmetic follows the reference's torch ops element by element
// (delta_attention/llama.py:69-74 RMSNorm, :161-192 RoPE with bf16/fp16 cos/sin
// tables), one rounding to the element type per tensor op:
//   norm:  y = rnd(w * rnd(x * rsqrt(mean(x^2) + eps)))          (fp32 inside)
//   rope:  out[i]       = rnd(rnd(y[i] * cos[i])       - rnd(y[i+D/2] * sin[i]))
//          out[i + D/2] = rnd(rnd(y[i+D/2] * cos[i+D/2]) + rnd(y[i] * sin[i+D/2]))
// HBM-bound: each row is read once and written once with 16-byte accesses,
// non-temporal for large inputs and ordinary below NT_MIN_BYTES (a decode
// step's rows are read next from L2); the cos/sin rows and the norm weight,
// shared by every head, with ordinary loads. One launch covers the q rows then
// the k rows; D/16 consecutive threads own one (token, head) row, 8 + 8
// elements each (one 16-byte access per half), for D in {32, 64, 128, 256}.
// Large inputs go through rope_stream_kernel, whose threads each take two
// such row pieces with every load issued before the arithmetic (60 -> 69 % of
// HBM at the 128K Llama shape). Indices are 32-bit with the launch's divisors
// as multiply-shift constants.
#include "device_common.h"
#include "capi_common.h"

namespace da {

// Inputs of at least this many bytes stream through non-temporal accesses.
constexpr int64_t NT_MIN_BYTES = 4 << 20;

struct RopePart {
  void* x;                 // [B, S, H, D] (strides b, s, h in elements) or nullptr
  int64_t xs_b, xs_s, xs_h;
  int H;
  const void* w;           // [D] norm weight or nullptr
  int64_t rows;            // B * S * H (0 without this part)
};

struct RopeArgs {
  RopePart q, k;           // rows [0, q.rows) are q's, the next k.rows are k's
  const void* cos;         // [Bc, S, D], Bc in {1, B}
  const void* sin;
  int64_t cs_b, cs_s;
  float eps;
  int B, S, D;
  int64_t rows;            // q.rows + k.rows + v_rows
  // one-token KV-cache append (S == 1): k rows are written to kc at cache
  // row *pos instead of in place, and rows [q.rows + k.rows, rows) copy v
  // into vc at the same row; a row *pos outside [0, max_len) writes neither
  // cache (q is still rotated)
  const int64_t* pos;
  int64_t max_len;
  void* kc;
  int64_t kc_b, kc_s, kc_h;
  const void* v;
  int64_t v_b, v_s, v_h;
  void* vc;
  int64_t vc_b, vc_s, vc_h;
  int64_t v_rows;
  FastDiv fd_hq, fd_hk, fd_s;   // the launch's divisors (q heads, k heads, tokens)
};

// Row pieces per thread of the streaming launch (measured at the 128K Llama
// shape: 1 / 2 / 4 / 8 -> 4.94 / 5.50 / 5.43 / 2.83 TB/s; 8 runs out of
// registers).
#ifndef DA_ROPE_R
#define DA_ROPE_R 2
#endif

// Thread indices are 32-bit: a launch covers fewer than 2^31 threads.
constexpr int64_t ROPE_MAX_THREADS = 0x7fffffffLL;

// threads per (token, head) row
constexpr int rope_tpr(int D) { return D / 16; }

template <typename T, int D, bool NT>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  using E = Elt<T>;
  constexpr int TPR = rope_tpr(D);    // threads per row
  constexpr int HALF = D / 2;
  constexpr int EPT = HALF / TPR;     // elements per thread in each half
  static_assert(EPT == 8, "one 16-byte access per half");
  const uint32_t gtid = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gtid / TPR;
  const int part = (int)(gtid % TPR);
  constexpr size_t esz = sizeof(T);
  // cache row of an append launch, and whether it lies inside the caches
  const int64_t crow = a.pos ? *a.pos : 0;
  const bool crow_ok = crow >= 0 && crow < a.max_len;
  if (a.v_rows > 0 && row >= a.q.rows + a.k.rows) {
    // cache append of v: this thread's 2 x EPT elements, no arithmetic
    if (row >= a.rows || !crow_ok) return;
    const uint32_t vr = (uint32_t)(row - a.q.rows - a.k.rows);
    const uint32_t bv_ = fdiv(vr, a.fd_hk);                      // S == 1
    const int hv = (int)fmodq(vr, bv_, a.fd_hk), bv = (int)bv_;
    const char* src = (const char*)a.v + ((int64_t)bv * a.v_b + (int64_t)hv * a.v_h) * esz;
    char* dst = (char*)a.vc + ((int64_t)bv * a.vc_b + crow * a.vc_s + (int64_t)hv * a.vc_h) * esz;
    const int j0 = part * EPT;
    *(u32x4*)(dst + j0 * esz) = *(const u32x4*)(src + j0 * esz);
    *(u32x4*)(dst + (HALF + j0) * esz) = *(const u32x4*)(src + (HALF + j0) * esz);
    return;
  }
  const bool live = row < a.rows;
  const bool kpart = live && row >= a.q.rows;
  const int64_t rr = live ? (kpart ? row - a.q.rows : row) : 0;
  // the part's fields by selects (dynamic indexing of kernel arguments would
  // copy them to scratch)
  const int64_t xs_b = kpart ? a.k.xs_b : a.q.xs_b;
  const int64_t xs_s = kpart ? a.k.xs_s : a.q.xs_s;
  const int64_t xs_h = kpart ? a.k.xs_h : a.q.xs_h;
  const void* w = kpart ? a.k.w : a.q.w;
  char* const xbase = (char*)(kpart ? a.k.x : a.q.x);
  const FastDiv fd_h = kpart ? a.fd_hk : a.fd_hq;
  const uint32_t bs = fdiv((uint32_t)rr, fd_h);
  const int h = (int)fmodq((uint32_t)rr, bs, fd_h);
  const uint32_t b_ = fdiv(bs, a.fd_s);
  const int s = (int)fmodq(bs, b_, a.fd_s);
  const int b = (int)b_;
  char* xp = xbase + ((int64_t)b * xs_b + (int64_t)s * xs_s + (int64_t)h * xs_h) * esz;
  const int i0 = part * EPT;          // first element of this thread in the low half

  float lo[EPT], hi[EPT];
  auto load8 = [&](const char* p, float* dst, bool nt = false) {
    const u32x4 v = nt ? ld_nt4(p) : *(const u32x4*)p;
#pragma unroll
    for (int e = 0; e < 4; ++e) { dst[2 * e] = E::lo(v[e]); dst[2 * e + 1] = E::hi(v[e]); }
  };
  if (live) {
    load8(xp + i0 * esz, lo, NT);
    load8(xp + (HALF + i0) * esz, hi, NT);
  } else {
#pragma unroll
    for (int e = 0; e < EPT; ++e) { lo[e] = 0.f; hi[e] = 0.f; }
  }

  if (w) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) ss += lo[e] * lo[e] + hi[e] * hi[e];
#pragma unroll
    for (int off = 1; off < TPR; off <<= 1) ss += __shfl_xor(ss, off);
    const float r = rsqrtf(ss / (float)D + a.eps);
    float wl[EPT], wh[EPT];
    load8((const char*)w + i0 * esz, wl);
    load8((const char*)w + (HALF + i0) * esz, wh);
#pragma unroll
    for (int e = 0; e < EPT; e += 2) {
      uint32_t p = E::pack2(lo[e] * r, lo[e + 1] * r);            // x * rsqrt(...) -> dtype
      p = E::pack2(wl[e] * E::lo(p), wl[e + 1] * E::hi(p));      // weight * x -> dtype
      lo[e] = E::lo(p); lo[e + 1] = E::hi(p);
      uint32_t q = E::pack2(hi[e] * r, hi[e + 1] * r);
      q = E::pack2(wh[e] * E::lo(q), wh[e + 1] * E::hi(q));
      hi[e] = E::lo(q); hi[e + 1] = E::hi(q);
    }
  }

  const char* cp = (const char*)a.cos + ((int64_t)(a.cs_b ? b : 0) * a.cs_b + (int64_t)s * a.cs_s) * esz;
  const char* sp = (const char*)a.sin + ((int64_t)(a.cs_b ? b : 0) * a.cs_b + (int64_t)s * a.cs_s) * esz;
  float cl[EPT], ch[EPT], sl[EPT], sh[EPT];
  load8(cp + i0 * esz, cl);
  load8(cp + (HALF + i0) * esz, ch);
  load8(sp + i0 * esz, sl);
  load8(sp + (HALF + i0) * esz, sh);

  uint32_t olo[EPT / 2], ohi[EPT / 2];
#pragma unroll
  for (int e = 0; e < EPT; e += 2) {
    // low half: x*cos + (-x_hi)*sin ; high half: x_hi*cos + x_lo*sin
    const uint32_t a1 = E::pack2(lo[e] * cl[e], lo[e + 1] * cl[e + 1]);
    const uint32_t a2 = E::pack2(-hi[e] * sl[e], -hi[e + 1] * sl[e + 1]);
    olo[e / 2] = E::pack2(E::lo(a1) + E::lo(a2), E::hi(a1) + E::hi(a2));
    const uint32_t b1 = E::pack2(hi[e] * ch[e], hi[e + 1] * ch[e + 1]);
    const uint32_t b2 = E::pack2(lo[e] * sh[e], lo[e + 1] * sh[e + 1]);
    ohi[e / 2] = E::pack2(E::lo(b1) + E::lo(b2), E::hi(b1) + E::hi(b2));
  }
  if (!live) return;
  if (kpart && a.kc) {   // rotated k goes to its cache row (k itself is kept)
    if (!crow_ok) return;
    xp = (char*)a.kc + ((int64_t)b * a.kc_b + crow * a.kc_s + (int64_t)h * a.kc_h) * esz;
  }
  const u32x4 vl = {olo[0], olo[1], olo[2], olo[3]}, vh = {ohi[0], ohi[1], ohi[2], ohi[3]};
  if constexpr (NT) {
    st_nt4(xp + i0 * esz, vl);
    st_nt4(xp + (HALF + i0) * esz, vh);
  } else {
    *(u32x4*)(xp + i0 * esz) = vl;
    *(u32x4*)(xp + (HALF + i0) * esz) = vh;
  }
}

// The in-place launch over large inputs (no cache append): R row pieces per
// thread, all their loads issued before any arithmetic, so that each thread
// keeps 2 R streaming loads (and 4 R loads of the cached cos / sin rows) in
// flight. Piece j of thread t is unit t + j * T (T threads in the grid):
// consecutive threads read consecutive 16-byte pieces at every j. The
// arithmetic is rope_kernel's, operation for operation.
template <typename T, int D, int R>
__global__ __launch_bounds__(256) void rope_stream_kernel(RopeArgs a) {
  using E = Elt<T>;
  constexpr int TPR = rope_tpr(D);
  constexpr int HALF = D / 2;
  constexpr int EPT = HALF / TPR;
  static_assert(EPT == 8, "one 16-byte access per half");
  constexpr size_t esz = sizeof(T);
  const uint32_t nthr = gridDim.x * blockDim.x;
  const uint32_t t0 = blockIdx.x * blockDim.x + threadIdx.x;
  const int part = (int)(t0 % TPR);       // nthr is a multiple of TPR
  const int i0 = part * EPT;
  char* xp[R];
  const void* wp[R];
  u32x4 xl[R], xh[R], cl[R], ch[R], sl[R], sh[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const uint32_t row = (t0 + j * nthr) / TPR;
    const bool live = row < (uint64_t)a.rows;
    const bool kpart = live && row >= (uint64_t)a.q.rows;
    const uint32_t rr = live ? (kpart ? row - (uint32_t)a.q.rows : row) : 0;
    const FastDiv fd_h = kpart ? a.fd_hk : a.fd_hq;
    const uint32_t bs = fdiv(rr, fd_h);
    const int h = (int)fmodq(rr, bs, fd_h);
    const uint32_t b = fdiv(bs, a.fd_s);
    const int s = (int)fmodq(bs, b, a.fd_s);
    const int64_t xs_b = kpart ? a.k.xs_b : a.q.xs_b;
    const int64_t xs_s = kpart ? a.k.xs_s : a.q.xs_s;
    const int64_t xs_h = kpart ? a.k.xs_h : a.q.xs_h;
    char* const xbase = (char*)(kpart ? a.k.x : a.q.x);
    wp[j] = kpart ? a.k.w : a.q.w;
    xp[j] = live ? xbase + ((int64_t)b * xs_b + (int64_t)s * xs_s + (int64_t)h * xs_h) * esz : nullptr;
    const int64_t cs = (int64_t)(a.cs_b ? b : 0) * a.cs_b + (int64_t)s * a.cs_s;
    const char* cp = (const char*)a.cos + cs * esz;
    const char* sp = (const char*)a.sin + cs * esz;
    if (live) {
      xl[j] = ld_nt4(xp[j] + i0 * esz);
      xh[j] = ld_nt4(xp[j] + (HALF + i0) * esz);
    } else {
      xl[j] = u32x4{0, 0, 0, 0};
      xh[j] = u32x4{0, 0, 0, 0};
    }
    cl[j] = *(const u32x4*)(cp + i0 * esz);
    ch[j] = *(const u32x4*)(cp + (HALF + i0) * esz);
    sl[j] = *(const u32x4*)(sp + i0 * esz);
    sh[j] = *(const u32x4*)(sp + (HALF + i0) * esz);
  }
#pragma unroll
  for (int j = 0; j < R; ++j) {
    float lo[EPT], hi[EPT];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[2 * e] = E::lo(xl[j][e]); lo[2 * e + 1] = E::hi(xl[j][e]);
      hi[2 * e] = E::lo(xh[j][e]); hi[2 * e + 1] = E::hi(xh[j][e]);
    }
    if (wp[j]) {     // uniform per row: the TPR lanes of a row share it
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < EPT; ++e) ss += lo[e] * lo[e] + hi[e] * hi[e];
#pragma unroll
      for (int off = 1; off < TPR; off <<= 1) ss += __shfl_xor(ss, off);
      const float r = rsqrtf(ss / (float)D + a.eps);
      const u32x4 wl4 = *(const u32x4*)((const char*)wp[j] + i0 * esz);
      const u32x4 wh4 = *(const u32x4*)((const char*)wp[j] + (HALF + i0) * esz);
#pragma unroll
      for (int e = 0; e < EPT; e += 2) {
        uint32_t p = E::pack2(lo[e] * r, lo[e + 1] * r);
        p = E::pack2(E::lo(wl4[e / 2]) * E::lo(p), E::hi(wl4[e / 2]) * E::hi(p));
        lo[e] = E::lo(p); lo[e + 1] = E::hi(p);
        uint32_t q = E::pack2(hi[e] * r, hi[e + 1] * r);
        q = E::pack2(E::lo(wh4[e / 2]) * E::lo(q), E::hi(wh4[e / 2]) * E::hi(q));
        hi[e] = E::lo(q); hi[e + 1] = E::hi(q);
      }
    }
    uint32_t olo[EPT / 2], ohi[EPT / 2];
#pragma unroll
    for (int e = 0; e < EPT; e += 2) {
      const float c0 = E::lo(cl[j][e / 2]), c1 = E::hi(cl[j][e / 2]);
      const float s0 = E::lo(sl[j][e / 2]), s1 = E::hi(sl[j][e / 2]);
      const float d0 = E::lo(ch[j][e / 2]), d1 = E::hi(ch[j][e / 2]);
      const float t0_ = E::lo(sh[j][e / 2]), t1_ = E::hi(sh[j][e / 2]);
      const uint32_t a1 = E::pack2(lo[e] * c0, lo[e + 1] * c1);
      const uint32_t a2 = E::pack2(-hi[e] * s0, -hi[e + 1] * s1);
      olo[e / 2] = E::pack2(E::lo(a1) + E::lo(a2), E::hi(a1) + E::hi(a2));
      const uint32_t b1 = E::pack2(hi[e] * d0, hi[e + 1] * d1);
      const uint32_t b2 = E::pack2(lo[e] * t0_, lo[e + 1] * t1_);
      ohi[e / 2] = E::pack2(E::lo(b1) + E::lo(b2), E::hi(b1) + E::hi(b2));
    }
    if (xp[j]) {
      st_nt4(xp[j] + i0 * esz, u32x4{olo[0], olo[1], olo[2], olo[3]});
      st_nt4(xp[j] + (HALF + i0) * esz, u32x4{ohi[0], ohi[1], ohi[2], ohi[3]});
    }
  }
}

template <typename T, int D, bool NT>
static void launch_rope_d(const RopeArgs& a, hipStream_t s) {
  const int64_t threads = a.rows * rope_tpr(D);
  const int grid = (int)((threads + 255) / 256);
  hipLaunchKernelGGL((rope_kernel<T, D, NT>), dim3(grid), dim3(256), 0, s, a);
}

template <typename T, bool NT>
static void launch_rope_nt(const RopeArgs& a, hipStream_t s) {
  if (a.D == 128) launch_rope_d<T, 128, NT>(a, s);
  else if (a.D == 64) launch_rope_d<T, 64, NT>(a, s);
  else if (a.D == 256) launch_rope_d<T, 256, NT>(a, s);
  else launch_rope_d<T, 32, NT>(a, s);
}

static bool rope_dim_ok(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }

constexpr int ROPE_STREAM_R = DA_ROPE_R;   // row pieces per thread of rope_stream_kernel

template <typename T, int D>
static void launch_rope_stream_d(const RopeArgs& a, hipStream_t s) {
  const int64_t units = a.rows * rope_tpr(D);
  const int grid = (int)((units + 256 * ROPE_STREAM_R - 1) / (256 * ROPE_STREAM_R));
  hipLaunchKernelGGL((rope_stream_kernel<T, D, ROPE_STREAM_R>), dim3(grid), dim3(256), 0, s, a);
}

template <typename T>
static void launch_rope(const RopeArgs& a, hipStream_t s) {
  if (a.rows * a.D * (int64_t)sizeof(T) >= NT_MIN_BYTES) {
    if (ROPE_STREAM_R <= 1) launch_rope_nt<T, true>(a, s);
    else if (a.D == 128) launch_rope_stream_d<T, 128>(a, s);
    else if (a.D == 64) launch_rope_stream_d<T, 64>(a, s);
    else if (a.D == 256) launch_rope_stream_d<T, 256>(a, s);
    else launch_rope_stream_d<T, 32>(a, s);
  } else {
    launch_rope_nt<T, false>(a, s);
  }
}

}  // namespace da

using namespace da;

// One part (q or k) of the launch, checked.
static int rope_part(RopePart& p, void* x, const int64_t x_str[3], int H, int B, int S,
                     const void* w) {
  p = RopePart{};
  if (!x) return DA_OK;
  if (!x_str || H < 1) return DA_ERR_INVALID_ARG;
  if (!aligned16(x) || !strides8(x_str)) return DA_ERR_ALIGNMENT;
  if (w && !aligned16(w)) return DA_ERR_ALIGNMENT;
  p.x = x; p.xs_b = x_str[0]; p.xs_s = x_str[1]; p.xs_h = x_str[2];
  p.H = H; p.w = w; p.rows = (int64_t)B * S * H;
  return DA_OK;
}

extern "C" int da_rope_qk(void* q, const int64_t q_str[3], int Hq,
                          void* k, const int64_t k_str[3], int Hkv,
                          int B, int S, int D,
                          const void* cos, const void* sin, const int64_t cs_str[2],
                          const void* q_norm_w, const void* k_norm_w, float eps,
                          int dtype, void* stream) {
  if (dtype != DA_BF16 && dtype != DA_FP16) return DA_ERR_DTYPE;
  if (!rope_dim_ok(D)) return DA_ERR_HEAD_DIM;
  if (B < 1 || S < 0) return DA_ERR_INVALID_ARG;
  if (S == 0) return DA_OK;
  if (!cos || !sin || !cs_str || cs_str[0] < 0 || cs_str[1] < D) return DA_ERR_INVALID_ARG;
  if (!aligned16(cos) || !aligned16(sin) || cs_str[0] % 8 || cs_str[1] % 8) return DA_ERR_ALIGNMENT;
  RopeArgs a = {};
  int rc;
  if ((rc = rope_part(a.q, q, q_str, Hq, B, S, q_norm_w)) != DA_OK) return rc;
  if ((rc = rope_part(a.k, k, k_str, Hkv, B, S, k_norm_w)) != DA_OK) return rc;
  a.cos = cos; a.sin = sin; a.cs_b = cs_str[0]; a.cs_s = cs_str[1];
  a.eps = eps; a.B = B; a.S = S; a.D = D;
  a.rows = a.q.rows + a.k.rows;
  if (a.rows == 0) return DA_OK;
  if (a.rows * rope_tpr(D) + 255 > ROPE_MAX_THREADS) return DA_ERR_INVALID_ARG;
  a.fd_hq = make_fastdiv((uint32_t)(Hq > 0 ? Hq : 1));
  a.fd_hk = make_fastdiv((uint32_t)(Hkv > 0 ? Hkv : 1));
  a.fd_s = make_fastdiv((uint32_t)S);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  if (dtype == DA_BF16) launch_rope<__bf16>(a, s);
  else launch_rope<_Float16>(a, s);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

extern "C" int da_rope_qk_append(void* q, const int64_t q_str[3], int Hq,
                                 const void* k, const int64_t k_str[3], int Hkv,
                                 const void* v, const int64_t v_str[3],
                                 int B, int D,
                                 const void* cos, const void* sin, const int64_t cs_str[2],
                                 const void* q_norm_w, const void* k_norm_w, float eps,
                                 void* k_cache, const int64_t kc_str[3],
                                 void* v_cache, const int64_t vc_str[3], int64_t max_len,
                                 const int64_t* pos, int dtype, void* stream) {
  if (dtype != DA_BF16 && dtype != DA_FP16) return DA_ERR_DTYPE;
  if (!rope_dim_ok(D)) return DA_ERR_HEAD_DIM;
  if (B < 1 || Hq < 1 || Hkv < 1 || max_len < 1) return DA_ERR_INVALID_ARG;
  if (!q || !k || !v || !k_cache || !v_cache || !pos || !v_str || !kc_str || !vc_str)
    return DA_ERR_INVALID_ARG;
  if (!cos || !sin || !cs_str || cs_str[0] < 0 || cs_str[1] < D) return DA_ERR_INVALID_ARG;
  if (!aligned16(cos) || !aligned16(sin) || cs_str[0] % 8 || cs_str[1] % 8) return DA_ERR_ALIGNMENT;
  if (!aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache) || !strides8(v_str) ||
      !strides8(kc_str) || !strides8(vc_str) || ((uintptr_t)pos & 7u))
    return DA_ERR_ALIGNMENT;
  RopeArgs a = {};
  int rc;
  if ((rc = rope_part(a.q, q, q_str, Hq, B, 1, q_norm_w)) != DA_OK) return rc;
  if ((rc = rope_part(a.k, const_cast<void*>(k), k_str, Hkv, B, 1, k_norm_w)) != DA_OK) return rc;
  a.cos = cos; a.sin = sin; a.cs_b = cs_str[0]; a.cs_s = cs_str[1];
  a.eps = eps; a.B = B; a.S = 1; a.D = D;
  a.pos = pos; a.max_len = max_len;
  a.kc = k_cache; a.kc_b = kc_str[0]; a.kc_s = kc_str[1]; a.kc_h = kc_str[2];
  a.v = v; a.v_b = v_str[0]; a.v_s = v_str[1]; a.v_h = v_str[2];
  a.vc = v_cache; a.vc_b = vc_str[0]; a.vc_s = vc_str[1]; a.vc_h = vc_str[2];
  a.v_rows = (int64_t)B * Hkv;
  a.rows = a.q.rows + a.k.rows + a.v_rows;
  if (a.rows * rope_tpr(D) + 255 > ROPE_MAX_THREADS) return DA_ERR_INVALID_ARG;
  a.fd_hq = make_fastdiv((uint32_t)Hq);
  a.fd_hk = make_fastdiv((uint32_t)Hkv);
  a.fd_s = make_fastdiv(1u);
  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  if (dtype == DA_BF16) launch_rope_nt<__bf16, false>(a, s);
  else launch_rope_nt<_Float16, false>(a, s);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

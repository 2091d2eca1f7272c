// Backward of the delta-attention composition on gfx950 (the training path,
// delta_attention/train/flex_delta.py:95-196 differentiated by autograd):
//   da_sparse_attn_bwd   gradients of key-sparse attention (sink + block-anchored
//                        window, the mask of kernel (1))
//   da_qsparse_attn_bwd  gradients of selected rows attending their causal keys
//                        (kernel (2) over the anchor and tail rows)
//   da_delta_compose_bwd gradients of the broadcast composition itself
//
// Flash-attention style recomputation: the forward saves each row's
// log2-domain log-sum-exp (lse = m + log2(l), scores scaled by
// sm_scale * log2(e)); the backward recomputes P = 2^(c2 S - lse) tile by
// tile and never materialises the attention matrix.
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dO * O)),
//   dQ = sm_scale dS K,  dK = sm_scale dS^T Q.
// Two kernels per attention:
//   * dq_kernel: one workgroup per 128 flattened (row, head) pairs (the G
//     query heads of a KV head packed, as in the forward) and a chunk of their
//     key-tile list; 64-key K and V tiles arrive in LDS by buffer-load DMA
//     through a ring (head_dim 128: two stages, each tile's two 32-key halves
//     computed in turn; else three stages), tiles wholly visible skip the
//     per-key mask; S^T = K Q^T and dP^T = V dO^T
//     with Q and dO fragments in registers, dQ^T += K^T dS^T from transposed
//     LDS reads. It also writes rowsum(dO * O) for the other kernel. Long
//     key lists (selected rows) are split; the splits' fp32 partial dQ are
//     summed by dq_reduce_kernel.
//   * dkdv_kernel: one workgroup per 128 keys (32 per wave, K and V fragments
//     in registers) and a chunk of the rows that see them; per 32-row tile and
//     query head it stages Q, dO, lse and rowsum(dO * O) in LDS (by
//     buffer-load DMA into two stages, the next tile's rows in flight under
//     this tile's products; selected rows' q rows gathered per lane) and forms
//     S = Q K^T, dP = dO V^T (rows x keys), then dV^T += dO^T P and
//     dK^T += Q^T dS from transposed LDS reads. Sink keys are seen by every
//     later row, so their row range is cut into chunks like any other; each
//     chunk writes fp32 partials that dkdv_reduce_kernel sums per key.
// Every MFMA is v_mfma_f32_32x32x16 (bf16 or fp16 operands, fp32 accumulate).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "device_common.h"
#include "capi_common.h"

namespace da {
namespace bwd {

constexpr int NWAVE = 4;
constexpr int NTHR = 64 * NWAVE;
constexpr int BM = 32 * NWAVE;   // dq kernel: flattened (row, head) pairs per workgroup
// dq kernel: keys per tile (at head_dim 128 computed as two 32-key halves one
// after the other, which keeps the score registers small enough for two waves
// per SIMD)
template <int D>
constexpr int dq_bn() { return 64; }
constexpr int KT = 32 * NWAVE;   // dkdv kernel: keys per workgroup
constexpr int RT = 32;           // dkdv kernel: rows per step
constexpr int RPC_MAX = 8192;    // dkdv kernel: rows per chunk at most (default)
constexpr int RED = 256;         // threads of the reduce / compose kernels

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  int64_t qs_b, qs_h, qs_s;
  int64_t ks_b, ks_h, ks_s;
  int64_t vs_b, vs_h, vs_s;
  int64_t os_b, os_h, os_s;      // o and dout: {batch, head, list position}
  int64_t gs_b, gs_h, gs_s;
  const float* lse;              // [B, Hq, n_rows]
  float* dvec;                   // [B, Hq, n_rows] rowsum(dout * o)
  void* dq;
  void* dk;
  void* dv;
  int64_t dqs_b, dqs_h, dqs_s;
  int64_t dks_b, dks_h, dks_s;
  int64_t dvs_b, dvs_h, dvs_s;
  int B, Hq, Hkv, G;
  int n_rows, n_q, n_kv;
  float scale_log2, sm_scale;
  int window, sink, q_block;
  const int64_t* q_rows;         // selected rows: q row of list position i
  const int64_t* row_last;       // selected rows: last visible key, ascending
  int accumulate;                // outputs: out = rnd(out + rnd(grad))
  int q32;                       // selected rows: every q row of a head within 32-bit byte offsets
  // dq kernel
  int n_mtiles, n_splits, chunk;
  float* dq_part;                // [item][BM][D] when n_splits > 1
  // dkdv kernel
  int n_blk, nsb, ncs, nco, rpc, items_per_bh;
  int red_keys;                  // keys per (batch, kv head) the reduce sums: blocks of several items
  int part_per_bh;               // partial slots per (batch, kv head): the items of those blocks
  float* kv_part;                // [B * Hkv * part_per_bh][2][KT][D]
};

// Key tiles (BN keys) a row tile visits, in order: the sink tiles, then the
// tiles from the one holding lo_min to the one holding hi_max.
template <int BN>
__device__ __forceinline__ void tile_list(int hi_max, int lo_min, int sink, int& n_first,
                                          int& second_t0, int& n_second) {
  int sink_end = min(min(sink, lo_min), hi_max + 1);
  if (sink_end < 0) sink_end = 0;
  n_first = (sink_end + BN - 1) / BN;
  second_t0 = max(max(lo_min, 0) / BN, n_first);
  n_second = hi_max >= 0 ? max(0, hi_max / BN - second_t0 + 1) : 0;
}

__device__ __forceinline__ int sigma32(int r) {
  return (r & 0x13) | ((r & 4) << 1) | ((r & 8) >> 1);
}

// LDS rows of D elements; 16-byte chunk c of row r sits at chunk c ^ swz(r).
// The tiles are read two ways: 16-byte row pieces (16 lanes, 16 rows r0 ..
// r0 + 15 in some order, one chunk) and transposed 8-byte reads (4
// consecutive rows 4m .. 4m + 3 x chunks 4 dt .. 4 dt + 3). A row read is
// conflict-free when the 16 rows land on 16 distinct 16-byte bank columns, a
// transposed read when the 4 rows' swizzles differ above bit 1. Bank column
// of (r, c): (r DCH + (c ^ swz(r))) mod 16. head_dim 128 (one row per bank
// row): the two 2-bit halves of r & 15 swapped; 64 (two rows per bank row):
// bit 2 from r bit 1, bits 0-1 from r bits 2-3; 32 (four): r bits 2-3.
// (4 (r & 3) alone left the row reads 4-way, at head_dim 64 8-way, in conflict.)
template <int D>
__device__ __forceinline__ int swz(int row) {
  if constexpr (D == 128) return ((row & 3) << 2) | ((row >> 2) & 3);
  else if constexpr (D == 64) return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
  else return (row >> 2) & 3;
}

// A-operand fragment (32 rows x 16 dims, k-step ds) of a row-major LDS tile:
// lane (ln, lg) reads row `row`, dims 16 ds + 8 lg .. +7.
template <int D>
__device__ __forceinline__ u32x4 read_rows(const DA_LDS char* t, int row, int ds, int lg) {
  return *(const DA_LDS u32x4*)(t + row * (2 * D) + (((2 * ds + lg) ^ swz<D>(row)) * 16));
}

// Offsets of the transposed reads that give the A operand X^T (32 dims x 16
// rows) of a row-major LDS tile X: 16-lane group (hh, g) covers dims
// 32 dt + 16 hh + (0..15) and rows 16 ks + 8 g + 4 rd + (0..3).
template <int D>
__device__ __forceinline__ int tr_offset(int lane, int dt) {
  const int g4 = lane >> 4, hh = g4 & 1, g = g4 >> 1, j = lane & 15;
  const int row = 8 * g + (j >> 2);
  const int lc = 4 * dt + 2 * hh + ((j & 3) >> 1);
  return row * (2 * D) + ((lc ^ swz<D>(row)) * 16) + (j & 1) * 8;
}
// The second read's rows are 4 on: their (r >> 2) is odd where the first
// read's is even, which under swz flips chunk bit 0 (address bit 4); 16 rows
// on, swz repeats.
template <int D>
__device__ __forceinline__ u32x4 read_tr(const DA_LDS char* t, int off, int kk) {
  const u32x2 a = read_tr16(t + off + (16 * kk) * (2 * D));
  const u32x2 b = read_tr16(t + (off ^ 16) + (16 * kk + 4) * (2 * D));
  return (u32x4){a[0], a[1], b[0], b[1]};
}

// Block-anchored window start of row r (the forward's mask, flex_delta.py:59-61).
__device__ __forceinline__ int win_lo(int r, int q_block, int window) {
  return (r / q_block) * q_block + q_block - window;
}

// Wait until this wave's DMAs (and other vector memory operations) are done
// (s_waitcnt vmcnt(0), gfx9 encoding; LDS and export counters not waited on).
__device__ __forceinline__ void wait_dma() {
  __builtin_amdgcn_s_waitcnt((0 & 15) | ((0 >> 4) << 14) | (7 << 4) | (15 << 8));
}
// ... until at most N vector memory operations are outstanding
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
constexpr int NST = 3;   // LDS stages of the dq kernel's DMA ring (head_dim < 128)

template <typename T>
__device__ __forceinline__ uint32_t acc_pack(uint32_t old, float lo, float hi, bool accumulate) {
  using E = Elt<T>;
  const uint32_t p = E::pack2(lo, hi);
  return accumulate ? E::pack2(E::lo(old) + E::lo(p), E::hi(old) + E::hi(p)) : p;
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool ROWS>
__global__ __launch_bounds__(NTHR, 2) void dq_kernel(BwdArgs a) {
  using E = Elt<T>;
  constexpr int BN = dq_bn<D>(), NH = BN / 32;
  // head_dim 128: two stages of 64-key tiles whose 32-key halves are computed
  // one after the other (the score registers of one half); else three stages
  constexpr int NSQ = D == 128 ? 2 : NST;
  constexpr bool SEQH = D == 128;
  constexpr int NDS = D / 16, NDT = D / 32, DCH = D / 8, RB = 2 * D;
  constexpr int TB = BN * RB;
  constexpr int NLD = TB / (NTHR * 16);   // 16-byte DMA chunks per thread per K (or V) tile
  static_assert(NLD >= 1, "tile load");
  // [stage][K, V][tile]
  __shared__ __attribute__((aligned(1024))) char smem[NSQ][2][TB];
  __shared__ int red[4][NWAVE];
  const size_t esz = sizeof(T);

  // `wave` stays a vector value: a scalar one makes the compiler treat the
  // DMA's LDS destination as aliasing the fragment reads and wait for every
  // DMA right after issuing it; the loop orders DMA and reads itself
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, lg = lane >> 5;
  // XCD-aware: workgroup b runs item (b % 8) per + b / 8, so each XCD takes a
  // contiguous range of row tiles, whose key/value tiles overlap in its L2
  const int per = (int)(gridDim.x >> 3);
  const int w = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (w >= a.B * a.Hkv * a.n_mtiles * a.n_splits) return;
  const int mt = w % a.n_mtiles;
  const int split = (w / a.n_mtiles) % a.n_splits;
  const int bh = w / a.n_mtiles / a.n_splits;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  const int G = a.G;

  const int mflat = mt * BM + wave * 32 + ln;
  const bool valid = mflat < a.n_rows * G;
  const int irow = valid ? mflat / G : 0;
  const int h = hk * G + (valid ? mflat % G : 0);
  int qrow, hi, lo;
  if (ROWS) {
    qrow = (int)min(max(a.q_rows[irow], (int64_t)0), (int64_t)(a.n_q - 1));
    int64_t lim = a.row_last[irow];
    if (lim > a.n_kv - 1) lim = a.n_kv - 1;
    hi = valid ? (int)(lim < -1 ? -1 : lim) : -1;
    lo = 0;
  } else {
    qrow = irow;
    hi = valid ? irow : -1;
    lo = win_lo(irow, a.q_block, a.window);
  }
  const int sink = ROWS ? 0 : a.sink;

  // Q, dO fragments (B operands, dims 16 ds + 8 lg .. +7 of this lane's row)
  // and rowsum(dO * O)
  u32x4 qf[NDS], df[NDS];
  float dsum = 0.f;
  {
    const char* qp = (const char*)a.q + ((int64_t)b * a.qs_b + (int64_t)h * a.qs_h + (int64_t)qrow * a.qs_s) * esz;
    const char* gp = (const char*)a.dout + ((int64_t)b * a.gs_b + (int64_t)h * a.gs_h + (int64_t)irow * a.gs_s) * esz;
    const char* op = (const char*)a.o + ((int64_t)b * a.os_b + (int64_t)h * a.os_h + (int64_t)irow * a.os_s) * esz;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int off = (16 * ds + 8 * lg) * (int)esz;
      qf[ds] = valid ? *(const u32x4*)(qp + off) : (u32x4){0, 0, 0, 0};
      df[ds] = valid ? *(const u32x4*)(gp + off) : (u32x4){0, 0, 0, 0};
      const u32x4 of = valid ? *(const u32x4*)(op + off) : (u32x4){0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        dsum += E::lo(df[ds][e]) * E::lo(of[e]) + E::hi(df[ds][e]) * E::hi(of[e]);
    }
  }
  const float Di = sum32(dsum);
  const int64_t rix = ((int64_t)b * a.Hq + h) * a.n_rows + irow;
  if (valid && lg == 0 && split == 0) a.dvec[rix] = Di;
  const float lse = valid ? a.lse[rix] : INFINITY;

  // tile-wide bounds over the valid rows
  int v_hmin = valid ? hi : 0x7fffffff, v_hmax = valid ? hi : -1;
  int v_lmin = valid ? lo : 0x7fffffff, v_lmax = valid ? lo : (int)0x80000000;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    v_hmin = min(v_hmin, __shfl_xor(v_hmin, off));
    v_hmax = max(v_hmax, __shfl_xor(v_hmax, off));
    v_lmin = min(v_lmin, __shfl_xor(v_lmin, off));
    v_lmax = max(v_lmax, __shfl_xor(v_lmax, off));
  }
  if (lane == 0) {
    red[0][wave] = v_hmin;
    red[1][wave] = v_hmax;
    red[2][wave] = v_lmin;
    red[3][wave] = v_lmax;
  }
  __syncthreads();
  int hi_min = red[0][0], hi_max = red[1][0], lo_min = red[2][0], lo_max = red[3][0];
#pragma unroll
  for (int i = 1; i < NWAVE; ++i) {
    hi_min = min(hi_min, red[0][i]);
    hi_max = max(hi_max, red[1][i]);
    lo_min = min(lo_min, red[2][i]);
    lo_max = max(lo_max, red[3][i]);
  }
  int n_first, second_t0, n_second;
  tile_list<BN>(hi_max, lo_min, sink, n_first, second_t0, n_second);
  int nt = n_first + n_second;
  const int t_off = split * a.chunk;
  nt = max(0, min(a.chunk, nt - t_off));

  const char* kbase = (const char*)a.k + ((int64_t)b * a.ks_b + (int64_t)hk * a.ks_h) * esz;
  const char* vbase = (const char*)a.v + ((int64_t)b * a.vs_b + (int64_t)hk * a.vs_h) * esz;
  const float c2 = a.scale_log2;
  // DMA of key tile t: lane chunk c fills LDS slot (c NWAVE + wave) 64 + lane,
  // i.e. row slot / DCH, position slot % DCH, from the source chunk that
  // position holds under the swizzle; keys past the last read as zero
  const uint32_t krow_b = (uint32_t)(a.ks_s * (int64_t)esz);
  const uint32_t vrow_b = (uint32_t)(a.vs_s * (int64_t)esz);
  const uint64_t kend = (uint64_t)kbase + (uint64_t)(uint32_t)a.n_kv * krow_b;
  const uint64_t vend = (uint64_t)vbase + (uint64_t)(uint32_t)a.n_kv * vrow_b;
  uint32_t koff[NLD], voff[NLD];
#pragma unroll
  for (int c = 0; c < NLD; ++c) {
    const int slot = (c * NWAVE + wave) * 64 + lane;
    const int row = slot / DCH, pc = slot % DCH;
    koff[c] = (uint32_t)row * krow_b + (uint32_t)((pc ^ swz<D>(row)) * 16);
    voff[c] = (uint32_t)row * vrow_b + (uint32_t)((pc ^ swz<D>(row)) * 16);
  }
  auto tile_n0 = [&](int t) -> int {
    const int u = t + t_off;
    return (u < n_first ? u : second_t0 + (u - n_first)) * BN;
  };
  auto issue = [&](int t, int st) {
    const int n0 = tile_n0(t);
    const uint64_t pk = (uint64_t)kbase + (uint64_t)(uint32_t)n0 * krow_b;
    const uint64_t pv = (uint64_t)vbase + (uint64_t)(uint32_t)n0 * vrow_b;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc((const void*)pk, ((kend - pk) >> 32) ? 0xffffffffu : (uint32_t)(kend - pk));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc((const void*)pv, ((vend - pv) >> 32) ? 0xffffffffu : (uint32_t)(vend - pv));
#pragma unroll
    for (int c = 0; c < NLD; ++c) {
      dma16(rk, (DA_LDS void*)(&smem[st][0][(c * NWAVE + wave) * 1024]), koff[c]);
      dma16(rv, (DA_LDS void*)(&smem[st][1][(c * NWAVE + wave) * 1024]), voff[c]);
    }
  };

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[dt][j] = 0.f;
  int tro[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) tro[dt] = tr_offset<D>(lane, dt);
  // ring of NSQ stages: with three, tiles t + 1 and t + 2 are in flight while
  // tile t is consumed (the stage tile t + 2 lands in was last read in step
  // t - 1, before its barrier); with two (head_dim 128, 64 KB of LDS for two
  // workgroups per CU), tile t + 1 is; each issue is 2 NLD DMAs per lane
  if (nt > 0) {
    issue(0, 0);
    if (NSQ == 3 && nt > 1) issue(1, 1);
    if (NSQ == 3 && nt > 1) wait_vm<2 * NLD>();
    else wait_dma();
    __syncthreads();
  }
  for (int t = 0; t < nt; ++t) {
    const int n0 = tile_n0(t);
    if (NSQ == 3) {
      if (t + 2 < nt) issue(t + 2, (t + 2) % NSQ);
    } else {
      if (t + 1 < nt) issue(t + 1, (t + 1) % NSQ);
    }
    const DA_LDS char* ks = (const DA_LDS char*)&smem[t % NSQ][0][0];
    const DA_LDS char* vs = (const DA_LDS char*)&smem[t % NSQ][1][0];
    const int n1 = n0 + BN - 1;
    const bool full = n1 <= hi_min && n1 < a.n_kv && (n1 < sink || n0 >= lo_max);
    auto halves = [&](int h0, auto nh_c) __attribute__((always_inline)) {
    constexpr int NHH = decltype(nh_c)::value;

    // S^T = K Q^T and dP^T = V dO^T; element j of half hf is key
    // n0 + 32 hf + 16 (j / 8) + 8 lg + j % 8 (rows sigma(ln) of the A tiles)
    f32x16 x[NHH], y[NHH];
#pragma unroll
    for (int hf = 0; hf < NHH; ++hf)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        x[hf][j] = 0.f;
        y[hf][j] = 0.f;
      }
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
      for (int hf = 0; hf < NHH; ++hf) {
        const int r = sigma32(ln) + 32 * (h0 + hf);
        x[hf] = E::mfma(read_rows<D>(ks, r, ds, lg), qf[ds], x[hf]);
        y[hf] = E::mfma(read_rows<D>(vs, r, ds, lg), df[ds], y[hf]);
      }
    uint32_t dsp[8 * NHH];
#pragma unroll
    for (int hf = 0; hf < NHH; ++hf)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float d2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int jj = 2 * j + e;
          const int key = n0 + 32 * (h0 + hf) + 16 * (jj >> 3) + 8 * lg + (jj & 7);
          const bool vis = full || (key <= hi && (key < sink || key >= lo));
          const float p = vis ? fast_exp2(fmaf(x[hf][jj], c2, -lse)) : 0.f;
          d2[e] = p * (y[hf][jj] - Di);
        }
        dsp[8 * hf + j] = E::pack2(d2[0], d2[1]);
      }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int kk = 0; kk < 2 * NHH; ++kk) {
      const u32x4 sf = {dsp[4 * kk], dsp[4 * kk + 1], dsp[4 * kk + 2], dsp[4 * kk + 3]};
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] = E::mfma(read_tr<D>(ks, tro[dt], 2 * h0 + kk), sf, acc[dt]);
    }
    };
    if constexpr (SEQH) {
#pragma unroll
      for (int h = 0; h < NH; ++h) halves(h, std::integral_constant<int, 1>());
    } else {
      halves(0, std::integral_constant<int, NH>());
    }
    // tile t + 1 must have landed (three stages: tile t + 2 may still be in flight)
    if (NSQ == 3 && t + 2 < nt) wait_vm<2 * NLD>();
    else wait_dma();
    __syncthreads();
  }

  if (!valid) return;
  if (a.n_splits == 1) {
    char* qp = (char*)a.dq + ((int64_t)b * a.dqs_b + (int64_t)h * a.dqs_h + (int64_t)qrow * a.dqs_s) * esz;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const int d = 32 * dt + 8 * jq + 4 * lg;
        u32x2* p = (u32x2*)(qp + d * esz);
        const u32x2 old = a.accumulate ? *p : (u32x2){0, 0};
        u32x2 nw;
        nw[0] = acc_pack<T>(old[0], acc[dt][4 * jq] * a.sm_scale, acc[dt][4 * jq + 1] * a.sm_scale, a.accumulate);
        nw[1] = acc_pack<T>(old[1], acc[dt][4 * jq + 2] * a.sm_scale, acc[dt][4 * jq + 3] * a.sm_scale, a.accumulate);
        *p = nw;
      }
  } else {
    float* po = a.dq_part + ((int64_t)w * BM + wave * 32 + ln) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const int d = 32 * dt + 8 * jq + 4 * lg;
        *(f32x4*)(po + d) = (f32x4){acc[dt][4 * jq], acc[dt][4 * jq + 1],
                                     acc[dt][4 * jq + 2], acc[dt][4 * jq + 3]};
      }
  }
}

// Sum of the dq splits of every valid (row, head), 8 dims per thread.
template <typename T, int D, bool ROWS>
__global__ __launch_bounds__(RED) void dq_reduce_kernel(BwdArgs a) {
  constexpr int CPR = D / 8;
  const int64_t task = (int64_t)blockIdx.x * RED + threadIdx.x;
  const int64_t per_bh = (int64_t)a.n_mtiles * BM * CPR;
  if (task >= (int64_t)a.B * a.Hkv * per_bh) return;
  const int bh = (int)(task / per_bh);
  const int rem = (int)(task % per_bh);
  const int mflat = rem / CPR, c = rem % CPR;
  if (mflat >= a.n_rows * a.G) return;
  const int mt = mflat / BM, r = mflat % BM;
  float s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.f;
  for (int sp = 0; sp < a.n_splits; ++sp) {
    const int64_t w = ((int64_t)bh * a.n_splits + sp) * a.n_mtiles + mt;
    const f32x4* p = (const f32x4*)(a.dq_part + (w * BM + r) * D + 8 * c);
    const f32x4 x0 = p[0], x1 = p[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[e] += x0[e];
      s[4 + e] += x1[e];
    }
  }
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  const int irow = mflat / a.G, h = hk * a.G + mflat % a.G;
  const int qrow = ROWS ? (int)min(max(a.q_rows[irow], (int64_t)0), (int64_t)(a.n_q - 1)) : irow;
  u32x4* p = (u32x4*)((char*)a.dq + ((int64_t)b * a.dqs_b + (int64_t)h * a.dqs_h +
                                     (int64_t)qrow * a.dqs_s + 8 * c) * sizeof(T));
  const u32x4 old = a.accumulate ? *p : (u32x4){0, 0, 0, 0};
  u32x4 nw;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    nw[e] = acc_pack<T>(old[e], s[2 * e] * a.sm_scale, s[2 * e + 1] * a.sm_scale, a.accumulate);
  *p = nw;
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool ROWS>
__global__ __launch_bounds__(NTHR, 1) void dkdv_kernel(BwdArgs a) {
  using E = Elt<T>;
  constexpr int NDS = D / 16, NDT = D / 32, DCH = D / 8, RB = 2 * D;
  constexpr int TB = RT * RB;
  // Q and dO rows of HGM = 4 query heads per step in two LDS stages filled by
  // buffer-load DMA, the next step's rows landing while this step's products
  // run. Selected rows whose q tensor does not fit 32-bit offsets fall back
  // to one stage filled through registers.
  constexpr int HGM = 4;
  constexpr int NSTG = 2;
  __shared__ __attribute__((aligned(1024))) char smem[NSTG][2][HGM][TB];   // [stage][Q, dO][head]
  __shared__ __attribute__((aligned(16))) float s_lse[NSTG][HGM][RT], s_d[NSTG][HGM][RT];
  __shared__ __attribute__((aligned(16))) int s_lim[NSTG][RT], s_lo[NSTG][RT];
  const size_t esz = sizeof(T);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 31, lg = lane >> 5;
  // XCD-aware: each XCD takes a contiguous range of key blocks, whose
  // query rows overlap in its L2
  const int per = (int)(gridDim.x >> 3);
  const int wi = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (wi >= a.B * a.Hkv * a.items_per_bh) return;
  const int item = wi % a.items_per_bh;
  const int bh = wi / a.items_per_bh;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  int blk, c;
  if (item < a.nsb * a.ncs) {
    blk = item / a.ncs;
    c = item % a.ncs;
  } else {
    const int r = item - a.nsb * a.ncs;
    blk = a.nsb + r / a.nco;
    c = r % a.nco;
  }
  const int k0 = blk * KT;
  const int key = k0 + wave * 32 + ln;

  // list positions that see a key of this block
  int p_start, p_end;
  if (ROWS) {
    // first position whose last visible key reaches k0 (row_last ascending)
    int lo_i = 0, hi_i = a.n_rows;
    while (lo_i < hi_i) {
      const int mid = (lo_i + hi_i) >> 1;
      const int64_t lim = min(a.row_last[mid], (int64_t)(a.n_kv - 1));
      if (lim >= k0) hi_i = mid;
      else lo_i = mid + 1;
    }
    p_start = lo_i;
    p_end = a.n_rows - 1;
  } else {
    p_start = k0;
    const int kl = min(k0 + KT - 1, a.n_kv - 1);
    if (k0 < a.sink) {
      p_end = a.n_rows - 1;
    } else {
      const int tq = kl + a.window - a.q_block;
      const int rmax = tq < 0 ? -1 : (tq / a.q_block + 1) * a.q_block - 1;
      p_end = min(a.n_rows - 1, rmax);
    }
  }
  const int c_start = p_start + c * a.rpc;
  const int c_end = min(p_end, c_start + a.rpc - 1);

  // K^T and V^T fragments of this lane's key (B operands)
  u32x4 kf[NDS], vf[NDS];
  {
    const bool in = key < a.n_kv;
    const char* kp = (const char*)a.k + ((int64_t)b * a.ks_b + (int64_t)hk * a.ks_h + (int64_t)(in ? key : 0) * a.ks_s) * esz;
    const char* vp = (const char*)a.v + ((int64_t)b * a.vs_b + (int64_t)hk * a.vs_h + (int64_t)(in ? key : 0) * a.vs_s) * esz;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int off = (16 * ds + 8 * lg) * (int)esz;
      kf[ds] = in ? *(const u32x4*)(kp + off) : (u32x4){0, 0, 0, 0};
      vf[ds] = in ? *(const u32x4*)(vp + off) : (u32x4){0, 0, 0, 0};
    }
  }
  f32x16 adk[NDT], adv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      adk[dt][j] = 0.f;
      adv[dt][j] = 0.f;
    }
  int tro[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) tro[dt] = tr_offset<D>(lane, dt);
  const float c2 = a.scale_log2;
  const int sink = ROWS ? 0 : a.sink;

  // Products of one step: the hg heads staged in stage st for list positions
  // r0 .. r0 + RT - 1 (rows past the chunk end read as zero, lse +inf)
  auto compute = [&](int st, int r0, int hg) __attribute__((always_inline)) {
    // this wave's 32 keys visible to every row of the step (wave-uniform):
    // the per-key test is skipped
    const int kw = k0 + wave * 32;
    const bool full = r0 + RT - 1 <= c_end &&
                      (ROWS ? kw + 31 <= s_lim[st][0]
                            : kw + 31 <= r0 && (kw + 31 < sink || kw >= s_lo[st][RT - 1]));
    for (int gg = 0; gg < hg; ++gg) {
      const DA_LDS char* qs = (const DA_LDS char*)&smem[st][0][gg][0];
      const DA_LDS char* gs = (const DA_LDS char*)&smem[st][1][gg][0];

      // S = Q K^T and dP = dO V^T (rows x keys); element e of this lane is
      // row 16 (e / 8) + 8 lg + e % 8 of the step, key `key`
      f32x16 x, y;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        x[j] = 0.f;
        y[j] = 0.f;
      }
      const int r = sigma32(ln);
      // Each MFMA pair's LDS fragments are read one pair ahead: at one wave
      // per SIMD nothing else hides a fragment read's latency, and read right
      // before its MFMA every pair waited for it (backward 35.6 -> 31.8 ms at
      // 128K keys; pinned by scheduling barriers it was slower, 37.7 ms)
      {
        u32x4 qa[2], ga[2];
        qa[0] = read_rows<D>(qs, r, 0, lg);
        ga[0] = read_rows<D>(gs, r, 0, lg);
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) {
          if (ds + 1 < NDS) {
            qa[(ds + 1) & 1] = read_rows<D>(qs, r, ds + 1, lg);
            ga[(ds + 1) & 1] = read_rows<D>(gs, r, ds + 1, lg);
          }
          x = E::mfma(qa[ds & 1], kf[ds], x);
          y = E::mfma(ga[ds & 1], vf[ds], y);
        }
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int rb = 16 * half + 8 * lg;
        const f32x4 l0 = *(const DA_LDS f32x4*)&s_lse[st][gg][rb], l1 = *(const DA_LDS f32x4*)&s_lse[st][gg][rb + 4];
        const f32x4 d0 = *(const DA_LDS f32x4*)&s_d[st][gg][rb], d1 = *(const DA_LDS f32x4*)&s_d[st][gg][rb + 4];
        const u32x4 m0 = *(const DA_LDS u32x4*)&s_lim[st][rb], m1 = *(const DA_LDS u32x4*)&s_lim[st][rb + 4];
        const u32x4 o0 = *(const DA_LDS u32x4*)&s_lo[st][rb], o1 = *(const DA_LDS u32x4*)&s_lo[st][rb + 4];
        float pv[8], dv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float le = e < 4 ? l0[e] : l1[e - 4];
          const float de = e < 4 ? d0[e] : d1[e - 4];
          const int lim = (int)(e < 4 ? m0[e] : m1[e - 4]);
          const int lo = (int)(e < 4 ? o0[e] : o1[e - 4]);
          const bool vis = full || (key <= lim && (key < sink || key >= lo));
          const int jj = 8 * half + e;
          const float p = vis ? fast_exp2(fmaf(x[jj], c2, -le)) : 0.f;
          pv[e] = p;
          dv[e] = p * (y[jj] - de);
        }
        u32x4 pf, sf;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pf[e] = E::pack2(pv[2 * e], pv[2 * e + 1]);
          sf[e] = E::pack2(dv[2 * e], dv[2 * e + 1]);
        }
        // dV^T += dO^T P and dK^T += Q^T dS for this half's 16 rows (k-step
        // `half`), the transposed fragments read one MFMA pair ahead
        u32x4 ta[2], tb[2];
        ta[0] = read_tr<D>(gs, tro[0], half);
        tb[0] = read_tr<D>(qs, tro[0], half);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          if (dt + 1 < NDT) {
            ta[(dt + 1) & 1] = read_tr<D>(gs, tro[dt + 1], half);
            tb[(dt + 1) & 1] = read_tr<D>(qs, tro[dt + 1], half);
          }
          adv[dt] = E::mfma(ta[dt & 1], pf, adv[dt]);
          adk[dt] = E::mfma(tb[dt & 1], sf, adk[dt]);
        }
      }
    }   // heads of the step
  };

  if (ROWS && !a.q32) {
    for (int r0 = c_start; r0 <= c_end; r0 += RT) {
      for (int g0 = 0; g0 < a.G; g0 += HGM) {
        const int hg = min(HGM, a.G - g0);
        // stage Q and dO rows of list positions r0 .. r0 + RT - 1 of heads
        // g0 .. g0 + hg - 1 (zero past the chunk end)
        for (int slot = tid; slot < hg * RT * DCH; slot += NTHR) {
          const int gg = slot / (RT * DCH), rem = slot % (RT * DCH);
          const int rr = rem / DCH, pc = rem % DCH;
          const int h = hk * a.G + g0 + gg;
          const int i = r0 + rr;
          const bool ok = i <= c_end;
          u32x4 qv = {0, 0, 0, 0}, gv = {0, 0, 0, 0};
          if (ok) {
            const int qrow = (int)min(max(a.q_rows[i], (int64_t)0), (int64_t)(a.n_q - 1));
            qv = *(const u32x4*)((const char*)a.q + ((int64_t)b * a.qs_b + (int64_t)h * a.qs_h + (int64_t)qrow * a.qs_s) * esz + pc * 16);
            gv = *(const u32x4*)((const char*)a.dout + ((int64_t)b * a.gs_b + (int64_t)h * a.gs_h + (int64_t)i * a.gs_s) * esz + pc * 16);
          }
          *(DA_LDS u32x4*)((DA_LDS char*)&smem[0][0][gg][0] + rr * RB + ((pc ^ swz<D>(rr)) * 16)) = qv;
          *(DA_LDS u32x4*)((DA_LDS char*)&smem[0][1][gg][0] + rr * RB + ((pc ^ swz<D>(rr)) * 16)) = gv;
        }
        if (tid < hg * RT) {
          const int gg = tid / RT, t = tid % RT;
          const int i = r0 + t;
          const bool ok = i <= c_end;
          const int64_t rix = ((int64_t)b * a.Hq + hk * a.G + g0 + gg) * a.n_rows + i;
          s_lse[0][gg][t] = ok ? a.lse[rix] : INFINITY;
          s_d[0][gg][t] = ok ? a.dvec[rix] : 0.f;
          if (gg == 0) {
            int lim = -1;
            if (ok) {
              const int64_t l = min(a.row_last[i], (int64_t)(a.n_kv - 1));
              lim = (int)(l < -1 ? -1 : l);
            }
            s_lim[0][t] = lim;
            s_lo[0][t] = 0;
          }
        }
        __syncthreads();
        compute(0, r0, hg);
        __syncthreads();
      }
    }
  } else {
    // steps j = (row step, head group), head groups innermost; step j's Q and
    // dO rows go to stage j & 1 by DMA: 16-byte chunk slot (c NWAVE + wave)
    // 64 + lane of the stage is [tensor][head][row][position], filled from
    // the source chunk that position holds under the swizzle. One buffer
    // resource per (tensor, head): key-sparse rows and dO from the step's
    // first row, with the range ending at the chunk's last row; selected Q
    // rows from the head's row 0, each lane at its gathered row (prefetched a
    // step ahead), rows past the chunk end out of range. Rows past the
    // chunk end and heads past the group read as zero.
    constexpr int NC = 2 * HGM * RT * DCH / NTHR;   // DMA chunks per thread per step
    static_assert(NC * NTHR == 2 * HGM * RT * DCH && (RT * DCH) % 64 == 0, "whole waves per (tensor, head)");
    // wave instructions per (tensor, head) block of the stage; when the four
    // waves' instructions c NWAVE + wave of one c fall in one block, the
    // block (hence the buffer resource) depends on c only
    constexpr int IPB = RT * DCH / 64;
    // a lane's Q chunks c cover QR distinct rows: row(c) = (rq0 + c * RPI) % RT
    constexpr int RPI = NWAVE * 64 / DCH;          // rows per instruction index step
    constexpr int QR = RT / (RPI % RT == 0 ? RT : (RPI % RT));
    static_assert(RPI % RT == 0 || RT % (RPI % RT) == 0, "row period");
    const int rq0 = (wave * 64 + lane) / DCH % RT;
    const int n_g = (a.G + HGM - 1) / HGM;
    const int n_steps = c_end >= c_start ? ((c_end - c_start) / RT + 1) * n_g : 0;
    const uint32_t qrow_b = (uint32_t)(a.qs_s * (int64_t)esz);
    const uint32_t grow_b = (uint32_t)(a.gs_s * (int64_t)esz);
    const char* qb0 = (const char*)a.q + ((int64_t)b * a.qs_b + (int64_t)hk * a.G * a.qs_h) * esz;
    const char* gb0 = (const char*)a.dout + ((int64_t)b * a.gs_b + (int64_t)hk * a.G * a.gs_h) * esz;
    // selected rows: the gathered q rows of this lane's QR rows of step j
    // (-1 past the chunk end)
    auto qrows_of = [&](int j, int (&qr)[QR]) __attribute__((always_inline)) {
      if constexpr (ROWS) {
        const int r0 = c_start + (j / n_g) * RT;
#pragma unroll
        for (int u = 0; u < QR; ++u) {
          const int i = r0 + (rq0 + u * RPI) % RT;
          qr[u] = i <= c_end ? (int)min(max(a.q_rows[i], (int64_t)0), (int64_t)(a.n_q - 1)) : -1;
        }
      }
    };
    auto issue = [&](int j, int st, const int (&qr)[QR]) __attribute__((always_inline)) {
      const int r0 = c_start + (j / n_g) * RT, g0 = (j % n_g) * HGM;
      const int hg = min(HGM, a.G - g0);
      const uint32_t nrow = (uint32_t)min(RT, c_end - r0 + 1);
      const char* qb = qb0 + ((int64_t)g0 * a.qs_h + (ROWS ? 0 : (int64_t)r0 * a.qs_s)) * esz;
      const char* gb = gb0 + ((int64_t)g0 * a.gs_h + (int64_t)r0 * a.gs_s) * esz;
      const uint32_t qrange = ROWS ? (uint32_t)a.n_q * qrow_b : nrow * qrow_b;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int slot = (c * NWAVE + wave) * 64 + lane;
        const int row = (slot / DCH) % RT, pc = slot % DCH;
        int blk;
        if constexpr (IPB % NWAVE == 0) blk = c / (IPB / NWAVE);
        else blk = (c * NWAVE + wave) / IPB;
        const int tensor = blk / HGM, gg = blk % HGM;
        const uint32_t chunk = (uint32_t)((pc ^ swz<D>(row)) * 16);
        const char* base;
        uint32_t range, voff;
        if (tensor == 0) {
          base = qb + (int64_t)gg * a.qs_h * esz;
          range = gg < hg ? qrange : 0u;
          if constexpr (ROWS) {
            const int q = qr[c % QR];
            voff = q >= 0 ? (uint32_t)q * qrow_b + chunk : 0xfffffff0u;
          } else {
            voff = (uint32_t)row * qrow_b + chunk;
          }
        } else {
          base = gb + (int64_t)gg * a.gs_h * esz;
          range = gg < hg ? nrow * grow_b : 0u;
          voff = (uint32_t)row * grow_b + chunk;
        }
        dma16(make_rsrc(base, range), (DA_LDS void*)((DA_LDS char*)&smem[st][0][0][0] + (c * NWAVE + wave) * 1024),
              voff);
      }
    };
    // row statistics of step j (threads below HGM * RT: head tid / RT, row
    // tid % RT; the row limits from threads below RT), loaded a step ahead
    // and stored to its stage after the current step's products
    auto stat_load = [&](int j, float& l, float& dd, int& lim) __attribute__((always_inline)) {
      l = INFINITY;
      dd = 0.f;
      lim = -1;
      const int r0 = c_start + (j / n_g) * RT, g0 = (j % n_g) * HGM;
      if (tid < HGM * RT) {
        const int gg = tid / RT, i = r0 + tid % RT;
        if (i <= c_end && g0 + gg < a.G) {
          const int64_t rix = ((int64_t)b * a.Hq + hk * a.G + g0 + gg) * a.n_rows + i;
          l = a.lse[rix];
          dd = a.dvec[rix];
        }
      }
      if (tid < RT) {
        const int i = r0 + tid;
        if (i <= c_end) {
          if constexpr (ROWS) {
            const int64_t lr = min(a.row_last[i], (int64_t)(a.n_kv - 1));
            lim = (int)(lr < -1 ? -1 : lr);
          } else {
            lim = i;
          }
        }
      }
    };
    auto stat_store = [&](int j, int st, float l, float dd, int lim) __attribute__((always_inline)) {
      if (tid < HGM * RT) {
        s_lse[st][tid / RT][tid % RT] = l;
        s_d[st][tid / RT][tid % RT] = dd;
      }
      if (tid < RT) {
        s_lim[st][tid] = lim;
        s_lo[st][tid] = ROWS ? 0 : win_lo(c_start + (j / n_g) * RT + tid, a.q_block, a.window);
      }
    };
    if (n_steps > 0) {
      float l, dd;
      int lim;
      int qr[QR], qn[QR];
      qrows_of(0, qr);
      stat_load(0, l, dd, lim);
      if (n_steps > 1) qrows_of(1, qn);
      issue(0, 0, qr);
      stat_store(0, 0, l, dd, lim);
      wait_dma();
      __syncthreads();
      for (int j = 0; j < n_steps; ++j) {
        const int st = j & 1;
        const bool more = j + 1 < n_steps;
        // stage st ^ 1 was last read in step j - 1, before the barrier
        if (more) {
#pragma unroll
          for (int u = 0; u < QR; ++u) qr[u] = qn[u];
          if (j + 2 < n_steps) qrows_of(j + 2, qn);
          stat_load(j + 1, l, dd, lim);
          issue(j + 1, st ^ 1, qr);
        }
        compute(st, c_start + (j / n_g) * RT, min(HGM, a.G - (j % n_g) * HGM));
        if (more) stat_store(j + 1, st ^ 1, l, dd, lim);
        wait_dma();
        __syncthreads();
      }
    }
  }

  // A block whose rows are one item writes its dK (scaled by sm_scale) and
  // dV directly, as the reduce would from a single partial (the same bits);
  // a block of several items writes partials [2][KT][D] for the reduce.
  if ((blk < a.nsb ? a.ncs : a.nco) == 1) {
    if (key >= a.n_kv) return;
    u32x2* ok = (u32x2*)((char*)a.dk + ((int64_t)b * a.dks_b + (int64_t)hk * a.dks_h + (int64_t)key * a.dks_s) * esz);
    u32x2* ov = (u32x2*)((char*)a.dv + ((int64_t)b * a.dvs_b + (int64_t)hk * a.dvs_h + (int64_t)key * a.dvs_s) * esz);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const int d4 = (32 * dt + 8 * jq + 4 * lg) / 4;
        const u32x2 pk0 = a.accumulate ? ok[d4] : (u32x2){0, 0};
        const u32x2 pv0 = a.accumulate ? ov[d4] : (u32x2){0, 0};
        u32x2 nk, nv;
        nk[0] = acc_pack<T>(pk0[0], adk[dt][4 * jq] * a.sm_scale, adk[dt][4 * jq + 1] * a.sm_scale, a.accumulate);
        nk[1] = acc_pack<T>(pk0[1], adk[dt][4 * jq + 2] * a.sm_scale, adk[dt][4 * jq + 3] * a.sm_scale, a.accumulate);
        nv[0] = acc_pack<T>(pv0[0], adv[dt][4 * jq], adv[dt][4 * jq + 1], a.accumulate);
        nv[1] = acc_pack<T>(pv0[1], adv[dt][4 * jq + 2], adv[dt][4 * jq + 3], a.accumulate);
        ok[d4] = nk;
        ov[d4] = nv;
      }
    return;
  }
  // (those items come first in a (batch, kv head)'s item order: every item
  // when the window blocks are cut too, else the sink blocks' items)
  float* pk = a.kv_part + ((int64_t)bh * a.part_per_bh + item) * 2 * KT * D + (int64_t)(wave * 32 + ln) * D;
  float* pv = pk + (int64_t)KT * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const int d = 32 * dt + 8 * jq + 4 * lg;
      *(f32x4*)(pk + d) = (f32x4){adk[dt][4 * jq] * a.sm_scale, adk[dt][4 * jq + 1] * a.sm_scale,
                                  adk[dt][4 * jq + 2] * a.sm_scale, adk[dt][4 * jq + 3] * a.sm_scale};
      *(f32x4*)(pv + d) = (f32x4){adv[dt][4 * jq], adv[dt][4 * jq + 1],
                                  adv[dt][4 * jq + 2], adv[dt][4 * jq + 3]};
    }
}

// dK, dV of the keys of blocks cut into several items (every key, or the
// sink blocks' keys 0 .. red_keys - 1 when only those are): the sum of its
// block's chunk partials, 8 dims per thread.
template <typename T, int D>
__global__ __launch_bounds__(RED) void dkdv_reduce_kernel(BwdArgs a) {
  constexpr int CPR = D / 8;
  const int64_t task = (int64_t)blockIdx.x * RED + threadIdx.x;
  const int64_t per_bh = (int64_t)a.red_keys * CPR;
  if (task >= (int64_t)a.B * a.Hkv * per_bh) return;
  const int bh = (int)(task / per_bh);
  const int rem = (int)(task % per_bh);
  const int key = rem / CPR, c = rem % CPR;
  const int blk = key / KT, kl = key % KT;
  int first, cnt;
  if (blk < a.nsb) {
    first = blk * a.ncs;
    cnt = a.ncs;
  } else {
    first = a.nsb * a.ncs + (blk - a.nsb) * a.nco;
    cnt = a.nco;
  }
  if (cnt == 1) return;   // written by its dkdv item
  float sk[8], sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sk[e] = 0.f;
    sv[e] = 0.f;
  }
  for (int it = 0; it < cnt; ++it) {
    const float* p = a.kv_part + ((int64_t)bh * a.part_per_bh + first + it) * 2 * KT * D +
                     (int64_t)kl * D + 8 * c;
    const f32x4 k0 = ((const f32x4*)p)[0], k1 = ((const f32x4*)p)[1];
    const f32x4 v0 = ((const f32x4*)(p + KT * D))[0], v1 = ((const f32x4*)(p + KT * D))[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sk[e] += k0[e];
      sk[4 + e] += k1[e];
      sv[e] += v0[e];
      sv[4 + e] += v1[e];
    }
  }
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  u32x4* pk = (u32x4*)((char*)a.dk + ((int64_t)b * a.dks_b + (int64_t)hk * a.dks_h + (int64_t)key * a.dks_s + 8 * c) * sizeof(T));
  u32x4* pv = (u32x4*)((char*)a.dv + ((int64_t)b * a.dvs_b + (int64_t)hk * a.dvs_h + (int64_t)key * a.dvs_s + 8 * c) * sizeof(T));
  const u32x4 ok = a.accumulate ? *pk : (u32x4){0, 0, 0, 0};
  const u32x4 ov = a.accumulate ? *pv : (u32x4){0, 0, 0, 0};
  u32x4 nk, nv;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    nk[e] = acc_pack<T>(ok[e], sk[2 * e], sk[2 * e + 1], a.accumulate);
    nv[e] = acc_pack<T>(ov[e], sv[2 * e], sv[2 * e + 1], a.accumulate);
  }
  *pk = nk;
  *pv = nv;
}

// ---------------------------------------------------------------------------
// Backward of the composition out[r] = sparse[r] + delta[r / gamma] (r < s_p),
// delta = dense_anchor - sparse[anchors], out[s_p + t] = dense_tail[t]:
//   ddelta[i] = rnd(scale * rnd(sum_j grad[i gamma + j]))  (0 when detached)
//   dsparse[r] = grad[r] for r < s_p, rnd(grad[r] - ddelta[i]) at anchor r = i gamma,
//                0 for r >= s_p
//   ddense[i] = ddelta[i] (i < n_anchor), ddense[n_anchor + t] = grad[s_p + t]
struct ComposeArgs {
  const void* g;
  int64_t gs_b, gs_h, gs_s;
  void* dsp;
  int64_t ss_b, ss_h, ss_s;
  void* dd;
  int64_t ds_b, ds_h, ds_s;
  int B, H, S, D, gamma, s_p, n_anchor;
  float scale;
  int detach;
};

template <typename T>
__global__ __launch_bounds__(RED) void compose_bwd_kernel(ComposeArgs a) {
  using E = Elt<T>;
  const int cpr = a.D / 8;
  const int n_units = a.n_anchor + (a.S - a.s_p);   // anchor groups, then tail rows
  const int64_t task = (int64_t)blockIdx.x * RED + threadIdx.x;
  if (task >= (int64_t)a.B * n_units * a.H * cpr) return;
  const int c = (int)(task % cpr);
  const int h = (int)((task / cpr) % a.H);
  const int u = (int)((task / cpr / a.H) % n_units);
  const int b = (int)(task / cpr / a.H / n_units);
  const size_t esz = sizeof(T);
  auto gp = [&](int r) {
    return (const u32x4*)((const char*)a.g + ((int64_t)b * a.gs_b + (int64_t)h * a.gs_h + (int64_t)r * a.gs_s + 8 * c) * esz);
  };
  auto sp = [&](int r) {
    return (u32x4*)((char*)a.dsp + ((int64_t)b * a.ss_b + (int64_t)h * a.ss_h + (int64_t)r * a.ss_s + 8 * c) * esz);
  };
  u32x4* dp = (u32x4*)((char*)a.dd + ((int64_t)b * a.ds_b + (int64_t)h * a.ds_h + (int64_t)u * a.ds_s + 8 * c) * esz);
  if (u >= a.n_anchor) {
    const int r = a.s_p + (u - a.n_anchor);
    *dp = *gp(r);
    *sp(r) = (u32x4){0, 0, 0, 0};
    return;
  }
  const int r0 = u * a.gamma;
  float s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.f;
  for (int j = 0; j < a.gamma; ++j) {
    const u32x4 x = *gp(r0 + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[2 * e] += E::lo(x[e]);
      s[2 * e + 1] += E::hi(x[e]);
    }
    if (j > 0) *sp(r0 + j) = x;
  }
  u32x4 dl;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t w = E::pack2(s[2 * e], s[2 * e + 1]);
    if (a.scale != 1.f) w = E::pack2(E::lo(w) * a.scale, E::hi(w) * a.scale);
    dl[e] = a.detach ? 0u : w;
  }
  *dp = dl;
  const u32x4 x0 = *gp(r0);
  u32x4 s0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    s0[e] = a.detach ? x0[e] : E::pack2(E::lo(x0[e]) - E::lo(dl[e]), E::hi(x0[e]) - E::hi(dl[e]));
  *sp(r0) = s0;
}

}  // namespace bwd
}  // namespace da

using namespace da;
using namespace da::bwd;

namespace {

struct DqPlan {
  int n_mtiles, n_splits, chunk;
};

// Key tiles per dq item: key-sparse rows take their whole (window-sized)
// list; selected rows split lists longer than 64 tiles into about 4096 items.
DqPlan plan_dq(int B, int Hkv, int G, int n_rows, int64_t list_tiles, bool rows) {
  DqPlan p;
  p.n_mtiles = (int)(((int64_t)n_rows * G + BM - 1) / BM);
  if (!rows) {
    p.n_splits = 1;
    p.chunk = 1 << 30;
    return p;
  }
  if (list_tiles < 1) list_tiles = 1;
  int64_t want = 1;
  if (list_tiles > 64) {
    const int64_t base = (int64_t)B * Hkv * p.n_mtiles;
    want = (4096 + base - 1) / base;
    want = std::min<int64_t>(std::max<int64_t>(want, 1), (list_tiles + 63) / 64);
  }
  p.chunk = (int)((list_tiles + want - 1) / want);
  p.n_splits = (int)((list_tiles + p.chunk - 1) / p.chunk);
  return p;
}

struct KvPlan {
  int n_blk, nsb, ncs, nco, rpc, items_per_bh;
  int part_per_bh;   // items whose block is cut into several (they write partials)
};

// Rows per dK/dV chunk at most (process-wide; da_set_bwd_rows_per_chunk).
static std::atomic<int> g_rpc_max{RPC_MAX};

// A block's rows are cut into equal chunks of at most the cap: with a fixed
// chunk of the cap, a span just past it left a chunk of a few rows per block
// (window 4096: 4096 + 128 rows), each a whole item with its K/V loads and
// dK/dV partials (Qwen3 64K x 2 backward 102 ms; 66 ms with one 4224-row
// chunk per block).
KvPlan plan_kv(int n_rows, int n_kv, int window, int sink, bool rows) {
  KvPlan p;
  p.n_blk = (n_kv + KT - 1) / KT;
  const int64_t cap = g_rpc_max.load(std::memory_order_relaxed);
  auto up = [](int64_t x) { return (int)(((x + RT - 1) / RT) * RT); };
  auto split = [&](int64_t span, int& rpc, int& n) {
    span = std::max<int64_t>(span, 1);
    const int64_t k = (span + cap - 1) / cap;
    rpc = up((span + k - 1) / k);
    n = (int)((span + rpc - 1) / rpc);
  };
  if (rows) {
    p.nsb = 0;
    split(n_rows, p.rpc, p.nco);
    p.ncs = 1;
  } else {
    p.nsb = std::min(p.n_blk, (sink + KT - 1) / KT);
    split((int64_t)KT + window, p.rpc, p.nco);   // rows a non-sink block can need
    p.ncs = (n_rows + p.rpc - 1) / p.rpc;
    if (p.ncs < 1) p.ncs = 1;
  }
  p.items_per_bh = p.nsb * p.ncs + (p.n_blk - p.nsb) * p.nco;
  p.part_per_bh = p.nco > 1 ? p.items_per_bh : p.ncs > 1 ? p.nsb * p.ncs : 0;
  return p;
}

// Workspace: rowsum(dO * O) [B, Hq, n_rows] fp32; the dq split partials; the
// dkdv partials.
size_t bwd_ws_bytes(int B, int Hq, int Hkv, int n_rows, int n_kv, int D, const DqPlan& dq,
                    const KvPlan& kv, bool rows, size_t esz = 2) {
  size_t bytes = (size_t)B * Hq * n_rows * sizeof(float);        // rowsum(dO * O)
  bytes = (bytes + 255) / 256 * 256;
  if (dq.n_splits > 1)
    bytes += (size_t)B * Hkv * dq.n_splits * dq.n_mtiles * BM * D * sizeof(float);
  bytes = (bytes + 255) / 256 * 256;
  bytes += (size_t)B * Hkv * kv.part_per_bh * 2 * KT * D * sizeof(float);
  (void)rows;
  (void)esz;
  return bytes;
}

template <typename T, int D, bool ROWS>
void launch_bwd(const BwdArgs& a, hipStream_t s) {
  const int gq = a.B * a.Hkv * a.n_mtiles * a.n_splits;
  hipLaunchKernelGGL((dq_kernel<T, D, ROWS>), dim3((gq + 7) / 8 * 8), dim3(NTHR), 0, s, a);
  if (a.n_splits > 1) {
    const int64_t tasks = (int64_t)a.B * a.Hkv * a.n_mtiles * BM * (D / 8);
    hipLaunchKernelGGL((dq_reduce_kernel<T, D, ROWS>), dim3((unsigned)((tasks + RED - 1) / RED)),
                       dim3(RED), 0, s, a);
  }
  const int gk = a.B * a.Hkv * a.items_per_bh;
  hipLaunchKernelGGL((dkdv_kernel<T, D, ROWS>), dim3((gk + 7) / 8 * 8), dim3(NTHR), 0, s, a);
  const int64_t tasks = (int64_t)a.B * a.Hkv * a.red_keys * (D / 8);
  if (tasks > 0)
    hipLaunchKernelGGL((dkdv_reduce_kernel<T, D>), dim3((unsigned)((tasks + RED - 1) / RED)),
                       dim3(RED), 0, s, a);
}

template <bool ROWS>
int dispatch_bwd(const BwdArgs& a, int D, int dtype, hipStream_t s) {
  (void)hipGetLastError();
  if (dtype == DA_BF16) {
    if (D == 128) launch_bwd<__bf16, 128, ROWS>(a, s);
    else if (D == 64) launch_bwd<__bf16, 64, ROWS>(a, s);
    else launch_bwd<__bf16, 32, ROWS>(a, s);
  } else {
    if (D == 128) launch_bwd<_Float16, 128, ROWS>(a, s);
    else if (D == 64) launch_bwd<_Float16, 64, ROWS>(a, s);
    else launch_bwd<_Float16, 32, ROWS>(a, s);
  }
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

bool ok3(const int64_t* s) { return s && strides8(s); }

// Common argument block; returns DA_OK or an error code.
int bwd_args(BwdArgs& a, const void* q, const void* k, const void* v, const void* o,
             const void* dout, const float* lse, void* dq, void* dk, void* dv,
             int B, int Hq, int Hkv, int n_rows, int n_q, int n_kv, int D,
             const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
             const int64_t o_str[3], const int64_t do_str[3], const int64_t dq_str[3],
             const int64_t dk_str[3], const int64_t dv_str[3], float sm_scale, int accumulate,
             int dtype) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (D > 128) return DA_ERR_HEAD_DIM;   // the backward kernels take 32, 64 and 128
  if (n_rows < 1 || n_q < 1 || n_kv < 1) return DA_ERR_INVALID_ARG;
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv) return DA_ERR_INVALID_ARG;
  if (!ok3(q_str) || !ok3(k_str) || !ok3(v_str) || !ok3(o_str) || !ok3(do_str) ||
      !ok3(dq_str) || !ok3(dk_str) || !ok3(dv_str))
    return q_str && k_str && v_str && o_str && do_str && dq_str && dk_str && dv_str
               ? DA_ERR_ALIGNMENT : DA_ERR_INVALID_ARG;
  const void* ps[] = {q, k, v, o, dout, dq, dk, dv};
  for (const void* p : ps)
    if (!aligned16(p)) return DA_ERR_ALIGNMENT;
  if (((uintptr_t)lse & 3u) != 0) return DA_ERR_ALIGNMENT;
  // the DMA tiles address rows with 32-bit byte offsets
  const int64_t rs[] = {q_str[2], k_str[2], v_str[2], do_str[2]};
  for (int64_t r : rs)
    if (r < D || r >= (1 << 23)) return DA_ERR_INVALID_ARG;
  a = BwdArgs{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.lse = lse;
  a.dq = dq; a.dk = dk; a.dv = dv;
  a.qs_b = q_str[0]; a.qs_h = q_str[1]; a.qs_s = q_str[2];
  a.ks_b = k_str[0]; a.ks_h = k_str[1]; a.ks_s = k_str[2];
  a.vs_b = v_str[0]; a.vs_h = v_str[1]; a.vs_s = v_str[2];
  a.os_b = o_str[0]; a.os_h = o_str[1]; a.os_s = o_str[2];
  a.gs_b = do_str[0]; a.gs_h = do_str[1]; a.gs_s = do_str[2];
  a.dqs_b = dq_str[0]; a.dqs_h = dq_str[1]; a.dqs_s = dq_str[2];
  a.dks_b = dk_str[0]; a.dks_h = dk_str[1]; a.dks_s = dk_str[2];
  a.dvs_b = dv_str[0]; a.dvs_h = dv_str[1]; a.dvs_s = dv_str[2];
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv;
  a.n_rows = n_rows; a.n_q = n_q; a.n_kv = n_kv;
  a.sm_scale = sm_scale;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.accumulate = accumulate ? 1 : 0;
  return DA_OK;
}

}  // namespace

extern "C" int da_set_bwd_rows_per_chunk(int rows) {
  if (rows == 0) rows = RPC_MAX;
  if (rows < RT || rows % RT != 0 || rows > (1 << 20)) return DA_ERR_INVALID_ARG;
  g_rpc_max.store(rows, std::memory_order_relaxed);
  return DA_OK;
}

extern "C" size_t da_sparse_attn_bwd_workspace_bytes(int B, int Hq, int Hkv, int S, int D,
                                                     int window, int sink, int q_block) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || S < 1 || q_block < 1 || window < 0 ||
      sink < 0 || (D != 32 && D != 64 && D != 128))
    return 0;
  const DqPlan dq = plan_dq(B, Hkv, Hq / Hkv, S, 0, false);
  const KvPlan kv = plan_kv(S, S, window, sink, false);
  return bwd_ws_bytes(B, Hq, Hkv, S, S, D, dq, kv, false);
}

extern "C" size_t da_qsparse_attn_bwd_workspace_bytes(int B, int Hq, int Hkv, int n, int Skv, int D) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || n < 1 || Skv < 1 ||
      (D != 32 && D != 64 && D != 128))
    return 0;
  const int bn = D == 128 ? 32 : 64;
  const DqPlan dq = plan_dq(B, Hkv, Hq / Hkv, n, ((int64_t)Skv + bn - 1) / bn, true);
  const KvPlan kv = plan_kv(n, Skv, 0, 0, true);
  return bwd_ws_bytes(B, Hq, Hkv, n, Skv, D, dq, kv, true);
}

static void place_workspace(BwdArgs& a, const DqPlan& dq, const KvPlan& kv, int D, void* ws,
                            bool rows) {
  a.n_mtiles = dq.n_mtiles; a.n_splits = dq.n_splits; a.chunk = dq.chunk;
  a.n_blk = kv.n_blk; a.nsb = kv.nsb; a.ncs = kv.ncs; a.nco = kv.nco; a.rpc = kv.rpc;
  a.items_per_bh = kv.items_per_bh;
  a.red_keys = kv.nco > 1 ? a.n_kv : kv.ncs > 1 ? std::min(a.n_kv, kv.nsb * KT) : 0;
  a.part_per_bh = kv.part_per_bh;
  char* p = (char*)ws;
  size_t off = (size_t)a.B * a.Hq * a.n_rows * sizeof(float);
  off = (off + 255) / 256 * 256;
  a.dvec = (float*)p;
  a.dq_part = (float*)(p + off);
  if (dq.n_splits > 1) off += (size_t)a.B * a.Hkv * dq.n_splits * dq.n_mtiles * BM * D * sizeof(float);
  off = (off + 255) / 256 * 256;
  a.kv_part = (float*)(p + off);
  (void)rows;
}

extern "C" int da_sparse_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                                  const void* dout, const float* lse,
                                  void* dq, void* dk, void* dv,
                                  int B, int Hq, int Hkv, int S, int D,
                                  const int64_t q_str[3], const int64_t k_str[3],
                                  const int64_t v_str[3], const int64_t o_str[3],
                                  const int64_t do_str[3], const int64_t dq_str[3],
                                  const int64_t dk_str[3], const int64_t dv_str[3],
                                  int window, int sink, int q_block, float sm_scale,
                                  int accumulate, void* workspace, size_t workspace_bytes,
                                  int dtype, void* stream) {
  if (window < 0 || sink < 0 || q_block < 1) return DA_ERR_INVALID_ARG;
  BwdArgs a;
  int rc = bwd_args(a, q, k, v, o, dout, lse, dq, dk, dv, B, Hq, Hkv, S, S, S, D, q_str, k_str,
                    v_str, o_str, do_str, dq_str, dk_str, dv_str, sm_scale, accumulate, dtype);
  if (rc != DA_OK) return rc;
  a.window = window; a.sink = sink; a.q_block = q_block;
  const DqPlan dqp = plan_dq(B, Hkv, a.G, S, 0, false);
  const KvPlan kvp = plan_kv(S, S, window, sink, false);
  const size_t need = bwd_ws_bytes(B, Hq, Hkv, S, S, D, dqp, kvp, false);
  if (!workspace || workspace_bytes < need) return DA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DA_ERR_ALIGNMENT;
  if ((int64_t)B * Hkv * kvp.items_per_bh > 0x7fffff00LL ||
      (int64_t)B * Hkv * dqp.n_mtiles * dqp.n_splits > 0x7fffff00LL)
    return DA_ERR_INVALID_ARG;
  place_workspace(a, dqp, kvp, D, workspace, false);
  return dispatch_bwd<false>(a, D, dtype, (hipStream_t)stream);
}

extern "C" int da_qsparse_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                                   const void* dout, const float* lse,
                                   const int64_t* q_rows, const int64_t* row_last, int n,
                                   void* dq, void* dk, void* dv,
                                   int B, int Hq, int Hkv, int Sq, int Skv, int D,
                                   const int64_t q_str[3], const int64_t k_str[3],
                                   const int64_t v_str[3], const int64_t o_str[3],
                                   const int64_t do_str[3], const int64_t dq_str[3],
                                   const int64_t dk_str[3], const int64_t dv_str[3],
                                   float sm_scale, int accumulate, void* workspace,
                                   size_t workspace_bytes, int dtype, void* stream) {
  if (!q_rows || !row_last) return DA_ERR_INVALID_ARG;
  BwdArgs a;
  int rc = bwd_args(a, q, k, v, o, dout, lse, dq, dk, dv, B, Hq, Hkv, n, Sq, Skv, D, q_str,
                    k_str, v_str, o_str, do_str, dq_str, dk_str, dv_str, sm_scale, accumulate,
                    dtype);
  if (rc != DA_OK) return rc;
  a.q_rows = q_rows; a.row_last = row_last;
  // the dK/dV kernel's DMA addresses a head's gathered q rows from its row 0
  // with 32-bit byte offsets (else it stages them through registers)
  a.q32 = (uint64_t)a.n_q * (uint64_t)a.qs_s * 2u <= 0xfffff000ull;
  a.window = 0; a.sink = 0; a.q_block = 1;
  const int bn = D == 128 ? 32 : 64;
  const DqPlan dqp = plan_dq(B, Hkv, a.G, n, ((int64_t)Skv + bn - 1) / bn, true);
  const KvPlan kvp = plan_kv(n, Skv, 0, 0, true);
  const size_t need = bwd_ws_bytes(B, Hq, Hkv, n, Skv, D, dqp, kvp, true);
  if (!workspace || workspace_bytes < need) return DA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DA_ERR_ALIGNMENT;
  if ((int64_t)B * Hkv * kvp.items_per_bh > 0x7fffff00LL ||
      (int64_t)B * Hkv * dqp.n_mtiles * dqp.n_splits > 0x7fffff00LL)
    return DA_ERR_INVALID_ARG;
  place_workspace(a, dqp, kvp, D, workspace, true);
  return dispatch_bwd<true>(a, D, dtype, (hipStream_t)stream);
}

extern "C" int da_delta_compose_bwd(const void* grad, const int64_t g_str[3],
                                    void* dsparse, const int64_t sp_str[3],
                                    void* ddense, const int64_t dd_str[3],
                                    int B, int H, int S, int D, int gamma, int s_p,
                                    float delta_grad_scale, int detach_delta,
                                    int dtype, void* stream) {
  if (dtype != DA_BF16 && dtype != DA_FP16) return DA_ERR_DTYPE;
  if (D != 32 && D != 64 && D != 128) return DA_ERR_HEAD_DIM;
  if (B < 1 || H < 1 || S < 1 || gamma < 1 || s_p < 0 || s_p > S || s_p % gamma != 0)
    return DA_ERR_INVALID_ARG;
  if (!grad || !dsparse || !ddense || !g_str || !sp_str || !dd_str) return DA_ERR_INVALID_ARG;
  if (!aligned16(grad) || !aligned16(dsparse) || !aligned16(ddense) || !strides8(g_str) ||
      !strides8(sp_str) || !strides8(dd_str))
    return DA_ERR_ALIGNMENT;
  ComposeArgs c{};
  c.g = grad; c.gs_b = g_str[0]; c.gs_h = g_str[1]; c.gs_s = g_str[2];
  c.dsp = dsparse; c.ss_b = sp_str[0]; c.ss_h = sp_str[1]; c.ss_s = sp_str[2];
  c.dd = ddense; c.ds_b = dd_str[0]; c.ds_h = dd_str[1]; c.ds_s = dd_str[2];
  c.B = B; c.H = H; c.S = S; c.D = D; c.gamma = gamma; c.s_p = s_p; c.n_anchor = s_p / gamma;
  c.scale = delta_grad_scale; c.detach = detach_delta ? 1 : 0;
  const int64_t tasks = (int64_t)B * (c.n_anchor + (S - s_p)) * H * (D / 8);
  if (tasks == 0) return DA_OK;
  (void)hipGetLastError();
  const unsigned grid = (unsigned)((tasks + RED - 1) / RED);
  if (dtype == DA_BF16)
    hipLaunchKernelGGL((compose_bwd_kernel<__bf16>), dim3(grid), dim3(RED), 0, (hipStream_t)stream, c);
  else
    hipLaunchKernelGGL((compose_bwd_kernel<_Float16>), dim3(grid), dim3(RED), 0, (hipStream_t)stream, c);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

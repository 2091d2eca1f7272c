// Attention kernels of the delta-attention path on gfx950:
//   kernel (1)  da_sparse_attn_fwd   sink + block-anchored sliding window;
//               da_sparse_attn_delta_fwd  the same with the delta broadcast-add
//                                    (kernel (3)) in its epilogue
//   kernel (2)  da_qsparse_attn_fwd  selected query rows against their causal
//                                    keys (optionally sinks + a window: the
//                                    decode rows of da_decode_attn_fwd), split
//                                    over each row tile's key-tile list,
//                                    merged by qsparse_merge_kernel, which also
//                                    runs the output / delta / dense epilogues.
//
// Tiling (one workgroup = 4 waves = 256 threads):
//   * M tile: BM flattened (query row, head-in-group) pairs. The G query heads
//     that share one key/value head are packed into the same tile, so K/V
//     tiles are read once per group (no repeat_kv copies).
//   * Each wave owns RG groups of 32 flattened rows. RG = 2 at head_dim 128
//     (64 rows per wave, BM = 256, one workgroup and one wave per SIMD per CU):
//     every K and V fragment read from LDS feeds one MFMA per row group, half
//     the LDS bytes per MFMA of RG = 1 (32 rows per wave, BM = 128, two
//     workgroups per CU), which the other head dims and the decode rows use.
//   * Scores are formed transposed, S^T = K * Q^T, with v_mfma_f32_32x32x16
//     (A = 32 keys x 16 dims from LDS, B = Q^T fragment kept in registers). In
//     the 32x32 accumulator layout a lane holds one query row (lane % 32) of
//     each row group and 16 of its keys, so the softmax row max/sum is in-lane
//     plus one permlane32 swap.
//   * O^T = V^T * P^T: the probabilities leave the score accumulator directly
//     as the B operand, and the O^T accumulator again keeps one query row per
//     lane, so the online-softmax rescale is a per-lane scalar.
//   * K/V tiles go global -> LDS by buffer-load DMA (no registers, no VALU
//     address math: one scalar buffer base per tile, hardware zero-fill past
//     the last key), double-buffered: the next tile is in flight while the
//     current one is consumed. XOR chunk swizzles applied on the source side
//     make the LDS fragment reads bank-conflict free.
//   * K A-fragments read rows in a bit-permuted order (sigma) so that each
//     lane's 8 keys per PV step are contiguous; V stays row-major in LDS and
//     its V^T A-fragments come from transposed reads (ds_read_b64_tr_b16).
//   * Softmax: one FMA + exp2 per score, row sum by v_dot2 over the packed P.
//     Lazy rescale: the running max only moves when a row's tile max exceeds
//     it by more than a bound (log2 domain: 40 for bf16, 15 for fp16, whose
//     packed probabilities must stay below 65504). The first pass over the
//     tiles takes no per-tile row max once every row has its first max; a row
//     sum above half of 2^bound (a max that would have moved) sends the
//     workgroup through a second, exact pass, whose bits equal the first
//     pass's for every other row.
//   * Per key tile, one scheduling region keeps the matrix pipe fed: the
//     exponentials of tile t run under the score MFMAs of tile t+1, then the
//     PV MFMAs of tile t follow with their V reads running ahead.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "device_common.h"
#include "agpr_tiles.h"
#include "capi_common.h"

namespace da {

// Split items a selected-rows launch aims for.
#ifndef DA_ROWS_ITEMS
#define DA_ROWS_ITEMS 8192
#endif
// Shortest split item of a selected-rows launch, in key tiles (binding on
// short launches such as 638 rows at 32K: 40 / 48 / 56 / 64 / 80 tiles ->
// kernel (2) 0.255 / 0.258 / 0.243 / 0.254 / 0.260 ms).
#ifndef DA_ROWS_MIN_TILES
#define DA_ROWS_MIN_TILES 56
#endif
// Longest split item of a selected-rows launch, in key tiles: past 256K keys
// the item target alone would give items of thousands of tiles, and the
// longest ones, dispatched last, would run alone at the end of the launch.
#ifndef DA_ROWS_MAX_TILES
#define DA_ROWS_MAX_TILES 512
#endif
// Split items a decode-row launch aims for: one workgroup per resident slot
// of the 256-CU gfx950 (two per CU), so the items run in a single round
// (dense row over 131072 keys: 106-111 us against 118 us at 1024 items and
// 131 us at 2048).
#ifndef DA_DECODE_ITEMS
#define DA_DECODE_ITEMS 512
#endif
// Row groups per wave of the head_dim-128 key-sparse launches (the default
// of da_set_sparse_rows_per_wave) and of the selected-rows launches (1 or 2).
#ifndef DA_RG_SPARSE
#define DA_RG_SPARSE 1
#endif
#ifndef DA_RG_ROWS
#define DA_RG_ROWS 1
#endif
constexpr int NWAVE = 4;
constexpr int NTHR = 64 * NWAVE;
constexpr int BN = 64;               // keys per tile
constexpr int NH = BN / 32;          // 32-key halves per tile
constexpr int MTHR = 256;            // threads of the split-merge kernel
constexpr int NSTAGE = 2;            // LDS stages for K and for V
constexpr int BM_MAX = 32 * NWAVE * 2;
constexpr int bm_of(int rg) { return 32 * NWAVE * rg; }   // flattened (row, head) pairs per workgroup
constexpr float NEG_BIG = -1.0e30f;  // finite "minus infinity" for the running max

// Lazy-rescale bound (log2 domain): a row's running max moves only when a
// tile's max exceeds it by more than `thresh`, so P <= 2^thresh and
// l <= 2^thresh * keys. A row sum above lsum / 2 tells the tile loop that ran
// without row maxima that a max would have moved (P <= l). The probabilities
// are packed into the element type for the PV product: fp16 holds at most
// 65504, so its bound is 15.
template <typename T> struct Rescale;
template <> struct Rescale<__bf16> {
  static constexpr float thresh = 40.0f;
  static constexpr float lsum = 1099511627776.0f;   // 2^40
};
template <> struct Rescale<_Float16> {
  static constexpr float thresh = 15.0f;
  static constexpr float lsum = 32768.0f;           // 2^15
};

// MODE_FUSED is MODE_SPARSE with the delta broadcast-add in its epilogue.
enum { MODE_SPARSE = 0, MODE_QSPARSE = 1, MODE_FUSED = 2 };

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t qs_b, qs_h, qs_s;
  int64_t ks_b, ks_h, ks_s;
  int64_t vs_b, vs_h, vs_s;
  void* o;
  int64_t os_b, os_h, os_s;
  int B, Hq, Hkv, G;
  int Gs, n_hs;     // key-sparse mode: query heads per row tile (Gs | G), G / Gs head splits
  int n_rows;       // query rows per (batch, head)
  int n_q;          // rows of q (selected rows index into it)
  int n_kv;         // keys
  int bm;           // flattened (row, head) pairs per workgroup: bm_of(RG) of the launch
  int n_mtiles;     // ceil(n_rows * G / bm)
  int n_items;      // work items before padding the grid to a multiple of 8
  float scale_log2; // sm_scale * log2(e)
  int window, sink, q_block;
  int row0;         // key-sparse mode: query row of local row 0 (rows row0 .. row0 + n_rows - 1)
  const int64_t* q_rows;
  const int64_t* row_last;
  int64_t rl_b;
  int chunk;        // query-sparse mode: key tiles of the tile list per split item
  int n_splits;
  // query-sparse mode: when set, the key count is *n_kv_dev (clamped to
  // [1, n_kv]) and chunk = ceil(list / n_splits): the launch stays valid as a
  // cache grows (decode rows under graph replay)
  const int* n_kv_dev;
  // query-sparse mode: when set, only the first *n_rows_dev rows (clamped to
  // [0, n_rows]) are computed; the items of their row tiles are spread over
  // the XCDs in contiguous ranges and the other blocks exit at once
  const int* n_rows_dev;
  uint32_t* part_o; // [item][ws_rows][D / 2]: element pairs of each row's O / l
  float* part_ml;   // [item][2][ws_rows]  (running max, row sum)
  int ws_rows;      // workspace rows per item: min(bm, n_rows * G) (a tile's valid rows)
  // MODE_FUSED: dense anchor rows [B, n_anchor, Hq, D] (strides batch, head,
  // anchor), optional delta output (same layout), stride and rows < s_p
  const void* dsel;
  int64_t dsel_b, dsel_h, dsel_a;
  void* dout;
  int64_t dout_b, dout_h, dout_a;
  int gamma, s_p, n_anchor;
  // MODE_SPARSE: optional row log-sum-exp [B, Hq, n_rows] (log2 domain of the
  // scaled scores, +inf for a row without visible keys), for the backward
  float* lse;
  // divisions by the launch's fixed divisors: n_hs, n_mtiles, n_splits, Hkv,
  // Gs (heads per tile), q_block, gamma
  FastDiv fd_hs, fd_mt, fd_sp, fd_hkv, fd_gt, fd_qb, fd_gamma;
  int tile_rows;    // bm / Gs: query rows per row tile
  int n_grp;        // MODE_FUSED: stride groups per row tile (tile_rows / gamma)
};

// Bytes of LDS that hold a fused tile's dense anchor rows, prefetched with the
// first K/V tiles (tiles with more anchor rows read them in the epilogue).
// Row slot s is DMA'd by wave s % 4 into its block of dpre, at row s / 4 of
// it; the four blocks are DPAD bytes more than 1 KB apart, so the anchor
// lanes of consecutive slots (the heads of a group) read different banks.
constexpr int DPRE_BYTES = 4096;
// The deltas those rows give, one 16-byte-padded slot per (group, head): the
// lanes of a wave read the slots of two heads at once, which the padding puts
// on different LDS banks.
constexpr int DPAD = 16;
constexpr int DLT_BYTES = DPRE_BYTES + 64 * DPAD;
constexpr int DPRE_BLOCK = DPRE_BYTES / 4 + DPAD;   // one wave's block of dpre

// sigma: swaps bits 2 and 3 of a key index within a 32-key half tile. Using
// K row sigma(r) as A-operand row r puts keys 8*g .. 8*g+7 (g = lane / 32) in
// accumulator elements 0..7 of every lane, the order the PV step consumes.
__device__ __forceinline__ int sigma32(int r) {
  return (r & 0x13) | ((r & 4) << 1) | ((r & 8) >> 1);
}

template <int D>
struct Tile {
  static constexpr int DCH = D / 8;          // 16-byte chunks per row
  static constexpr int RB = D * 2;           // row bytes
  static constexpr int BYTES = BN * RB;      // one K or V tile
  // LDS chunk swizzles (XOR on the chunk index). K rows: sigma(row) & (DCH-1),
  // so the A-fragment reads (rows sigma(lane)) hit every chunk column once per
  // 16 lanes. V rows: 4 * (row & 3), so each transposed read of 4 rows x 32
  // bytes spreads over distinct chunk columns.
  static __device__ __forceinline__ int kswz(int row) { return sigma32(row & 31) & (DCH - 1); }
  static __device__ __forceinline__ int vswz(int row) { return (4 * (row & 3)) & (DCH - 1); }
};

// Key tiles a row tile visits, in order: the sink tiles [0, ceil(min(sink,
// lo_min, hi_max + 1) / BN)), then the tiles from the one holding lo_min to the
// one holding hi_max (lo_min: the smallest first window key of the tile's
// rows; without a window lo_min = 0 and the list is tiles 0 .. hi_max / BN).
__device__ __forceinline__ void tile_list(int hi_max, int lo_min, int sink, int& n_first,
                                          int& second_t0, int& n_second) {
  int sink_end = min(min(sink, lo_min), hi_max + 1);
  if (sink_end < 0) sink_end = 0;
  n_first = (sink_end + BN - 1) / BN;
  second_t0 = max(max(lo_min, 0) / BN, n_first);
  n_second = hi_max >= 0 ? max(0, hi_max / BN - second_t0 + 1) : 0;
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most `vm` vector
// memory operations are outstanding; LDS and export counters are not waited on.
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(VM >= 0 && VM < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroups per CU: two at 32 rows per wave and head_dim <= 128; one at 64
// rows per wave (a wave's accumulators, scores and Q fragments take most of a
// SIMD's 512 registers) and at head_dim 256 (whose K/V stages take 128 KB).
constexpr int attn_occupancy(int D, int RG) { return (D > 128 || RG > 1) ? 1 : 2; }

template <typename T, int D, int MODE, int RG>
__global__ __launch_bounds__(NTHR, attn_occupancy(D, RG)) void attn_fwd_kernel(AttnArgs a) {
  using TL = Tile<D>;
  constexpr int DCH = TL::DCH;
  constexpr int RB = TL::RB;
  constexpr int BMK = bm_of(RG);
  constexpr int NDS = D / 16;                // MFMA k-steps of K.Q^T
  constexpr int NDT = D / 32;                // 32-row tiles of O^T
  constexpr int NQK = NDS * NH;              // K fragments per score tile
  constexpr int NDMA = TL::BYTES / (NTHR * 16);   // 16-byte DMA chunks per thread per K (or V) tile
  constexpr float THRESH = Rescale<T>::thresh;
  constexpr float LSUM = Rescale<T>::lsum;
  // 64 rows per wave: O lives in the reserved AGPR tiles of agpr_tiles.h
  // (tile NDT * rg + dt), accumulated, scaled and read by asm only; the score
  // MFMAs, whose results the softmax reads, stay compiler-built in VGPRs
  constexpr bool AGPR_O = RG > 1;
  static_assert(!AGPR_O || RG * NDT <= 8, "eight reserved accumulator tiles");
  using E = Elt<T>;

  // [stage][K, V][tile bytes]
  __shared__ __attribute__((aligned(1024))) char smem[NSTAGE][2][TL::BYTES];
  __shared__ int red[4][NWAVE];
  __shared__ __attribute__((aligned(16))) char dpre[MODE == MODE_FUSED ? 4 * DPRE_BLOCK : 16];
  __shared__ __attribute__((aligned(16))) char dlt[MODE == MODE_FUSED ? DLT_BYTES : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Kept as a vector value: with a readfirstlane-uniform wave index the
  // compiler's wait-count pass treats the DMA's LDS destination as aliasing
  // the fragment reads and inserts a vmcnt(0) wait right after each DMA
  // issue. The loop orders DMA and reads itself (wait + barrier per tile).
  const int wave = tid >> 6;
  const int ln = lane & 31;
  const int lg = lane >> 5;

  // ---- work item (XCD-aware: each XCD walks a contiguous range) ----
  constexpr bool KSPARSE = MODE != MODE_QSPARSE;
  const bool live = !KSPARSE && a.n_rows_dev;
  int w;
  int mt, split = 0, bh, hs = 0;
  if (live) {
    // items of the live row tiles only: (bh, split, mt < mt_live), each XCD
    // a contiguous range of them (the row tiles of one split share its
    // key/value chunk in that XCD's L2); blocks past the range exit
    const int n_live = min(max(*a.n_rows_dev, 0), a.n_rows);
    const int mt_live = (int)(((int64_t)n_live * a.G + BMK - 1) / BMK);
    const int total = a.B * a.Hkv * a.n_splits * mt_live;
    const int per = (total + 7) >> 3;
    if (mt_live == 0 || (int)(blockIdx.x >> 3) >= per) return;
    w = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (w >= total) return;
    const int t = w / mt_live;
    mt = w - t * mt_live;
    bh = (int)fdiv(t, a.fd_sp);
    split = (int)fmodq(t, bh, a.fd_sp);
    // partials keep the full grid's item index, which the merge recomputes
    w = (bh * a.n_splits + split) * a.n_mtiles + mt;
  } else {
    const int per_xcd = gridDim.x >> 3;
    w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  }
  if (w >= a.n_items) return;
  if (live) {
  } else if (KSPARSE) {
    // head split innermost: the tiles of one row block share K/V in L2
    const int t = (int)fdiv(w, a.fd_hs);
    hs = (int)fmodq(w, t, a.fd_hs);
    bh = (int)fdiv(t, a.fd_mt);
    mt = (int)fmodq(t, bh, a.fd_mt);
  } else {
    const int t = (int)fdiv(w, a.fd_mt);
    mt = (int)fmodq(w, t, a.fd_mt);
    bh = (int)fdiv(t, a.fd_sp);
    split = (int)fmodq(t, bh, a.fd_sp);
  }
  const int b = (int)fdiv(bh, a.fd_hkv);
  const int hk = (int)fmodq(bh, b, a.fd_hkv);
  const int G = a.G;
  const int GT = KSPARSE ? a.Gs : G;   // heads packed in this row tile
  const int n_kv = (KSPARSE || !a.n_kv_dev) ? a.n_kv : min(max(*a.n_kv_dev, 1), a.n_kv);
  // Fused epilogue: a tile wholly in the dense tail writes nothing. The other
  // tiles keep the row grouping of the plain launch (the per-row rescale
  // decisions make the rounded results independent of it anyway).
  if (MODE == MODE_FUSED && mt * a.tile_rows >= a.s_p) return;

  // ---- this lane's (query row, head) of row group rg: flattened pair
  //      mt * BMK + 32 * (RG * wave + rg) + ln of the tile's GT heads
  //      hk * G + hs * GT + (0 .. GT-1) ----
  bool valid[RG];
  int irow[RG], hin[RG], hrow[RG], qrow[RG], lo[RG], hi[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const int mflat = mt * BMK + (RG * wave + rg) * 32 + ln;
    valid[rg] = mflat < a.n_rows * GT;
    const int mq = (int)fdiv(mflat, a.fd_gt);
    irow[rg] = (KSPARSE ? a.row0 : 0) + (valid[rg] ? mq : 0);
    hin[rg] = valid[rg] ? (int)fmodq(mflat, mq, a.fd_gt) : 0;   // head within the tile
    hrow[rg] = hk * G + hs * GT + hin[rg];
    if (KSPARSE) {
      qrow[rg] = irow[rg];
      hi[rg] = valid[rg] ? irow[rg] : -1;
      lo[rg] = (int)fdiv(irow[rg], a.fd_qb) * a.q_block + a.q_block - a.window;
    } else {
      // row_last == NULL: every row sees all keys (a decode row at the end of
      // the cache); window > 0: the row sees sinks + its last `window` keys
      qrow[rg] = a.q_rows ? (int)min(max(a.q_rows[irow[rg]], (int64_t)0), (int64_t)(a.n_q - 1))
                          : irow[rg];
      int64_t lim = a.row_last ? a.row_last[(int64_t)b * a.rl_b + irow[rg]] : (int64_t)n_kv - 1;
      if (lim > n_kv - 1) lim = n_kv - 1;
      hi[rg] = valid[rg] ? (int)(lim < -1 ? -1 : lim) : -1;
      lo[rg] = a.window > 0 ? hi[rg] - a.window + 1 : 0;
    }
  }
  const int sink = (KSPARSE || a.window > 0) ? a.sink : 0;
  constexpr size_t esz = sizeof(T);

  // ---- Q^T fragments (registers for the whole kernel). Key-sparse modes
  //      load them first, so that their latency overlaps the set-up below;
  //      the query-sparse mode loads them once the item is known not to be
  //      past the end of its tile's list (about half of the split items at
  //      long causal row lists), still ahead of the first K/V wait ----
  u32x4 qf[RG][NDS];
  auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      const char* qp = (const char*)a.q + ((int64_t)b * a.qs_b + (int64_t)hrow[rg] * a.qs_h +
                                           (int64_t)qrow[rg] * a.qs_s) * esz;
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds)
        qf[rg][ds] = valid[rg] ? *(const u32x4*)(qp + (16 * ds + 8 * lg) * esz) : (u32x4){0, 0, 0, 0};
    }
  };
  // 64 rows per wave: the Q fragments stay in AGPRs, from which the score
  // MFMAs read their B operand directly (the VGPRs hold the two score tiles,
  // the packed probabilities and the addressing)
  auto pin_q = [&]() __attribute__((always_inline)) {
    if constexpr (RG > 1) {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) asm volatile("" : "+a"(qf[rg][ds]));
    }
  };
  if constexpr (KSPARSE) load_q();

  // ---- tile-wide bounds over the valid rows ----
  int hi_min, hi_max, lo_min, lo_max;
  if (KSPARSE) {
    // the tile holds rows r0 .. r1 (BMK / GT of them, the last tile fewer);
    // hi = row and lo grow with the row
    const int r0 = a.row0 + mt * a.tile_rows;
    const int r1 = min(r0 + a.tile_rows, a.row0 + a.n_rows) - 1;
    hi_min = r0;
    hi_max = r1;
    lo_min = (int)fdiv(r0, a.fd_qb) * a.q_block + a.q_block - a.window;
    lo_max = (int)fdiv(r1, a.fd_qb) * a.q_block + a.q_block - a.window;
  } else {
    int v_hmin = 0x7fffffff, v_hmax = -1, v_lmin = 0x7fffffff, v_lmax = (int)0x80000000;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      v_hmin = min(v_hmin, valid[rg] ? hi[rg] : 0x7fffffff);
      v_hmax = max(v_hmax, valid[rg] ? hi[rg] : -1);
      v_lmin = min(v_lmin, valid[rg] ? lo[rg] : 0x7fffffff);
      v_lmax = max(v_lmax, valid[rg] ? lo[rg] : (int)0x80000000);
    }
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
    hi_min = red[0][0], hi_max = red[1][0], lo_min = red[2][0], lo_max = red[3][0];
#pragma unroll
    for (int i = 1; i < NWAVE; ++i) {
      hi_min = min(hi_min, red[0][i]);
      hi_max = max(hi_max, red[1][i]);
      lo_min = min(lo_min, red[2][i]);
      lo_max = max(lo_max, red[3][i]);
    }
  }

  // ---- key tiles to visit: the tile list, or (query-sparse mode) this
  //      split's `chunk` tiles of it ----
  int n_first, n_second, second_t0;
  tile_list(hi_max, lo_min, sink, n_first, second_t0, n_second);
  int nt = n_first + n_second, t_off = 0;
  if (!KSPARSE) {
    const int chunk = a.n_kv_dev ? max(1, (int)fdiv(nt + a.n_splits - 1, a.fd_sp)) : a.chunk;
    t_off = split * chunk;
    if (t_off >= nt) return;   // past the list: the merge skips this split
    nt = min(chunk, nt - t_off);
    load_q();
  }

  const char* kbase = (const char*)a.k + ((int64_t)b * a.ks_b + (int64_t)hk * a.ks_h) * esz;
  const char* vbase = (const char*)a.v + ((int64_t)b * a.vs_b + (int64_t)hk * a.vs_h) * esz;
  // row strides in bytes are below 2^24 (checked on the host), so tile
  // offsets are 32 x 32 -> 64-bit products
  const uint32_t krow_b = (uint32_t)(a.ks_s * (int64_t)esz);
  const uint32_t vrow_b = (uint32_t)(a.vs_s * (int64_t)esz);
  const uint64_t kend = (uint64_t)kbase + (uint64_t)(uint32_t)n_kv * krow_b;
  const uint64_t vend = (uint64_t)vbase + (uint64_t)(uint32_t)n_kv * vrow_b;

  // ---- DMA source offsets: wave `wave`, chunk c fills LDS slots
  //      (c * NWAVE + wave) * 64 + lane of the tile; slot -> (row, swizzled chunk) ----
  uint32_t koff[NDMA], voff[NDMA];
#pragma unroll
  for (int c = 0; c < NDMA; ++c) {
    const int slot = (c * NWAVE + wave) * 64 + lane;
    const int row = slot / DCH, pc = slot % DCH;
    koff[c] = (uint32_t)row * krow_b + (uint32_t)((pc ^ TL::kswz(row)) * 16);
    voff[c] = (uint32_t)row * vrow_b + (uint32_t)((pc ^ TL::vswz(row)) * 16);
  }
  auto tile_n0 = [&](int t) __attribute__((always_inline)) -> int {
    const int u = t + t_off;
    return (u < n_first ? u : second_t0 + (u - n_first)) * BN;
  };
  // DMA of key tile t into LDS stage `slot` (K) / (V); the buffer covers the
  // rows from the tile start to the last key (n0 <= hi_max < n_kv), so the
  // hardware range check zero-fills keys past the end
  auto tile_rsrc = [&](const char* base, uint64_t end, uint32_t row_b, int t) __attribute__((always_inline)) {
    const uint64_t p = (uint64_t)base + (uint64_t)(uint32_t)tile_n0(t) * row_b;
    const uint64_t rem = end - p;
    return make_rsrc((const void*)p, (rem >> 32) ? 0xffffffffu : (uint32_t)rem);
  };
  auto issue_k = [&](int t, int slot) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kbase, kend, krow_b, t);
#pragma unroll
    for (int c = 0; c < NDMA; ++c)
      dma16(rk, (DA_LDS void*)(&smem[slot][0][(c * NWAVE + wave) * 1024]), koff[c]);
  };
  auto issue_v = [&](int t, int slot) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vbase, vend, vrow_b, t);
#pragma unroll
    for (int c = 0; c < NDMA; ++c)
      dma16(rv, (DA_LDS void*)(&smem[slot][1][(c * NWAVE + wave) * 1024]), voff[c]);
  };

  // ---- LDS read offsets ----
  // K A-fragment for k-step ds: row sigma(ln) (+32 for keys 32..63), chunk
  // (2 ds + lg) ^ kswz(row), and kswz(sigma(ln)) == ln & (DCH - 1).
  int kread[NDS];
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds)
    kread[ds] = sigma32(ln) * RB + (((2 * ds + lg) ^ (ln & (DCH - 1))) * 16);
  // V^T A-fragment via transposed reads: 16-lane group (hh, g) covers d-rows
  // 32 dt + 16 hh + (0..15) and keys 16 ks + 8 g + 4 rd + (0..3); lane j of the
  // group points at key row (j / 4), dims 4 (j % 4) .. +3.
  int vread[NDT];
  {
    const int g4 = lane >> 4, hh = g4 & 1, g = g4 >> 1, j = lane & 15;
    const int row = 8 * g + (j >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int lc = 4 * dt + 2 * hh + ((j & 3) >> 1);
      vread[dt] = row * RB + ((lc ^ TL::vswz(row)) * 16) + (j & 1) * 8;
    }
  }

  f32x16 acc[RG][NDT];
  float m_i[RG], l_i[RG];
  // First pass: a wave takes row maxima only while one of its rows has no
  // reference max yet and can still see keys.
  bool track = true;
  const float c2 = a.scale_log2;
  const DA_LDS char* lds0 = (const DA_LDS char*)&smem[0][0][0];

  // S^T = K(stage) Q^T into x (raw scores): x[rg][hf] holds keys 32 hf ..
  // 32 hf + 31 of the tile for row group rg. K fragment q (k-step q / NH of
  // half q % NH) is read once and feeds the MFMA of every row group.
  auto qk = [&](int stage, f32x16 (&x)[RG][NH]) __attribute__((always_inline)) {
    const DA_LDS char* ks = lds0 + stage * (2 * TL::BYTES);
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int hf = 0; hf < NH; ++hf)
#pragma unroll
        for (int j = 0; j < 16; ++j) x[rg][hf][j] = 0.f;
#pragma unroll
    for (int q = 0; q < NQK; ++q) {
      const int ds = q / NH, hf = q % NH;
      const u32x4 ka = *(const DA_LDS u32x4*)(ks + kread[ds] + 32 * hf * RB);
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) x[rg][hf] = E::mfma(ka, qf[rg][ds], x[rg][hf]);
    }
  };
  // mask of tile t: element j of half hf is key n0 + 32 hf + 16 (j / 8) + 8 lg + j % 8
  auto mask = [&](int t, f32x16 (&x)[RG][NH]) __attribute__((always_inline)) {
    const int n0 = tile_n0(t);
    const int n1 = n0 + BN - 1;
    const bool full = (n1 <= hi_min) && (n1 < n_kv) && (n1 < sink || n0 >= lo_max);
    if (!full) {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int hf = 0; hf < NH; ++hf)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = n0 + 32 * hf + 16 * (j >> 3) + 8 * lg + (j & 7);
            const bool vis = key <= hi[rg] && (key < sink || key >= lo[rg]);
            x[rg][hf][j] = vis ? x[rg][hf][j] : -INFINITY;
          }
    }
  };
  // scaled row max of a score tile: four independent chains, then one
  // permlane32 swap (lanes l and l + 32 hold the two key groups of a row).
  // IEEE `maximum` (v_maximum3_f32) instead of fmaxf: fmaxf must quiet
  // signalling NaNs first, one extra v_max per chain start on the MFMA
  // results; scores hold no NaN, where the two agree.
  auto rowmax = [&](const f32x16 (&x)[NH]) __attribute__((always_inline)) -> float {
    float p[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int hf = c >> 1, j0 = 8 * (c & 1);
      float m = x[hf][j0];
#pragma unroll
      for (int j = 1; j < 8; ++j) m = __builtin_elementwise_maximum(m, x[hf][j0 + j]);
      p[c] = m;
    }
    const float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(p[0], p[1]),
                                                   __builtin_elementwise_maximum(p[2], p[3]));
    float s0, s1;
    swap32(mx, s0, s1);
    return __builtin_elementwise_maximum(s0, s1) * c2;   // scaling by c2 > 0 keeps the max
  };
  // lazy online-softmax update of every row group with its scaled tile max:
  // a row's running max moves (and its O, l are rescaled) only when its tile
  // max exceeds it by more than THRESH (log2 domain). The decision is per row
  // (the other rows of the wave multiply by exactly 1), so a row's result does
  // not depend on which rows share its wave: every head packing and row
  // grouping gives the same bits.
  auto update = [&](const f32x16 (&x)[RG][NH]) __attribute__((always_inline)) {
    StaticFor<0, RG>::run([&](auto rg_c) __attribute__((always_inline)) {
      constexpr int rg = decltype(rg_c)::value;
      const float mx = rowmax(x[rg]);
      const bool up = mx > m_i[rg] + THRESH;
      // a row without a max yet has O = 0 and l = 0: it only takes the max
      const bool first = m_i[rg] == NEG_BIG;
      if (__any(up && first)) m_i[rg] = up && first ? mx : m_i[rg];
      if (__any(up && !first)) {
        const float alpha = up ? fast_exp2(m_i[rg] - mx) : 1.f;
        m_i[rg] = up ? mx : m_i[rg];
        l_i[rg] *= alpha;
        if constexpr (AGPR_O) {
          ot_pad();
          StaticFor<0, NDT>::run([&](auto dt_c) __attribute__((always_inline)) {
            ot_scale<NDT * rg + decltype(dt_c)::value>(alpha);
          });
        } else {
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[rg][dt][j] *= alpha;
        }
      }
    });
  };
  // Whether a row of this wave has no reference max yet (nothing visible in
  // the tiles so far) but can still see a key from tile t on: the list runs
  // through increasing keys, and a row sees no key above `hi`.
  auto pending = [&](int t) __attribute__((always_inline)) -> bool {
    const int n0 = tile_n0(t);
    bool p = false;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) p = p || (valid[rg] && m_i[rg] == NEG_BIG && hi[rg] >= n0);
    return __any(p);
  };

  // Step t. On entry: S(t) (masked) is in `cur` and the running max covers it;
  // K(t+1) and V(t) are resident in LDS stages (t+1) & 1 and t & 1.
  //   DMA: K(t+2) -> stage t & 1 (K(t) was read in step t-1), V(t+1) -> stage
  //        (t+1) & 1 (V(t-1) was read in step t-1).
  //   phase A: P(t) = 2^(c2 S(t) - m) packed, l += rowsum(P(t)), interleaved
  //            with the score MFMAs of S(t+1) = K(t+1) Q^T.
  //   phase B: O^T += V(t)^T P(t)^T.
  //   Both phases are one basic block, so that the exponentials stay under
  //   the score MFMAs instead of sinking to their use in phase B.
  //   Then S(t+1) is masked (boundary tiles only), its max taken (overlapping
  //   the PV MFMAs still in the pipe) and the running max moved if needed,
  //   when `track` is set; wait for the DMA, barrier.
  auto step = [&](int t, auto last_tag, auto exact_tag, f32x16 (&cur)[RG][NH],
                  f32x16 (&nxt)[RG][NH]) __attribute__((always_inline)) {
    constexpr bool LAST = decltype(last_tag)::value;   // t == nt - 1
    constexpr bool EXACT = decltype(exact_tag)::value;
    // Key-sparse modes with two waves per SIMD: the wave runs its MFMA block
    // (exponentials, score MFMAs, PV MFMAs) at raised priority and drops it
    // for the mask, row max, DMA wait and barrier, so that the other wave on
    // the SIMD fills those phases instead of competing for issue while this
    // one's MFMAs are ready (kernel (1) 0.9-1.3 % faster; the query-sparse
    // mode measured neutral to slower and keeps one priority).
    constexpr bool PRIO = KSPARSE && RG == 1;
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
    const int P = t & 1;
    if (t + 2 < nt) issue_k(t + 2, P);
    if (t + 1 < nt) issue_v(t + 1, P ^ 1);

    uint32_t pk[RG][8 * NH];
    const DA_LDS char* vs = lds0 + TL::BYTES + P * (2 * TL::BYTES);
    // V^T fragment (kk, dt): keys 16 kk .. 16 kk + 15, d-rows 32 dt .. 32 dt + 31
    auto vfrag = [&](int kk, int dt) __attribute__((always_inline)) -> u32x4 {
      const u32x2 v0 = read_tr16(vs + vread[dt] + (16 * kk) * RB);
      const u32x2 v1 = read_tr16(vs + vread[dt] + (16 * kk + 4) * RB);
      return (u32x4){v0[0], v0[1], v1[0], v1[1]};
    };
    if constexpr (RG > 1) {
      // One wave per SIMD: nothing else on the SIMD hides the softmax or the
      // latencies of its dependent chain (FMA -> exp -> pack -> dot2), so the
      // step is one static software-pipelined schedule of NSL = 64 slots, one
      // MFMA each: slots 0..31 the score MFMAs of S(t+1) (K fragment s / 2,
      // row group s % 2; none in the last step), slots 32..63 the PV MFMAs
      // (fragment f = (s - 32) / 2 = NDT kk + dt, row group s % 2). The 64
      // score elements per lane of S(t), in the order the PV MFMAs consume
      // their pairs (e = 2 p + i, pair p = 8 kk + 4 rg + jj), have their
      // exponential in slot xs(e) = 54 e / 64, the FMA one slot earlier, the
      // pack one slot after the pair's second exponential and the row-sum dot2
      // two slots after that; a pair is packed at least two slots before its
      // first PV MFMA (the asm MFMAs' 2 wait states after a VALU write). K
      // and V fragment reads run two fragments (four slots) ahead. Scheduling
      // barriers between slots keep this order.
      constexpr int NSL = 64, XS = 54;
      static_assert(NQK * RG == 32 && 2 * NH * NDT * RG == 32 && RG * NH * 16 == 64,
                    "64 MFMA slots and 64 score elements per lane");
      // element e -> (rg, hf, index within the half)
      auto erg = [](int e) constexpr { return ((e / 2) / 4) % 2; };
      auto ehf = [](int e) constexpr { return ((e / 2) / 8) / 2; };
      auto ej = [](int e) constexpr { return 2 * (4 * (((e / 2) / 8) % 2) + (e / 2) % 4) + e % 2; };
      const DA_LDS char* ks = lds0 + (P ^ 1) * (2 * TL::BYTES);
      auto kfrag = [&](int q) __attribute__((always_inline)) -> u32x4 {
        return *(const DA_LDS u32x4*)(ks + kread[q / NH] + 32 * (q % NH) * RB);
      };
      u32x4 kq[3], vq[3];
      float fv[64], xv[64];
      if (!LAST) {
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
          for (int hf = 0; hf < NH; ++hf)
#pragma unroll
            for (int jx = 0; jx < 16; ++jx) nxt[rg][hf][jx] = 0.f;
      }
      __builtin_amdgcn_sched_barrier(0);
      // first element whose exponential is in slot x (xs is monotonic)
      auto e_lo = [](int x) constexpr { return (64 * x + XS - 1) / XS; };
      StaticFor<0, NSL + 1>::run([&](auto i_c) __attribute__((always_inline)) {
        constexpr int sl = decltype(i_c)::value - 1;
        // fragment reads for the MFMAs four slots on
        if constexpr (sl >= -1 && sl <= 2 * (NQK - 1) - 4) {
          if (!LAST) {
            if constexpr (sl == -1) {
              kq[0] = kfrag(0);
              kq[1] = kfrag(1);
            } else if constexpr (sl % 2 == 0) {
              kq[((sl + 4) / 2) % 3] = kfrag((sl + 4) / 2);
            }
          }
        }
        if constexpr (sl >= 28 && sl % 2 == 0 && (sl - 28) / 2 < 2 * NH * NDT) {
          constexpr int f = (sl - 28) / 2;
          vq[f % 3] = vfrag(f / NDT, f % NDT);
        }
        // this slot's MFMA
        if constexpr (sl >= 0 && sl < 32) {
          if (!LAST) {
            constexpr int q = sl / 2, rg = sl % 2;
            nxt[rg][q % NH] = E::mfma(kq[q % 3], qf[rg][q / NH], nxt[rg][q % NH]);
          }
        } else if constexpr (sl >= 32) {
          constexpr int f = (sl - 32) / 2, rg = sl % 2, kk = f / NDT, dt = f % NDT;
          const u32x4 pf = {pk[rg][4 * kk], pk[rg][4 * kk + 1], pk[rg][4 * kk + 2],
                            pk[rg][4 * kk + 3]};
          ot_mfma<T, NDT * rg + dt>(vq[f % 3], pf);
        }
        // this slot's softmax work: FMAs of the elements exponentiated in the
        // next slot (slot -1 also those of slot 0), exponentials, packs of the
        // pairs completed in the previous slot, dot2s three slots after
        constexpr int f0 = sl == -1 ? 0 : e_lo(sl + 1), f1 = sl + 2 <= XS ? e_lo(sl + 2) : 64;
#pragma unroll
        for (int e = f0; e < f1; ++e) fv[e] = fmaf(cur[erg(e)][ehf(e)][ej(e)], c2, -m_i[erg(e)]);
        if constexpr (sl >= 0 && sl < XS) {
#pragma unroll
          for (int e = e_lo(sl); e < e_lo(sl + 1); ++e) xv[e] = fast_exp2(fv[e]);
        }
        if constexpr (sl >= 1 && sl <= XS) {
#pragma unroll
          for (int e = e_lo(sl - 1) | 1; e < e_lo(sl); e += 2)
            pk[erg(e)][8 * ehf(e) + ej(e) / 2] = E::pack2(xv[e - 1], xv[e]);
        }
        if constexpr (sl >= 3 && sl <= XS + 2) {
#pragma unroll
          for (int e = e_lo(sl - 3) | 1; e < e_lo(sl - 2); e += 2)
            l_i[erg(e)] = E::add_pair(pk[erg(e)][8 * ehf(e) + ej(e) / 2], l_i[erg(e)]);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
    } else {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const float nm = -m_i[rg];
#pragma unroll
        for (int hf = 0; hf < NH; ++hf)
#pragma unroll
          for (int jx = 0; jx < 8; ++jx)
            pk[rg][8 * hf + jx] = E::pack2(fast_exp2(fmaf(cur[rg][hf][2 * jx], c2, nm)),
                                           fast_exp2(fmaf(cur[rg][hf][2 * jx + 1], c2, nm)));
#pragma unroll
        for (int jx = 0; jx < 8 * NH; ++jx) l_i[rg] = E::add_pair(pk[rg][jx], l_i[rg]);
      }
      if (!LAST) qk(P ^ 1, nxt);
#pragma unroll
      for (int kk = 0; kk < 2 * NH; ++kk) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const u32x4 va = vfrag(kk, dt);
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            const u32x4 pf = {pk[rg][4 * kk], pk[rg][4 * kk + 1], pk[rg][4 * kk + 2],
                              pk[rg][4 * kk + 3]};
            acc[rg][dt] = E::mfma(va, pf, acc[rg][dt]);
          }
        }
      }
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    if (!LAST) {
      mask(t + 1, nxt);
      if (EXACT || track) {
        update(nxt);
        if (!EXACT) track = pending(t + 2);
      }
      // K(t+2) and V(t+1) must have landed (nothing younger is in flight)
      wait_vmcnt<0>();
      __syncthreads();
    }
  };

  // Fused epilogue: DMA the tile's dense anchor rows ([group][head][D]) into
  // dpre now, so the epilogue does not wait on global memory. Slots past the
  // tile's anchors point beyond the buffer and read as zero.
  bool pre = false;
  if constexpr (MODE == MODE_FUSED) {
    const int n_grp = a.n_grp;
    pre = n_grp * GT * D * (int)esz <= DPRE_BYTES;
    if (pre) {
      const int g0 = mt * n_grp;
      const int slot = (lane / DCH) * NWAVE + wave, ch = lane % DCH;
      const int gl = (int)fdiv(slot, a.fd_gt), hl = (int)fmodq(slot, gl, a.fd_gt);
      const int64_t span = ((int64_t)(a.n_anchor - 1) * a.dsel_a + (int64_t)(a.Hq - 1) * a.dsel_h + D) * esz;
      const char* dbase = (const char*)a.dsel + (int64_t)b * a.dsel_b * esz;
      const __amdgpu_buffer_rsrc_t rd =
          make_rsrc(dbase, span > 0xffffffffLL ? 0xffffffffu : (uint32_t)span);
      const bool ok = slot < n_grp * GT && g0 + gl < a.n_anchor;
      const int64_t off = ((int64_t)(g0 + gl) * a.dsel_a + (int64_t)(hk * G + hs * GT + hl) * a.dsel_h) * esz + ch * 16;
      if (tid < DPRE_BYTES / 16)
        dma16(rd, (DA_LDS void*)(&dpre[wave * DPRE_BLOCK]), ok && off < 0xffff0000LL ? (uint32_t)off : 0xffffffffu);
    }
  }

  // Two passes at most. Every row's reference max is its first visible tile's
  // max; it moves only by more than THRESH. The first pass takes row maxima
  // only while a row lacks its reference (in the key-sparse modes with sinks,
  // the first tile sets every row's), which keeps the max reduction off the
  // per-tile path between the PV products and the barrier. A row whose max
  // would have moved has a tile probability above 2^(THRESH - 1), hence a
  // larger partial sum; if any row of the workgroup shows one (or a
  // non-finite sum), all its tiles run again with every row max taken. Rows
  // whose max never moves go through identical operations in both passes, so
  // each row's bits are those of the exact pass whichever rows share its
  // workgroup.
  f32x16 sa[RG][NH], sb[RG][NH];
  using NotLast = std::integral_constant<bool, false>;
  using Last = std::integral_constant<bool, true>;
  auto run = [&](auto exact_tag) __attribute__((always_inline)) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    if constexpr (AGPR_O) {
      ot_pad();
      StaticFor<0, RG * NDT>::run([&](auto i_c) __attribute__((always_inline)) {
        ot_zero<decltype(i_c)::value>();
      });
    } else {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[rg][dt][j] = 0.f;
    }
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      m_i[rg] = NEG_BIG;
      l_i[rg] = 0.f;
    }
    if (nt > 0) {
      // prologue: K(0), V(0), K(1); S(0) and its running max
      issue_k(0, 0);
      issue_v(0, 0);
      if (nt > 1) issue_k(1, 1);
      wait_vmcnt<0>();
      __syncthreads();
      // (64 rows per wave) Q into AGPRs only now, so that the prologue waits
      // for the Q loads and the first DMAs at once
      pin_q();
      qk(0, sa);
      mask(0, sa);
      update(sa);
      if (!EXACT) track = pending(1);
      __syncthreads();   // every wave is done with K stage 0 before it is refilled
    }
    int t = 0;
    for (; t + 2 < nt; t += 2) {
      step(t, NotLast(), exact_tag, sa, sb);
      step(t + 1, NotLast(), exact_tag, sb, sa);
    }
    if (t + 1 < nt) {          // two tiles left
      step(t, NotLast(), exact_tag, sa, sb);
      step(t + 1, Last(), exact_tag, sb, sa);
    } else if (t < nt) {       // one tile left
      step(t, Last(), exact_tag, sa, sb);
    }
  };
  if constexpr (D > 128) {
    // one wave per SIMD: the exact pass only (the first pass's second loop
    // copy would not fit beside the head_dim-256 state without spills)
    run(std::true_type());
  } else {
    run(std::false_type());
    // the barrier inside also orders the first pass's last LDS reads before
    // the second pass refills the stages
    bool big = false;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) big = big || (valid[rg] && !(l_i[rg] <= 0.5f * LSUM));
    if (__syncthreads_or(big)) run(std::true_type());
  }

  // ---- epilogue ----
  if constexpr (AGPR_O) {
    ot_pad();
    StaticFor<0, RG>::run([&](auto rg_c) __attribute__((always_inline)) {
      StaticFor<0, NDT>::run([&](auto dt_c) __attribute__((always_inline)) {
        constexpr int rg = decltype(rg_c)::value, dt = decltype(dt_c)::value;
        acc[rg][dt] = ot_read<NDT * rg + dt>();
      });
    });
  }
  // Row stores of 16 bytes: lanes l and l + 32 hold dims 8 jq + 0..3 and
  // + 4..7 of the same row; one permlane32 swap per register pair gives lane
  // l dims 8 (2p) + 0..7 and lane l + 32 dims 8 (2p + 1) + 0..7, so each
  // store instruction writes 32 rows x 32 bytes instead of 32 rows x 16.
  auto store_rows16 = [&](char* op, u32x2 (&o)[NDT][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        u32x2& x0 = o[dt][2 * p2];
        u32x2& x1 = o[dt][2 * p2 + 1];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          auto r = __builtin_amdgcn_permlane32_swap(x0[e], x1[e], false, false);
          x0[e] = r[0];
          x1[e] = r[1];
        }
        const u32x4 v = {x0[0], x0[1], x1[0], x1[1]};
        *(u32x4*)(op + (32 * dt + 16 * p2 + 8 * lg) * esz) = v;
      }
  };
  float l_tot[RG], inv[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    l_tot[rg] = sum32(l_i[rg]);
    inv[rg] = l_tot[rg] > 0.f ? 1.f / l_tot[rg] : 0.f;
  }
  if (MODE == MODE_FUSED) {
    // out[r] = rnd(rnd(sparse[r]) + delta[r / gamma]) for rows r < s_p, with
    // delta[g] = rnd(dense[g] - rnd(sparse[g * gamma])) formed by the anchor
    // row's lanes (gamma divides the tile height, so every group of the tile
    // has its anchor in it) and shared through LDS. Rows >= s_p are not
    // written: they hold the dense tail.
    u32x2 sp[RG][NDT][4];
    bool rlive[RG];
    int ga[RG];
    DA_LDS u32x2* dl[RG];
    DA_LDS u32x2* dn_pre[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          sp[rg][dt][jq][0] = E::pack2(acc[rg][dt][4 * jq + 0] * inv[rg], acc[rg][dt][4 * jq + 1] * inv[rg]);
          sp[rg][dt][jq][1] = E::pack2(acc[rg][dt][4 * jq + 2] * inv[rg], acc[rg][dt][4 * jq + 3] * inv[rg]);
        }
      rlive[rg] = valid[rg] && irow[rg] < a.s_p;
      ga[rg] = (int)fdiv(irow[rg], a.fd_gamma);      // this row's stride group
      const int gl = ga[rg] - mt * a.n_grp;          // its group within the tile (gamma
                                                     // divides the tile's rows)
      // delta rows in LDS. With the dense rows prefetched (dpre,
      // [group][head][D]), each anchor lane writes its delta elements to the
      // padded slots of dlt, so one barrier suffices. Otherwise they go to the
      // K/V stage memory ([group][head][lg][D/2]) once every wave is done with it.
      if (pre) {
        const int ps = gl * GT + hin[rg];      // this row's dpre slot
        dn_pre[rg] = (DA_LDS u32x2*)&dpre[(ps % NWAVE) * DPRE_BLOCK + (ps / NWAVE) * RB] + lg;
        dl[rg] = (DA_LDS u32x2*)&dlt[(gl * GT + hin[rg]) * (D * (int)esz + DPAD)] + lg;
      } else {
        dn_pre[rg] = nullptr;
        dl[rg] = (DA_LDS u32x2*)&smem[0][0][0] + ((gl * GT + hin[rg]) * 2 + lg) * (NDT * 4);
      }
    }
    static_assert(DLT_BYTES >= DPRE_BYTES + (DPRE_BYTES / (2 * 32)) * DPAD, "padded slots fit");
    static_assert(BM_MAX * 2 * D <= NSTAGE * 2 * TL::BYTES, "delta slots fit the stages");
    if (pre) {
      if (nt == 0) {     // no key tile ran: make every wave's dpre DMA visible
        wait_vmcnt<0>();
        __syncthreads();
      }
    } else {
      wait_vmcnt<0>();
      __syncthreads();   // every wave is done with the K/V stages
    }
    // element (dt, jq) of this lane: dims 32 dt + 8 jq + 4 lg .. +3. One code
    // path per delta layout (PRE: the prefetched dense rows), so that the
    // anchor lanes issue all their reads, then all their writes, instead of
    // one LDS round trip per element while the other waves wait.
    auto fused_out = [&](auto pre_tag) __attribute__((always_inline)) {
      constexpr bool PRE = decltype(pre_tag)::value;
      auto dslot = [&](int rg, int dt, int jq) __attribute__((always_inline)) -> DA_LDS u32x2* {
        return PRE ? dl[rg] + 8 * dt + 2 * jq : dl[rg] + dt * 4 + jq;
      };
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        if (rlive[rg] && irow[rg] == ga[rg] * a.gamma) {
          const int64_t g = ga[rg];
          u32x2 dn[NDT][4];
          if constexpr (PRE) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
              for (int jq = 0; jq < 4; ++jq) dn[dt][jq] = dn_pre[rg][8 * dt + 2 * jq];
          } else {
            const char* dp = (const char*)a.dsel +
                             ((int64_t)b * a.dsel_b + (int64_t)hrow[rg] * a.dsel_h + g * a.dsel_a) * esz;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
              for (int jq = 0; jq < 4; ++jq)
                dn[dt][jq] = *(const u32x2*)(dp + (32 * dt + 8 * jq + 4 * lg) * esz);
          }
          u32x2 dv[NDT][4];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int jq = 0; jq < 4; ++jq)
#pragma unroll
              for (int e = 0; e < 2; ++e)
                dv[dt][jq][e] = E::pack2(E::lo(dn[dt][jq][e]) - E::lo(sp[rg][dt][jq][e]),
                                         E::hi(dn[dt][jq][e]) - E::hi(sp[rg][dt][jq][e]));
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) *dslot(rg, dt, jq) = dv[dt][jq];
          if (a.dout) {
            char* op = (char*)a.dout +
                       ((int64_t)b * a.dout_b + (int64_t)hrow[rg] * a.dout_h + g * a.dout_a) * esz;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
              for (int jq = 0; jq < 4; ++jq)
                *(u32x2*)(op + (32 * dt + 8 * jq + 4 * lg) * esz) = dv[dt][jq];
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        if (rlive[rg]) {
          char* op = (char*)a.o + ((int64_t)b * a.os_b + (int64_t)hrow[rg] * a.os_h +
                                   (int64_t)qrow[rg] * a.os_s) * esz;
          u32x2 dv[NDT][4];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) dv[dt][jq] = *dslot(rg, dt, jq);
          u32x2 o[NDT][4];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int jq = 0; jq < 4; ++jq)
#pragma unroll
              for (int e = 0; e < 2; ++e)
                o[dt][jq][e] = E::pack2(E::lo(sp[rg][dt][jq][e]) + E::lo(dv[dt][jq][e]),
                                        E::hi(sp[rg][dt][jq][e]) + E::hi(dv[dt][jq][e]));
          store_rows16(op, o);
        }
      }
    };
    if (pre) fused_out(std::true_type());
    else fused_out(std::false_type());
    return;
  }
  if (MODE == MODE_SPARSE) {
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      if (!valid[rg]) continue;
      if (a.lse && lg == 0)
        a.lse[((int64_t)b * a.Hq + hrow[rg]) * a.n_rows + irow[rg]] =
            l_tot[rg] > 0.f ? m_i[rg] + __builtin_log2f(l_tot[rg]) : INFINITY;
      char* op = (char*)a.o + ((int64_t)b * a.os_b + (int64_t)hrow[rg] * a.os_h +
                               (int64_t)qrow[rg] * a.os_s) * esz;
      u32x2 o[NDT][4];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          o[dt][jq][0] = E::pack2(acc[rg][dt][4 * jq + 0] * inv[rg], acc[rg][dt][4 * jq + 1] * inv[rg]);
          o[dt][jq][1] = E::pack2(acc[rg][dt][4 * jq + 2] * inv[rg], acc[rg][dt][4 * jq + 3] * inv[rg]);
        }
      store_rows16(op, o);
    }
  } else {
    // normalised split rows O / l in the element type, a 16-byte row piece
    // per lane after one permlane32 swap (the merge reads them back once).
    // At half the fp32 volume, plain stores through L2 measured 0.5-1 %
    // faster than non-temporal ones; with fp32 partials the non-temporal form
    // had kept the shared key/value chunk in L2 (split-kernel fetch 1.78 ->
    // 1.59 GB).
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      if (!valid[rg]) continue;   // the merge reads the rows of the selection only
      const int r = (RG * wave + rg) * 32 + ln;
      uint32_t* po = a.part_o + ((int64_t)w * a.ws_rows + r) * (D / 2);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2) {
          u32x2 x0, x1;
          const int j0 = 2 * p2, j1 = 2 * p2 + 1;
          x0[0] = E::pack2(acc[rg][dt][4 * j0 + 0] * inv[rg], acc[rg][dt][4 * j0 + 1] * inv[rg]);
          x0[1] = E::pack2(acc[rg][dt][4 * j0 + 2] * inv[rg], acc[rg][dt][4 * j0 + 3] * inv[rg]);
          x1[0] = E::pack2(acc[rg][dt][4 * j1 + 0] * inv[rg], acc[rg][dt][4 * j1 + 1] * inv[rg]);
          x1[1] = E::pack2(acc[rg][dt][4 * j1 + 2] * inv[rg], acc[rg][dt][4 * j1 + 3] * inv[rg]);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            auto sw = __builtin_amdgcn_permlane32_swap(x0[e], x1[e], false, false);
            x0[e] = sw[0];
            x1[e] = sw[1];
          }
          *(u32x4*)(po + (32 * dt + 16 * p2 + 8 * lg) / 2) = (u32x4){x0[0], x0[1], x1[0], x1[1]};
        }
      if (lg == 0) {
        a.part_ml[(int64_t)w * 2 * a.ws_rows + r] = m_i[rg];
        a.part_ml[(int64_t)w * 2 * a.ws_rows + a.ws_rows + r] = l_tot[rg];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split-KV merge + epilogue of kernel (2). `wgs` workgroups per (b, kv head,
// m tile) cover its valid rows x D/8 column chunks; each (row, chunk) task is
// shared by P = `lanes` consecutive threads that take every P-th split and
// combine (max, sum, O) by xor-shuffles, so long split lists (decode rows)
// are read with P loads in flight per task.
struct MergeArgs {
  const int64_t* q_rows;
  const int64_t* row_last;
  int64_t rl_b;
  int n_rows, G, Hkv, n_kv, n_mtiles, n_splits, chunk;
  int B;
  const int* n_kv_dev;   // as in AttnArgs
  const int* n_rows_dev; // as in AttnArgs: only the live row tiles are merged
  int window, sink;
  int lanes;        // P: threads sharing one (row, 8-column) task, splits s = p mod P
  int wgs;          // workgroups per row tile
  const uint32_t* part_o;   // element pairs of O / l per split row
  const float* part_ml;
  int ws_rows;      // as in AttnArgs
  int bm;           // as in AttnArgs: flattened rows per row tile of the split launch
  int epi, n_anchor, n_q;
  void* o;
  int64_t os_b, os_h, os_s;
  void* delta;
  int64_t ds_b, ds_h, ds_a;
  // DA_EPI_OUTPUT: optional addend [B, Hq, n, D] (strides batch, head, row):
  // out = rnd(rnd(merged) + addend), the bf16 add of a cached decode delta
  const void* add;
  int64_t as_b, as_h, as_s;
  // DA_EPI_OUTPUT: optional row log-sum-exp [B, Hq, n] (as AttnArgs::lse)
  float* lse;
};

template <typename T, int D>
__global__ __launch_bounds__(MTHR) void qsparse_merge_kernel(MergeArgs a) {
  using E = Elt<T>;
  constexpr int CPR = D / 8;   // 8-column chunks per row
  __shared__ int s_hmax[4], s_lmin[4];
  int tile = blockIdx.x / a.wgs;
  const int sub = blockIdx.x % a.wgs;
  if (a.n_rows_dev) {
    // live row tiles of every (b, kv head) first, as the split items
    const int n_live = min(max(*a.n_rows_dev, 0), a.n_rows);
    const int mt_live = (n_live * a.G + a.bm - 1) / a.bm;
    if (mt_live == 0 || tile >= a.B * a.Hkv * mt_live) return;
    tile = (tile / mt_live) * a.n_mtiles + tile % mt_live;
  }
  const int mt = tile % a.n_mtiles;
  const int bh = tile / a.n_mtiles;
  const int hk = bh % a.Hkv;
  const int b = bh / a.Hkv;
  const int tid = threadIdx.x;
  const int G = a.G;

  // Same tile list as the split kernel saw, hence the same set of written splits.
  const int n_kv = a.n_kv_dev ? min(max(*a.n_kv_dev, 1), a.n_kv) : a.n_kv;
  int my_hmax = -1, my_lmin = 0x7fffffff;
  if (tid < a.bm) {
    const int mflat = mt * a.bm + tid;
    if (mflat < a.n_rows * G) {
      int64_t lim = a.row_last ? a.row_last[(int64_t)b * a.rl_b + mflat / G] : (int64_t)n_kv - 1;
      if (lim > n_kv - 1) lim = n_kv - 1;
      my_hmax = (int)(lim < -1 ? -1 : lim);
      my_lmin = a.window > 0 ? my_hmax - a.window + 1 : 0;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    my_hmax = max(my_hmax, __shfl_xor(my_hmax, off));
    my_lmin = min(my_lmin, __shfl_xor(my_lmin, off));
  }
  if ((tid & 63) == 0) {
    s_hmax[tid >> 6] = my_hmax;
    s_lmin[tid >> 6] = my_lmin;
  }
  __syncthreads();
  const int hi_max = max(max(s_hmax[0], s_hmax[1]), max(s_hmax[2], s_hmax[3]));
  const int lo_min = min(min(s_lmin[0], s_lmin[1]), min(s_lmin[2], s_lmin[3]));
  int n_first, second_t0, n_second;
  tile_list(hi_max, lo_min, a.window > 0 ? a.sink : 0, n_first, second_t0, n_second);
  const int n_list = n_first + n_second;
  const int chunk = a.n_kv_dev ? max(1, (n_list + a.n_splits - 1) / a.n_splits) : a.chunk;
  const int nsv = (n_list + chunk - 1) / chunk;

  const size_t esz = sizeof(T);
  const int P = a.lanes;
  const int p = tid % P;
  {
    const int task = sub * (MTHR / P) + tid / P;
    const int r = task / CPR;
    const int c = task % CPR;
    const int mflat = mt * a.bm + r;
    // whole P-lane groups leave together (the shuffles stay inside a group)
    if (r >= a.bm || mflat >= a.n_rows * G) return;
    const int i = mflat / G;
    const int h = hk * G + mflat % G;

    // One pass over this lane's splits s = p, p + P, ... with an online max:
    // the (max, sum, O) state takes split s as M' = max(M, m_s), weights
    // 2^(M - M') on the state and 2^(m_s - M') l_s on the stored O_s / l_s.
    // The loads of MU splits are issued before any of them is combined, so
    // a lane has all its partial reads in flight at once.
    constexpr int MU = 4;
    float M = NEG_BIG, L = 0.f;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    auto take = [&](float m, float l, const float (&o)[8]) __attribute__((always_inline)) {
      const float mn = fmaxf(M, m);
      const float wa = fast_exp2(M - mn), wb = fast_exp2(m - mn) * l;
      L = L * wa + wb;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] * wa + o[e] * wb;
      M = mn;
    };
    for (int s0 = p; s0 < nsv; s0 += MU * P) {
      float ms[MU], ls[MU];
      u32x4 xs[MU];
#pragma unroll
      for (int u = 0; u < MU; ++u) {
        const int s = s0 + u * P;
        if (s < nsv) {
          const int64_t w = ((int64_t)bh * a.n_splits + s) * a.n_mtiles + mt;
          ms[u] = a.part_ml[w * 2 * a.ws_rows + r];
          ls[u] = a.part_ml[w * 2 * a.ws_rows + a.ws_rows + r];
          xs[u] = *(const u32x4*)(a.part_o + (w * a.ws_rows + r) * (D / 2) + 4 * c);
        } else {
          ms[u] = NEG_BIG;
          ls[u] = 0.f;
          xs[u] = (u32x4){0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int u = 0; u < MU; ++u) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[2 * e] = E::lo(xs[u][e]);
          o[2 * e + 1] = E::hi(xs[u][e]);
        }
        take(ms[u], ls[u], o);
      }
    }
    // the P lanes of the task combine their states the same way
    for (int off = 1; off < P; off <<= 1) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __shfl_xor(acc[e], off);
      const float mo = __shfl_xor(M, off), lo = __shfl_xor(L, off);
      const float mn = fmaxf(M, mo);
      const float wa = fast_exp2(M - mn), wb = fast_exp2(mo - mn);
      L = L * wa + lo * wb;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] * wa + o[e] * wb;
      M = mn;
    }
    if (p != 0) return;
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= inv;

    const int qrow = a.q_rows ? (int)min(max(a.q_rows[i], (int64_t)0), (int64_t)(a.n_q - 1)) : i;
    if (a.epi == DA_EPI_OUTPUT) {
      if (a.lse && c == 0)
        a.lse[((int64_t)b * a.Hkv * G + h) * a.n_rows + i] = L > 0.f ? M + __builtin_log2f(L) : INFINITY;
      char* op = (char*)a.o + ((int64_t)b * a.os_b + (int64_t)h * a.os_h + (int64_t)i * a.os_s + 8 * c) * esz;
      u32x4 pk = {E::pack2(acc[0], acc[1]), E::pack2(acc[2], acc[3]),
                  E::pack2(acc[4], acc[5]), E::pack2(acc[6], acc[7])};
      if (a.add) {
        const u32x4 av = *(const u32x4*)((const char*)a.add +
            ((int64_t)b * a.as_b + (int64_t)h * a.as_h + (int64_t)i * a.as_s + 8 * c) * esz);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pk[e] = E::pack2(E::lo(pk[e]) + E::lo(av[e]), E::hi(pk[e]) + E::hi(av[e]));
      }
      *(u32x4*)op = pk;
    } else {
      char* op = (char*)a.o + ((int64_t)b * a.os_b + (int64_t)h * a.os_h + (int64_t)qrow * a.os_s + 8 * c) * esz;
      const u32x4 pk = {E::pack2(acc[0], acc[1]), E::pack2(acc[2], acc[3]),
                        E::pack2(acc[4], acc[5]), E::pack2(acc[6], acc[7])};
      if (a.epi == DA_EPI_DELTA && i < a.n_anchor) {
        // delta = rnd(rnd(dense) - sparse): the reference's bf16 subtraction.
        const u32x4 sp = *(const u32x4*)op;
        u32x4 dl;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          dl[e] = E::pack2(E::lo(pk[e]) - E::lo(sp[e]), E::hi(pk[e]) - E::hi(sp[e]));
        char* dp = (char*)a.delta +
                   ((int64_t)b * a.ds_b + (int64_t)h * a.ds_h + (int64_t)i * a.ds_a + 8 * c) * esz;
        *(u32x4*)dp = dl;
      } else if (a.epi == DA_EPI_DENSE && i < a.n_anchor) {
        char* dp = (char*)a.delta +
                   ((int64_t)b * a.ds_b + (int64_t)h * a.ds_h + (int64_t)i * a.ds_a + 8 * c) * esz;
        *(u32x4*)dp = pk;
      } else {
        *(u32x4*)op = pk;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.

struct QsparsePlan {
  int n_mtiles, n_splits, chunk, n_items;
  int ws_rows;      // workspace rows per item: a tile's valid (row, head) pairs at most
  int bm;           // flattened (row, head) pairs per row tile of the split launch
  size_t ws_bytes;
};

// Rows per workgroup of a launch: for the head_dim-128 key-sparse launches
// 32 (bm 128, two workgroups per CU) or 64 query rows per wave (bm 256, one
// workgroup per CU; da_set_sparse_rows_per_wave); 64 for the selected-rows
// launches when DA_RG_ROWS is 2; 32 for the other head dims and for decode
// rows (one query row per batch).
static std::atomic<int> g_rg_sparse{DA_RG_SPARSE};
static int sparse_bm(int D) {
  return D == 128 ? bm_of(g_rg_sparse.load(std::memory_order_relaxed)) : bm_of(1);
}
static int rows_bm(int D) { return D == 128 ? bm_of(DA_RG_ROWS) : bm_of(1); }

// Merge workgroups per row tile at most: bm rows x D / 8 column chunks x 16
// lanes per task, 256 threads each.
constexpr int64_t MERGE_WGS_MAX = (int64_t)BM_MAX * (256 / 8) * 16 / MTHR;

// Split plan over the tile lists: `vis` bounds a row tile's list length, each
// item takes `chunk` consecutive tiles of it (at least `min_chunk`); `target`
// items in total.
static QsparsePlan plan_qsparse(int B, int Hq, int Hkv, int n, int64_t vis, int D, int target,
                                int min_chunk, int bm, int max_chunk = 0x7fffffff) {
  QsparsePlan p;
  const int G = Hq / Hkv;
  p.bm = bm;
  p.n_mtiles = (int)(((int64_t)n * G + bm - 1) / bm);
  const int64_t base = (int64_t)B * Hkv * p.n_mtiles;
  if (vis < 1) vis = 1;
  int64_t want = (target + base - 1) / base;
  if (want < 1) want = 1;
  if (want > vis) want = vis;
  p.chunk = (int)((vis + want - 1) / want);
  if (p.chunk > max_chunk) p.chunk = max_chunk;
  if (p.chunk < min_chunk) p.chunk = (int)min((int64_t)min_chunk, vis);
  p.n_splits = (int)((vis + p.chunk - 1) / p.chunk);
  const int64_t items = base * p.n_splits;
  // grids past 2^31 workgroups (split kernel or merge) are refused by the
  // entry points (n_items = 0)
  const bool fits = items <= 0x7fffff00LL && base * MERGE_WGS_MAX <= 0x7fffff00LL;
  p.n_items = fits ? (int)items : 0;
  p.ws_rows = (int)min((int64_t)bm, (int64_t)n * G);
  p.ws_bytes = fits ? (size_t)p.n_items * p.ws_rows * (D * sizeof(uint16_t) + 2 * sizeof(float)) : 0;
  return p;
}

// Causal selected rows: ~8192 items (about half of them past the end of a
// causal row tile's list), but at least 56 key tiles each: short items pay
// their prologue and partials, and at 32K keys (638 rows x 32 heads) 56 packs
// the ~1K useful items into two rounds of resident workgroups (0.258 ms vs
// 0.269-0.272 at 40; neutral at 128K keys, where the 8K target binds).
// A short row list (fewer than 64 (batch, kv head, row tile) triples: the
// adaptive stride's chunks, a dense tail alone) cannot fill the GPU with
// 56-tile items, and one item's latency would bound the launch: ~1024 items of
// at least 16 tiles instead.
static QsparsePlan plan_rows(int B, int Hq, int Hkv, int n, int Skv, int D) {
  const int64_t vis = (Skv + BN - 1) / BN;
  const int bm = rows_bm(D);
  const int64_t tiles = (int64_t)B * Hkv * (((int64_t)n * (Hq / Hkv) + bm - 1) / bm);
  if (tiles < 64) return plan_qsparse(B, Hq, Hkv, n, vis, D, 1024, 16, bm);
  return plan_qsparse(B, Hq, Hkv, n, vis, D, DA_ROWS_ITEMS, DA_ROWS_MIN_TILES, bm, DA_ROWS_MAX_TILES);
}

// Split plan for n rows of which about n_live hold keys (the others are -1
// rows with empty tile lists: the adaptive stride's padded row lists): the
// items per row tile follow the plan of n_live rows, the grid covers all n.
static QsparsePlan plan_rows_live(int B, int Hq, int Hkv, int n, int n_live, int Skv, int D) {
  if (n_live >= n || n_live < 1) return plan_rows(B, Hq, Hkv, n, Skv, D);
  QsparsePlan p = plan_rows(B, Hq, Hkv, n_live, Skv, D);
  const int G = Hq / Hkv;
  p.n_mtiles = (int)(((int64_t)n * G + p.bm - 1) / p.bm);
  const int64_t base = (int64_t)B * Hkv * p.n_mtiles;
  const int64_t items = base * p.n_splits;
  const bool fits = p.n_items > 0 && items <= 0x7fffff00LL && base * MERGE_WGS_MAX <= 0x7fffff00LL;
  p.n_items = fits ? (int)items : 0;
  p.ws_rows = (int)min((int64_t)p.bm, (int64_t)n * G);
  p.ws_bytes = fits ? (size_t)p.n_items * p.ws_rows * (D * sizeof(uint16_t) + 2 * sizeof(float)) : 0;
  return p;
}

// One decode row per batch at the end of the cache: its list is the sink
// tiles plus the window tiles (all tiles without a window); ~512 items.
static QsparsePlan plan_decode(int B, int Hq, int Hkv, int n_keys, int D, int window, int sink) {
  const int64_t all = (n_keys + BN - 1) / BN;
  int64_t vis = all;
  if (window > 0) vis = min(all, (int64_t)(min(sink, n_keys) + BN - 1) / BN + (window + BN - 1) / BN + 1);
  return plan_qsparse(B, Hq, Hkv, 1, vis, D, DA_DECODE_ITEMS, 1, bm_of(1));
}

template <typename T, int D, int MODE>
static void launch_attn(const AttnArgs& a, hipStream_t stream) {
  const int grid = (a.n_items + 7) / 8 * 8;
  constexpr bool has_rg2 = D == 128 && (MODE != MODE_QSPARSE || DA_RG_ROWS == 2);
  if constexpr (has_rg2) {
    if (a.bm == bm_of(2)) {
      hipLaunchKernelGGL((attn_fwd_kernel<T, D, MODE, 2>), dim3(grid), dim3(NTHR), 0, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((attn_fwd_kernel<T, D, MODE, 1>), dim3(grid), dim3(NTHR), 0, stream, a);
}

template <int MODE>
static void dispatch_attn(const AttnArgs& a, int D, int dtype, hipStream_t s) {
  if (dtype == DA_BF16) {
    if (D == 128) launch_attn<__bf16, 128, MODE>(a, s);
    else if (D == 64) launch_attn<__bf16, 64, MODE>(a, s);
    else if (D == 256) launch_attn<__bf16, 256, MODE>(a, s);
    else launch_attn<__bf16, 32, MODE>(a, s);
  } else {
    if (D == 128) launch_attn<_Float16, 128, MODE>(a, s);
    else if (D == 64) launch_attn<_Float16, 64, MODE>(a, s);
    else if (D == 256) launch_attn<_Float16, 256, MODE>(a, s);
    else launch_attn<_Float16, 32, MODE>(a, s);
  }
}

template <typename T, int D>
static void launch_merge(const MergeArgs& m, int n_tiles, hipStream_t s) {
  hipLaunchKernelGGL((qsparse_merge_kernel<T, D>), dim3(n_tiles), dim3(MTHR), 0, s, m);
}

// Query heads per key-sparse row tile: bm / 64 heads (64-row tiles) when
// they divide the GQA group, else half as many, down to one head (bm-row
// tiles). Short tiles keep the window's tile list close to the keys each row
// sees, and a stride group of up to 64 rows has its anchor in the tile.
// Sharing each K/V tile between fewer heads measured free (the tiles of one
// row block read K/V from L2 back to back).
static int tile_heads(int G, int bm) {
  int gs = bm / 64;
  while (gs > 1 && G % gs != 0) gs /= 2;
  return gs;
}

// Key/value row strides (elements) in [0, 2^23): row byte strides below 2^24.
static bool kv_rows_ok(const int64_t k_str[3], const int64_t v_str[3]) {
  return k_str[2] >= 0 && k_str[2] < (1 << 23) && v_str[2] >= 0 && v_str[2] < (1 << 23);
}

}  // namespace da

using namespace da;

// Checks and argument block shared by the two key-sparse entry points.
static int sparse_args(AttnArgs& a, const void* q, const void* k, const void* v, void* out,
                       int B, int Hq, int Hkv, int S, int D,
                       const int64_t q_str[3], const int64_t k_str[3],
                       const int64_t v_str[3], const int64_t o_str[3],
                       int window, int sink, int q_block, float sm_scale, int dtype) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (S < 0 || window < 0 || sink < 0 || q_block < 1) return DA_ERR_INVALID_ARG;
  if (!q_str || !k_str || !v_str || !o_str) return DA_ERR_INVALID_ARG;
  if (S == 0) return DA_OK;
  if (!q || !k || !v || !out) return DA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      !strides8(q_str) || !strides8(k_str) || !strides8(v_str) || !strides8(o_str))
    return DA_ERR_ALIGNMENT;
  if (!kv_rows_ok(k_str, v_str)) return DA_ERR_INVALID_ARG;
  a = AttnArgs{};
  a.q = q; a.k = k; a.v = v; a.o = out;
  a.qs_b = q_str[0]; a.qs_h = q_str[1]; a.qs_s = q_str[2];
  a.ks_b = k_str[0]; a.ks_h = k_str[1]; a.ks_s = k_str[2];
  a.vs_b = v_str[0]; a.vs_h = v_str[1]; a.vs_s = v_str[2];
  a.os_b = o_str[0]; a.os_h = o_str[1]; a.os_s = o_str[2];
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv;
  a.n_rows = S; a.n_q = S; a.n_kv = S;
  a.bm = sparse_bm(D);
  a.Gs = tile_heads(a.G, a.bm); a.n_hs = a.G / a.Gs;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.window = window; a.sink = sink; a.q_block = q_block;
  a.fd_hkv = make_fastdiv(Hkv); a.fd_qb = make_fastdiv(q_block);
  a.fd_sp = make_fastdiv(1); a.fd_gamma = make_fastdiv(1);
  return DA_OK;
}

// Work items for rows [0, n_rows) of the argument block.
static int sparse_items(AttnArgs& a) {
  a.n_mtiles = (int)(((int64_t)a.n_rows * a.Gs + a.bm - 1) / a.bm);
  const int64_t items = (int64_t)a.B * a.Hkv * a.n_hs * a.n_mtiles;
  if (items > 0x7fffff00LL) return DA_ERR_INVALID_ARG;
  a.n_items = (int)items;
  a.tile_rows = a.bm / a.Gs;
  a.fd_hs = make_fastdiv(a.n_hs); a.fd_mt = make_fastdiv(a.n_mtiles);
  a.fd_gt = make_fastdiv(a.Gs);
  return DA_OK;
}

extern "C" int da_set_sparse_rows_per_wave(int rows) {
  if (rows != 32 && rows != 64) return DA_ERR_INVALID_ARG;
  g_rg_sparse.store(rows / 32, std::memory_order_relaxed);
  return DA_OK;
}

extern "C" int da_sparse_rows_per_wave(void) { return 32 * g_rg_sparse.load(std::memory_order_relaxed); }

extern "C" int da_sparse_attn_fwd(const void* q, const void* k, const void* v, void* out,
                                  int B, int Hq, int Hkv, int S, int D,
                                  const int64_t q_str[3], const int64_t k_str[3],
                                  const int64_t v_str[3], const int64_t o_str[3],
                                  int window, int sink, int q_block, float sm_scale,
                                  int dtype, void* stream) {
  AttnArgs a;
  int rc = sparse_args(a, q, k, v, out, B, Hq, Hkv, S, D, q_str, k_str, v_str, o_str,
                       window, sink, q_block, sm_scale, dtype);
  if (rc != DA_OK || S == 0) return rc;
  if ((rc = sparse_items(a)) != DA_OK) return rc;
  (void)hipGetLastError();
  dispatch_attn<MODE_SPARSE>(a, D, dtype, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

extern "C" int da_sparse_attn_fwd_rows(const void* q, const void* k, const void* v, void* out,
                                       int B, int Hq, int Hkv, int S, int D,
                                       const int64_t q_str[3], const int64_t k_str[3],
                                       const int64_t v_str[3], const int64_t o_str[3],
                                       int window, int sink, int q_block, float sm_scale,
                                       int row0, int n_rows, int dtype, void* stream) {
  AttnArgs a;
  int rc = sparse_args(a, q, k, v, out, B, Hq, Hkv, S, D, q_str, k_str, v_str, o_str,
                       window, sink, q_block, sm_scale, dtype);
  if (rc != DA_OK) return rc;
  if (row0 < 0 || n_rows < 0 || (int64_t)row0 + n_rows > S) return DA_ERR_INVALID_ARG;
  if (S == 0 || n_rows == 0) return DA_OK;
  a.row0 = row0;
  a.n_rows = n_rows;
  if ((rc = sparse_items(a)) != DA_OK) return rc;
  (void)hipGetLastError();
  dispatch_attn<MODE_SPARSE>(a, D, dtype, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

extern "C" int da_sparse_attn_fwd_lse(const void* q, const void* k, const void* v, void* out,
                                      int B, int Hq, int Hkv, int S, int D,
                                      const int64_t q_str[3], const int64_t k_str[3],
                                      const int64_t v_str[3], const int64_t o_str[3],
                                      int window, int sink, int q_block, float sm_scale,
                                      float* lse, int dtype, void* stream) {
  AttnArgs a;
  int rc = sparse_args(a, q, k, v, out, B, Hq, Hkv, S, D, q_str, k_str, v_str, o_str,
                       window, sink, q_block, sm_scale, dtype);
  if (rc != DA_OK || S == 0) return rc;
  if (!lse) return DA_ERR_INVALID_ARG;
  if (((uintptr_t)lse & 3u) != 0) return DA_ERR_ALIGNMENT;
  a.lse = lse;
  if ((rc = sparse_items(a)) != DA_OK) return rc;
  (void)hipGetLastError();
  dispatch_attn<MODE_SPARSE>(a, D, dtype, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

extern "C" int da_fused_delta_rows(int Hq, int Hkv) {
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return 0;
  return bm_of(1);   // every launch's rows per workgroup is a multiple of it
}

extern "C" int da_sparse_attn_delta_fwd(const void* q, const void* k, const void* v, void* out,
                                        int B, int Hq, int Hkv, int S, int D,
                                        const int64_t q_str[3], const int64_t k_str[3],
                                        const int64_t v_str[3], const int64_t o_str[3],
                                        int window, int sink, int q_block, float sm_scale,
                                        const void* dense_sel, const int64_t ds_str[3],
                                        int gamma, int s_p,
                                        void* delta_out, const int64_t dl_str[3],
                                        int dtype, void* stream) {
  AttnArgs a;
  int rc = sparse_args(a, q, k, v, out, B, Hq, Hkv, S, D, q_str, k_str, v_str, o_str,
                       window, sink, q_block, sm_scale, dtype);
  if (rc != DA_OK) return rc;
  const int rows = da_fused_delta_rows(Hq, Hkv);
  if (gamma < 1 || rows == 0 || rows % gamma != 0) return DA_ERR_INVALID_ARG;
  if (s_p < 0 || s_p > S || s_p % gamma != 0) return DA_ERR_INVALID_ARG;
  if (s_p == 0) return DA_OK;
  if (!dense_sel || !ds_str) return DA_ERR_INVALID_ARG;
  if (!aligned16(dense_sel) || !strides8(ds_str)) return DA_ERR_ALIGNMENT;
  if (delta_out && (!dl_str)) return DA_ERR_INVALID_ARG;
  if (delta_out && (!aligned16(delta_out) || !strides8(dl_str))) return DA_ERR_ALIGNMENT;
  a.dsel = dense_sel; a.dsel_b = ds_str[0]; a.dsel_h = ds_str[1]; a.dsel_a = ds_str[2];
  a.dout = delta_out;
  if (delta_out) { a.dout_b = dl_str[0]; a.dout_h = dl_str[1]; a.dout_a = dl_str[2]; }
  a.gamma = gamma; a.s_p = s_p; a.n_anchor = s_p / gamma;
  a.fd_gamma = make_fastdiv(gamma);
  // every stride group needs its anchor in the row tile: a gamma that does not
  // divide the tile height takes tiles of fewer heads and more rows (the
  // per-row softmax makes the packing invisible in the results)
  while (a.Gs > 1 && (a.bm / a.Gs) % gamma != 0) a.Gs /= 2;
  a.n_hs = a.G / a.Gs;
  if (a.bm % gamma != 0) return DA_ERR_INVALID_ARG;
  if ((rc = sparse_items(a)) != DA_OK) return rc;
  a.n_grp = a.tile_rows / gamma;
  (void)hipGetLastError();
  dispatch_attn<MODE_FUSED>(a, D, dtype, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

// Split kernel + merge for a plan (arguments already validated).
static int run_qsparse(const QsparsePlan& p, const void* q, const void* k, const void* v,
                       const int64_t* q_rows, const int64_t* row_last, int64_t rl_bstride,
                       int n, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                       const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
                       void* o, const int64_t o_str[3],
                       int epi, int n_anchor, void* delta, const int64_t d_str[3],
                       int window, int sink, float sm_scale, void* workspace,
                       size_t workspace_bytes, int dtype, void* stream,
                       const int* n_kv_dev = nullptr, const void* add = nullptr,
                       const int64_t* add_str = nullptr, float* lse = nullptr,
                       const int* n_rows_dev = nullptr) {
  if (p.n_items <= 0) return DA_ERR_INVALID_ARG;
  if (!workspace || workspace_bytes < p.ws_bytes) return DA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DA_ERR_ALIGNMENT;

  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.o = nullptr;
  a.qs_b = q_str[0]; a.qs_h = q_str[1]; a.qs_s = q_str[2];
  a.ks_b = k_str[0]; a.ks_h = k_str[1]; a.ks_s = k_str[2];
  a.vs_b = v_str[0]; a.vs_h = v_str[1]; a.vs_s = v_str[2];
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.Gs = a.G; a.n_hs = 1;
  a.n_rows = n; a.n_q = Sq; a.n_kv = Skv;
  a.bm = p.bm;
  a.n_mtiles = p.n_mtiles;
  a.n_items = p.n_items;
  a.tile_rows = a.bm / a.Gs;
  a.fd_hs = make_fastdiv(1); a.fd_mt = make_fastdiv(p.n_mtiles);
  a.fd_sp = make_fastdiv(p.n_splits); a.fd_hkv = make_fastdiv(Hkv);
  a.fd_gt = make_fastdiv(a.Gs); a.fd_qb = make_fastdiv(1); a.fd_gamma = make_fastdiv(1);
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.q_rows = q_rows; a.row_last = row_last; a.rl_b = rl_bstride;
  a.chunk = p.chunk; a.n_splits = p.n_splits; a.n_kv_dev = n_kv_dev;
  a.n_rows_dev = n_rows_dev;
  a.window = window; a.sink = sink;
  a.part_o = (uint32_t*)workspace;
  a.part_ml = (float*)((char*)workspace + (size_t)p.n_items * p.ws_rows * D * sizeof(uint16_t));
  a.ws_rows = p.ws_rows;

  MergeArgs m = {};
  m.q_rows = q_rows; m.row_last = row_last; m.rl_b = rl_bstride;
  m.n_rows = n; m.n_q = Sq; m.G = a.G; m.Hkv = Hkv; m.n_kv = Skv; m.n_mtiles = p.n_mtiles;
  m.n_splits = p.n_splits; m.chunk = p.chunk; m.n_kv_dev = n_kv_dev;
  m.B = B; m.n_rows_dev = n_rows_dev;
  m.window = window; m.sink = sink;
  // P threads per (row, column chunk) task: about 4 splits each, up to 16,
  // but no more threads than about half the GPU holds (2^18): a merge with
  // that many tasks already has enough loads in flight with one lane each,
  // and more lanes only add rounds of waves (128K layer: 36 us at one lane
  // vs 62 us at four; 32K: 11 vs 20 us), while a few decode rows need the
  // lanes; workgroups per row tile cover its valid rows only
  {
    const int64_t rows = min((int64_t)p.bm, (int64_t)n * a.G);
    const int64_t tasks = (int64_t)B * Hkv * p.n_mtiles * rows * (D / 8);
    m.lanes = 1;
    while (m.lanes < 16 && m.lanes * 4 < p.n_splits) m.lanes <<= 1;
    while (m.lanes > 1 && tasks * m.lanes > (1 << 18)) m.lanes >>= 1;
    m.wgs = (int)((rows * (D / 8) * m.lanes + MTHR - 1) / MTHR);
  }
  m.part_o = a.part_o; m.part_ml = a.part_ml; m.ws_rows = p.ws_rows; m.bm = p.bm;
  m.epi = epi; m.n_anchor = (epi == DA_EPI_DELTA || epi == DA_EPI_DENSE) ? n_anchor : 0;
  m.o = o; m.os_b = o_str[0]; m.os_h = o_str[1]; m.os_s = o_str[2];
  m.delta = delta;
  if (d_str) { m.ds_b = d_str[0]; m.ds_h = d_str[1]; m.ds_a = d_str[2]; }
  m.add = add;
  if (add) { m.as_b = add_str[0]; m.as_h = add_str[1]; m.as_s = add_str[2]; }
  m.lse = lse;

  hipStream_t s = (hipStream_t)stream;
  (void)hipGetLastError();
  dispatch_attn<MODE_QSPARSE>(a, D, dtype, s);
  const int n_tiles = B * Hkv * p.n_mtiles * m.wgs;
  if (dtype == DA_BF16) {
    if (D == 128) launch_merge<__bf16, 128>(m, n_tiles, s);
    else if (D == 64) launch_merge<__bf16, 64>(m, n_tiles, s);
    else if (D == 256) launch_merge<__bf16, 256>(m, n_tiles, s);
    else launch_merge<__bf16, 32>(m, n_tiles, s);
  } else {
    if (D == 128) launch_merge<_Float16, 128>(m, n_tiles, s);
    else if (D == 64) launch_merge<_Float16, 64>(m, n_tiles, s);
    else if (D == 256) launch_merge<_Float16, 256>(m, n_tiles, s);
    else launch_merge<_Float16, 32>(m, n_tiles, s);
  }
  return hipGetLastError() == hipSuccess ? DA_OK : DA_ERR_LAUNCH;
}

extern "C" size_t da_qsparse_workspace_bytes(int B, int Hq, int Hkv, int n, int Skv, int D) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || n < 1 || Skv < 1 ||
      !head_dim_ok(D))
    return 0;
  return plan_rows(B, Hq, Hkv, n, Skv, D).ws_bytes;
}

static int qsparse_fwd(const void* q, const void* k, const void* v,
                       const int64_t* q_rows, const int64_t* row_last, int64_t rl_bstride,
                       int n, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                       const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
                       void* o, const int64_t o_str[3],
                       int epi, int n_anchor, void* delta, const int64_t d_str[3],
                       float sm_scale, void* workspace, size_t workspace_bytes,
                       int dtype, void* stream, float* lse, int n_live,
                       const int* n_rows_dev = nullptr) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (n < 0 || Sq < 0 || Skv < 0 || rl_bstride < 0 || n_live < 1) return DA_ERR_INVALID_ARG;
  if (epi != DA_EPI_OUTPUT && epi != DA_EPI_DELTA && epi != DA_EPI_SCATTER && epi != DA_EPI_DENSE)
    return DA_ERR_INVALID_ARG;
  if (!q_str || !k_str || !v_str || !o_str) return DA_ERR_INVALID_ARG;
  if (n == 0) return DA_OK;
  if (!q || !k || !v || !o || !row_last || Sq < 1 || Skv < 1) return DA_ERR_INVALID_ARG;
  if (q_rows == nullptr && n > Sq) return DA_ERR_INVALID_ARG;
  if (epi == DA_EPI_DELTA || epi == DA_EPI_DENSE) {
    if (n_anchor < 0 || n_anchor > n) return DA_ERR_INVALID_ARG;
    if (n_anchor > 0 && (!delta || !d_str)) return DA_ERR_INVALID_ARG;
    if (n_anchor > 0 && (!aligned16(delta) || !strides8(d_str))) return DA_ERR_ALIGNMENT;
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) ||
      !strides8(q_str) || !strides8(k_str) || !strides8(v_str) || !strides8(o_str))
    return DA_ERR_ALIGNMENT;
  if (!kv_rows_ok(k_str, v_str)) return DA_ERR_INVALID_ARG;
  const QsparsePlan p = plan_rows_live(B, Hq, Hkv, n, n_live, Skv, D);
  return run_qsparse(p, q, k, v, q_rows, row_last, rl_bstride, n, B, Hq, Hkv, Sq, Skv, D,
                     q_str, k_str, v_str, o, o_str, epi, n_anchor, delta, d_str, 0, 0,
                     sm_scale, workspace, workspace_bytes, dtype, stream, nullptr, nullptr,
                     nullptr, lse, n_rows_dev);
}

extern "C" int da_qsparse_attn_fwd(const void* q, const void* k, const void* v,
                                   const int64_t* q_rows, const int64_t* row_last, int64_t rl_bstride,
                                   int n, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                                   const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
                                   void* o, const int64_t o_str[3],
                                   int epi, int n_anchor, void* delta, const int64_t d_str[3],
                                   float sm_scale, void* workspace, size_t workspace_bytes,
                                   int dtype, void* stream) {
  return qsparse_fwd(q, k, v, q_rows, row_last, rl_bstride, n, B, Hq, Hkv, Sq, Skv, D, q_str,
                     k_str, v_str, o, o_str, epi, n_anchor, delta, d_str, sm_scale, workspace,
                     workspace_bytes, dtype, stream, nullptr, 0x7fffffff);
}

extern "C" size_t da_qsparse_workspace_bytes_live(int B, int Hq, int Hkv, int n, int n_live, int Skv,
                                                  int D) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || n < 1 || n_live < 1 || Skv < 1 ||
      !head_dim_ok(D))
    return 0;
  return plan_rows_live(B, Hq, Hkv, n, n_live, Skv, D).ws_bytes;
}

extern "C" int da_qsparse_attn_fwd_live(const void* q, const void* k, const void* v,
                                        const int64_t* q_rows, const int64_t* row_last,
                                        int64_t rl_bstride, int n, int n_live,
                                        const int* n_dev, int B, int Hq,
                                        int Hkv, int Sq, int Skv, int D, const int64_t q_str[3],
                                        const int64_t k_str[3], const int64_t v_str[3],
                                        void* o, const int64_t o_str[3], float sm_scale,
                                        void* workspace, size_t workspace_bytes, int dtype,
                                        void* stream) {
  return qsparse_fwd(q, k, v, q_rows, row_last, rl_bstride, n, B, Hq, Hkv, Sq, Skv, D, q_str,
                     k_str, v_str, o, o_str, DA_EPI_OUTPUT, 0, nullptr, nullptr, sm_scale,
                     workspace, workspace_bytes, dtype, stream, nullptr, n_live, n_dev);
}

extern "C" int da_qsparse_attn_fwd_lse(const void* q, const void* k, const void* v,
                                       const int64_t* q_rows, const int64_t* row_last,
                                       int64_t rl_bstride, int n, int B, int Hq, int Hkv,
                                       int Sq, int Skv, int D, const int64_t q_str[3],
                                       const int64_t k_str[3], const int64_t v_str[3],
                                       void* o, const int64_t o_str[3], float* lse,
                                       float sm_scale, void* workspace, size_t workspace_bytes,
                                       int dtype, void* stream) {
  if (n > 0 && !lse) return DA_ERR_INVALID_ARG;
  if (((uintptr_t)lse & 3u) != 0) return DA_ERR_ALIGNMENT;
  return qsparse_fwd(q, k, v, q_rows, row_last, rl_bstride, n, B, Hq, Hkv, Sq, Skv, D, q_str,
                     k_str, v_str, o, o_str, DA_EPI_OUTPUT, 0, nullptr, nullptr, sm_scale,
                     workspace, workspace_bytes, dtype, stream, lse, 0x7fffffff);
}

extern "C" size_t da_decode_workspace_bytes(int B, int Hq, int Hkv, int n_keys, int D, int window,
                                            int sink) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || n_keys < 1 || !head_dim_ok(D) ||
      window < 0 || sink < 0)
    return 0;
  return plan_decode(B, Hq, Hkv, n_keys, D, window, sink).ws_bytes;
}

extern "C" int da_decode_attn_fwd(const void* q, const void* k, const void* v, void* out,
                                  int B, int Hq, int Hkv, int n_keys, int D,
                                  const int64_t q_str[3], const int64_t k_str[3],
                                  const int64_t v_str[3], const int64_t o_str[3],
                                  int window, int sink, float sm_scale,
                                  void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (n_keys < 0 || window < 0 || sink < 0) return DA_ERR_INVALID_ARG;
  if (!q_str || !k_str || !v_str || !o_str) return DA_ERR_INVALID_ARG;
  if (!q || !k || !v || !out) return DA_ERR_INVALID_ARG;
  if (n_keys == 0) return DA_ERR_INVALID_ARG;   // a decode row has at least its own key
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      !strides8(q_str) || !strides8(k_str) || !strides8(v_str) || !strides8(o_str))
    return DA_ERR_ALIGNMENT;
  if (!kv_rows_ok(k_str, v_str)) return DA_ERR_INVALID_ARG;
  const QsparsePlan p = plan_decode(B, Hq, Hkv, n_keys, D, window, sink);
  if (!workspace || workspace_bytes < p.ws_bytes) return DA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DA_ERR_ALIGNMENT;
  return run_qsparse(p, q, k, v, nullptr, nullptr, 0, 1, B, Hq, Hkv, 1, n_keys, D,
                     q_str, k_str, v_str, out, o_str, DA_EPI_OUTPUT, 0, nullptr, nullptr,
                     window, sink, sm_scale, workspace, workspace_bytes, dtype, stream);
}

extern "C" int da_decode_attn_fwd_dev(const void* q, const void* k, const void* v, void* out,
                                      int B, int Hq, int Hkv, const int32_t* n_keys_dev,
                                      int max_keys, int D,
                                      const int64_t q_str[3], const int64_t k_str[3],
                                      const int64_t v_str[3], const int64_t o_str[3],
                                      int window, int sink, float sm_scale,
                                      const void* addend, const int64_t add_str[3],
                                      void* workspace, size_t workspace_bytes, int dtype,
                                      void* stream) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (max_keys < 1 || window < 0 || sink < 0) return DA_ERR_INVALID_ARG;
  if (addend && (!add_str || !aligned16(addend) || !strides8(add_str))) return DA_ERR_ALIGNMENT;
  if (!q_str || !k_str || !v_str || !o_str) return DA_ERR_INVALID_ARG;
  if (!q || !k || !v || !out || !n_keys_dev) return DA_ERR_INVALID_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      ((uintptr_t)n_keys_dev & 3) != 0 ||
      !strides8(q_str) || !strides8(k_str) || !strides8(v_str) || !strides8(o_str))
    return DA_ERR_ALIGNMENT;
  if (!kv_rows_ok(k_str, v_str)) return DA_ERR_INVALID_ARG;
  // launch shape and workspace of the longest cache: the key count is read
  // on the device when the kernels run
  const QsparsePlan p = plan_decode(B, Hq, Hkv, max_keys, D, window, sink);
  if (!workspace || workspace_bytes < p.ws_bytes) return DA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DA_ERR_ALIGNMENT;
  return run_qsparse(p, q, k, v, nullptr, nullptr, 0, 1, B, Hq, Hkv, 1, max_keys, D,
                     q_str, k_str, v_str, out, o_str, DA_EPI_OUTPUT, 0, nullptr, nullptr,
                     window, sink, sm_scale, workspace, workspace_bytes, dtype, stream,
                     n_keys_dev, addend, add_str);
}

// ---------------------------------------------------------------------------
// Decode row without a caller workspace (da_decode_attn_fwd_dev_noalloc): the
// split-KV partials live in `scratch`, a file-scope device array of
// DA_DECODE_SCRATCH_BYTES of which each GPU holds its own copy until the
// process ends. Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address): the address comes from
// hipGetSymbolAddress, once per device with that device current, and is kept
// per device. Nothing in the scratch needs to start at zero (the merge reads
// only the partials the split kernel of the same call wrote); calls that
// overlap on one GPU share the array and race.
static __device__ __align__(256) char scratch[DA_DECODE_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];
}  // namespace

// This device's address of `scratch` (looked up on the first call on it).
static int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return DA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return DA_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DA_OK;
}

extern "C" size_t da_decode_scratch_bytes(void) { return DA_DECODE_SCRATCH_BYTES; }

extern "C" int da_decode_attn_fwd_dev_noalloc(const void* q, const void* k, const void* v,
                                              void* out, int B, int Hq, int Hkv,
                                              const int32_t* n_keys_dev, int max_keys, int D,
                                              const int64_t q_str[3], const int64_t k_str[3],
                                              const int64_t v_str[3], const int64_t o_str[3],
                                              int window, int sink, float sm_scale,
                                              const void* addend, const int64_t add_str[3],
                                              int dtype, void* stream) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (max_keys < 1 || window < 0 || sink < 0) return DA_ERR_INVALID_ARG;
  const size_t need = plan_decode(B, Hq, Hkv, max_keys, D, window, sink).ws_bytes;
  if (need == 0 || need > DA_DECODE_SCRATCH_BYTES) return DA_ERR_SCRATCH;
  void* ws = nullptr;
  if ((rc = scratch_address(&ws)) != DA_OK) return rc;
  return da_decode_attn_fwd_dev(q, k, v, out, B, Hq, Hkv, n_keys_dev, max_keys, D, q_str, k_str,
                                v_str, o_str, window, sink, sm_scale, addend, add_str, ws,
                                DA_DECODE_SCRATCH_BYTES, dtype, stream);
}

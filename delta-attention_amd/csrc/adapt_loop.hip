// The adaptive-stride layer (llama.py:759-824) as one host call.
//
// delta_adaptive_forward's chunk loop, enqueued from C++: a Python loop
// issues one chunk's launches in about 190 us, longer than the GPU takes to
// run them, so the GPU waited for the host between chunks. Here the host
// enqueues the whole layer in a few hundred microseconds and reads nothing
// back; the per-chunk logs hold what the caller needs afterwards.
//
// Chunks are the [start, end) ranges of adapt_chunk rows of the s_p prefix
// rows (stride.py:111-112); chunk c's anchors are start + j * gamma_c.
// Each chunk's stride depends on the previous chunk's dense rows, so
// computing them chunk by chunk makes a chain of small kernel (2) launches
// (at 128K, 32 launches that together take half again as long as one launch
// over the same rows). When gamma0 divides adapt_chunk, the dense rows at
// every multiple of gamma0 below s_p are computed ahead in one launch; a
// chunk whose stride is a multiple of gamma0 (the starting stride and every
// doubling of it) takes its anchors' rows from there, any other chunk
// recomputes its anchors. Per chunk c:
//   kernel (2) over the chunk's anchors when it recomputes them (a launch
//     over a device-held row count that is zero otherwise), into one of two
//     row buffers;
//   on `stream`, once the chunk's key-sparse rows are in out: its delta
//     cosines, their log, the next stride and anchor rows (the
//     da_adapt_chunk_step kernels), then its broadcast-add in place: rows
//     [start, end) of out += rnd(dense - out[anchor]) per stride group.
// With a second stream, that stream takes the key-sparse pass over each
// chunk's rows (kernel (1) over a row range) followed by the chunk's
// recompute launch, then an event for `stream`; at the end it takes the dense
// tail rows [s_p, S) scattered into out, and `stream` waits for it. The
// recompute launch waits behind the key-sparse launch there, where its
// workgroups (nearly always all of them empty) start in that launch's tail,
// and not on `stream`, where they would wait for slots that the concurrent
// key-sparse workgroups hold. Without a second stream, rows [0, s_p) of out
// hold the key-sparse pass already and everything runs on `stream`.
#include "device_common.h"
#include "capi_common.h"
#include "adapt_args.h"

#include <algorithm>

namespace da {

int delta_add_chunk(void* out, const int64_t o_str[3], const void* dense,
                    const int64_t ds_str[3], const int* sel, const void* alt,
                    const int64_t alt_str[3], const int64_t* anchors, const int* n_dev,
                    int max_n, int row_end, int s_p, int B, int H, int D, int n_grid, int dtype,
                    hipStream_t s);

namespace {

constexpr int NEV = 4;      // events per ring; a ring slot is reused NEV chunks later

// Rows per key-sparse launch on the second stream, in whole chunks of at least
// this many rows (1: one chunk per launch). Fewer, longer launches have fewer
// partly idle tail rounds but hold back each chunk's decision until the whole
// launch ends; at 128K tokens with 4096-row chunks the layer took 7.40 / 7.65 /
// 7.75 / 7.87 ms at 4096 / 8192 / 16384 / 32768 rows per launch.
#ifndef DA_ADAPT_SPARSE_ROWS
#define DA_ADAPT_SPARSE_ROWS 1
#endif

// Sizes of one layer's chunk loop, shared by the workspace query and the call.
struct AdaptPlan {
  int nc = 0;          // chunks
  int max_n = 0;       // anchor slots per chunk: the finest stride a chunk can get
  int n_live = 0;      // anchors the recompute plans are sized for (a chunk at the first stride)
  int cut_n = 0;       // dense tail rows
  int n_ahead = 0;     // rows computed ahead (multiples of gamma0 below s_p), 0: none
  size_t off_rows, off_tail, off_ahead_rows, off_state, off_sel, off_cos, off_dense,
      off_ahead, off_ws, off_ws_ahead, off_ws_tail;
  size_t dense_bytes = 0, ws_bytes = 0, ws_ahead_bytes = 0, ws_tail_bytes = 0, bytes = 0;
};

inline size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

// bytes 0: the sizes do not form a launch.
AdaptPlan plan_adapt(int B, int Hq, int Hkv, int S, int D, int s_p, int adapt_chunk, int gamma0,
                     int gamma_min) {
  AdaptPlan p;
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || S < 1 || s_p < 0 || s_p >= S ||
      adapt_chunk < 1 || gamma0 < 1 || gamma_min < 1)
    return p;
  p.nc = (int)(((int64_t)s_p + adapt_chunk - 1) / adapt_chunk);
  p.cut_n = S - s_p;
  const int g_low = std::min(gamma0, gamma_min);
  const int longest = std::min(adapt_chunk, s_p);
  p.max_n = p.nc > 0 ? (longest + g_low - 1) / g_low : 1;
  p.n_live = std::min(p.max_n, std::max(1, (adapt_chunk + gamma0 - 1) / gamma0));
  if (p.nc > 0 && adapt_chunk % gamma0 == 0) p.n_ahead = (s_p + gamma0 - 1) / gamma0;
  const size_t esz = 2;
  size_t o = 0;
  p.off_rows = o;  o = up256(o + (size_t)std::max(p.nc, 1) * p.max_n * 8);
  p.off_tail = o;  o = up256(o + (size_t)p.cut_n * 8);
  p.off_ahead_rows = o; o = up256(o + (size_t)p.n_ahead * 8);
  p.off_state = o; o = up256(o + 5 * sizeof(int));
  p.off_sel = o;   o = up256(o + (size_t)2 * std::max(p.nc, 1) * sizeof(int));
  p.off_cos = o;   o = up256(o + (size_t)B * std::max(p.max_n - 1, 1) * Hq * sizeof(float));
  p.dense_bytes = up256((size_t)B * Hq * p.max_n * D * esz);
  p.off_dense = o; o += 2 * p.dense_bytes;
  p.off_ahead = o; o = up256(o + (size_t)B * Hq * p.n_ahead * D * esz);
  for (int c = 0; c < p.nc; ++c) {
    const int end = (int)std::min<int64_t>((int64_t)(c + 1) * adapt_chunk, s_p);
    const size_t w = da_qsparse_workspace_bytes_live(B, Hq, Hkv, p.max_n, p.n_live, end, D);
    if (w == 0) return p;
    p.ws_bytes = std::max(p.ws_bytes, w);
  }
  p.off_ws = o;    o = up256(o + p.ws_bytes);
  if (p.n_ahead > 0) {
    p.ws_ahead_bytes = da_qsparse_workspace_bytes(B, Hq, Hkv, p.n_ahead, s_p, D);
    if (p.ws_ahead_bytes == 0) return p;
  }
  p.off_ws_ahead = o; o = up256(o + p.ws_ahead_bytes);
  p.ws_tail_bytes = da_qsparse_workspace_bytes(B, Hq, Hkv, p.cut_n, S, D);
  if (p.ws_tail_bytes == 0) return p;
  p.off_ws_tail = o; o = up256(o + p.ws_tail_bytes);
  p.bytes = o;
  return p;
}

// The first chunk's anchor rows and state, the tail rows and the rows
// computed ahead.
__global__ __launch_bounds__(256) void adapt_init_kernel(int64_t* rows0, int max_n, int n0,
                                                         int gamma0, int64_t* tail, int s_p,
                                                         int cut_n, int64_t* ahead, int n_ahead,
                                                         int* state) {
  for (int j = threadIdx.x; j < max_n; j += 256)
    rows0[j] = j < n0 ? (int64_t)j * gamma0 : (int64_t)-1;
  for (int j = threadIdx.x; j < cut_n; j += 256) tail[j] = (int64_t)s_p + j;
  for (int j = threadIdx.x; j < n_ahead; j += 256) ahead[j] = (int64_t)j * gamma0;
  if (threadIdx.x == 0) {
    // {stride, anchors, anchors to recompute, first slot ahead (-1: none), slot step}
    state[0] = gamma0;
    state[1] = n0;
    state[2] = n_ahead > 0 ? 0 : n0;
    state[3] = n_ahead > 0 ? 0 : -1;
    state[4] = 1;
  }
}

}  // namespace
}  // namespace da

using namespace da;

extern "C" size_t da_adapt_layer_workspace_bytes(int B, int Hq, int Hkv, int S, int D, int s_p,
                                                 int adapt_chunk, int gamma0, int gamma_min) {
  if (!head_dim_ok(D)) return 0;
  return plan_adapt(B, Hq, Hkv, S, D, s_p, adapt_chunk, gamma0, gamma_min).bytes;
}

extern "C" int da_adapt_layer_fwd(const void* q, const void* k, const void* v, void* out,
                                  int B, int Hq, int Hkv, int S, int D,
                                  const int64_t q_str[3], const int64_t k_str[3],
                                  const int64_t v_str[3], const int64_t o_str[3],
                                  int window, int sink, int q_block, float sm_scale,
                                  int s_p, int adapt_chunk, int gamma0, int gamma_min,
                                  int gamma_max, int trigger, double threshold, double margin,
                                  double k_sd, double* log_mean, float* log_min, int* log_gamma,
                                  int* log_n, int n_log, void* workspace, size_t ws_bytes,
                                  int dtype, void* stream, void* side_stream) {
  int rc;
  if ((rc = check_common(B, Hq, Hkv, D, dtype)) != DA_OK) return rc;
  if (!q || !k || !v || !out || !q_str || !k_str || !v_str || !o_str) return DA_ERR_INVALID_ARG;
  if (gamma_max < gamma_min || (trigger != 0 && trigger != 1)) return DA_ERR_INVALID_ARG;
  const AdaptPlan p = plan_adapt(B, Hq, Hkv, S, D, s_p, adapt_chunk, gamma0, gamma_min);
  if (p.bytes == 0) return DA_ERR_INVALID_ARG;
  if (!workspace || ws_bytes < p.bytes) return DA_ERR_INVALID_ARG;
  if (((uintptr_t)workspace & 255u) != 0) return DA_ERR_ALIGNMENT;
  if (p.nc > 0 && (!log_mean || !log_min || !log_gamma || !log_n || n_log < p.nc))
    return DA_ERR_INVALID_ARG;
  if (!aligned16(out) || !strides8(o_str)) return DA_ERR_ALIGNMENT;

  char* ws = (char*)workspace;
  int64_t* rows_all = (int64_t*)(ws + p.off_rows);
  int64_t* tail = (int64_t*)(ws + p.off_tail);
  int64_t* ahead_rows = (int64_t*)(ws + p.off_ahead_rows);
  int* state = (int*)(ws + p.off_state);
  int* sel_log = (int*)(ws + p.off_sel);
  float* cos_work = (float*)(ws + p.off_cos);
  // a recomputed chunk's rows [B, Hq, max_n, D], chunk c in buffer c % 2
  auto dense_of = [&](int c) { return (void*)(ws + p.off_dense + (size_t)(c % 2) * p.dense_bytes); };
  void* ahead = ws + p.off_ahead;          // the rows ahead [B, Hq, n_ahead, D]
  void* ws_split = ws + p.off_ws;
  void* ws_ahead = ws + p.off_ws_ahead;
  void* ws_tail = ws + p.off_ws_tail;
  const int max_n = p.max_n;
  const bool use_ahead = p.n_ahead > 0;
  // strides (batch, head, row) for kernel (2) and the broadcast, (batch, row,
  // head) for the cosines
  const int64_t dn_bhr[3] = {(int64_t)Hq * max_n * D, (int64_t)max_n * D, D};
  const int64_t dn_brh[3] = {dn_bhr[0], dn_bhr[2], dn_bhr[1]};
  const int64_t ah_bhr[3] = {(int64_t)Hq * p.n_ahead * D, (int64_t)p.n_ahead * D, D};
  const int64_t ah_brh[3] = {ah_bhr[0], ah_bhr[2], ah_bhr[1]};
  const int64_t out_brh[3] = {o_str[0], o_str[2], o_str[1]};

  hipStream_t st = (hipStream_t)stream;
  hipStream_t side = (hipStream_t)side_stream;
  // events, rings indexed by chunk: ev_rows = the chunk's key-sparse rows and
  // recomputed anchors are ready (second stream -> stream), ev_next = the
  // chunk's decision is made, so the next chunk's row list and count are
  // final (stream -> second stream)
  hipEvent_t ev[2 * NEV + 1] = {};
  hipEvent_t *ev_rows = ev, *ev_next = ev + NEV, &ev_join = ev[2 * NEV];
  int n_ev = 0;
  if (side) {
    for (; n_ev < 2 * NEV + 1; ++n_ev)
      if (hipEventCreateWithFlags(&ev[n_ev], hipEventDisableTiming) != hipSuccess) break;
    if (n_ev < 2 * NEV + 1) {
      for (int i = 0; i < n_ev; ++i) (void)hipEventDestroy(ev[i]);
      return DA_ERR_LAUNCH;
    }
  }
  auto ok = [](hipError_t e) { return e == hipSuccess; };
  rc = DA_OK;
  const int n0 = p.nc > 0 ? std::min((std::min(adapt_chunk, s_p) + gamma0 - 1) / gamma0, max_n) : 0;
  (void)hipGetLastError();
  hipLaunchKernelGGL(adapt_init_kernel, dim3(1), dim3(256), 0, st, rows_all, max_n, n0, gamma0,
                     tail, s_p, p.cut_n, ahead_rows, p.n_ahead, state);
  if (hipGetLastError() != hipSuccess) rc = DA_ERR_LAUNCH;
  // the second stream starts once the inputs and the first chunk's state are ready
  if (rc == DA_OK && side &&
      !(ok(hipEventRecord(ev_join, st)) && ok(hipStreamWaitEvent(side, ev_join, 0))))
    rc = DA_ERR_LAUNCH;
  if (rc == DA_OK && use_ahead)
    rc = da_qsparse_attn_fwd(q, k, v, ahead_rows, ahead_rows, 0, p.n_ahead, B, Hq, Hkv, S, s_p, D,
                             q_str, k_str, v_str, ahead, ah_bhr, DA_EPI_OUTPUT, 0, nullptr,
                             nullptr, sm_scale, ws_ahead, p.ws_ahead_bytes, dtype, st);

  CosArgs cs = {};
  cs.s = out; cs.s_b = out_brh[0]; cs.s_r = out_brh[1]; cs.s_h = out_brh[2];
  cs.n_rows = S; cs.cos = cos_work; cs.B = B; cs.n = max_n; cs.H = Hq; cs.D = D;
  cs.n_dev = state + 1;
  if (use_ahead) {
    cs.a = ahead; cs.a_b = ah_brh[0]; cs.a_n = ah_brh[1]; cs.a_h = ah_brh[2];
    cs.sel = state + 3;
    cs.alt_b = dn_brh[0]; cs.alt_n = dn_brh[1]; cs.alt_h = dn_brh[2];
  } else {
    cs.a_b = dn_brh[0]; cs.a_n = dn_brh[1]; cs.a_h = dn_brh[2];
  }
  AdaptArgs ad = {};
  ad.cos = cos_work; ad.B = B; ad.H = Hq; ad.state = state; ad.max_n = max_n;
  ad.trigger = trigger; ad.threshold = threshold; ad.margin = margin; ad.k = k_sd;
  ad.gamma_min = gamma_min; ad.gamma_max = gamma_max;
  ad.log_mean = log_mean; ad.log_min = log_min; ad.log_gamma = log_gamma; ad.log_n = log_n;
  ad.full_state = true;
  ad.spec_gamma = use_ahead ? gamma0 : 0;
  ad.sel_log = use_ahead ? sel_log : nullptr;

  // chunk c's recompute launch and its decision chain (the key-sparse rows
  // running further ahead of it on the second stream measured slower: 4 and
  // 8 chunks ahead, +1 % and +2 % at 128K)
  auto chain = [&](int c) -> int {
    int r;
    const int end = (int)std::min<int64_t>((int64_t)(c + 1) * adapt_chunk, s_p);
    const int next_end = (int)std::min<int64_t>((int64_t)end + adapt_chunk, s_p);
    int64_t* rows_c = rows_all + (size_t)c * max_n;
    void* dense = dense_of(c);
    hipStream_t rs = side ? side : st;   // the stream of the recompute launch
    // the chunk's rows and count come from the previous chunk's decision;
    // it also ends the broadcast that read this row buffer two chunks ago
    if (side && c >= 1 && !ok(hipStreamWaitEvent(side, ev_next[(c - 1) % NEV], 0)))
      return DA_ERR_LAUNCH;
    // the chunk's anchors that are not among the rows ahead (state[2] of them)
    r = da_qsparse_attn_fwd_live(q, k, v, rows_c, rows_c, 0, max_n, p.n_live, state + 2, B, Hq,
                                 Hkv, S, end, D, q_str, k_str, v_str, dense, dn_bhr, sm_scale,
                                 ws_split, p.ws_bytes, dtype, rs);
    if (r != DA_OK) return r;
    if (side && !(ok(hipEventRecord(ev_rows[c % NEV], side)) &&
                  ok(hipStreamWaitEvent(st, ev_rows[c % NEV], 0))))
      return DA_ERR_LAUNCH;
    cs.rows = rows_c;
    if (use_ahead) cs.a_alt = dense;
    else cs.a = dense;
    ad.chunk = c; ad.next_start = end; ad.next_end = next_end;
    ad.rows_next = next_end > end ? rows_c + max_n : nullptr;
    // the grids of the cosines and the broadcast are sized for a chunk at the
    // first stride and loop over more anchors (fewer empty workgroups; the
    // launches' time beside the key-sparse launches did not change)
    if ((r = adapt_step_launch(cs, ad, p.n_live, dtype, st)) != DA_OK) return r;
    if (side && !ok(hipEventRecord(ev_next[c % NEV], st))) return DA_ERR_LAUNCH;
    return use_ahead
        ? delta_add_chunk(out, o_str, ahead, ah_bhr, sel_log + 2 * c, dense, dn_bhr, rows_c,
                          log_n + c, max_n, end, s_p, B, Hq, D, p.n_live, dtype, st)
        : delta_add_chunk(out, o_str, dense, dn_bhr, nullptr, nullptr, nullptr, rows_c,
                          log_n + c, max_n, end, s_p, B, Hq, D, p.n_live, dtype, st);
  };
  const int per_launch =
      (int)std::max<int64_t>(1, ((int64_t)DA_ADAPT_SPARSE_ROWS + adapt_chunk - 1) / adapt_chunk);
  for (int c = 0; c < p.nc && rc == DA_OK; ++c) {
    if (side && c % per_launch == 0) {
      const int start = c * adapt_chunk;
      const int end = (int)std::min<int64_t>((int64_t)start + (int64_t)per_launch * adapt_chunk,
                                             s_p);
      rc = da_sparse_attn_fwd_rows(q, k, v, out, B, Hq, Hkv, S, D, q_str, k_str, v_str, o_str,
                                   window, sink, q_block, sm_scale, start, end - start, dtype,
                                   side);
      if (rc != DA_OK) break;
    }
    rc = chain(c);
  }
  if (rc == DA_OK)
    rc = da_qsparse_attn_fwd(q, k, v, tail, tail, 0, p.cut_n, B, Hq, Hkv, S, S, D, q_str, k_str,
                             v_str, out, o_str, DA_EPI_SCATTER, 0, nullptr, nullptr, sm_scale,
                             ws_tail, p.ws_tail_bytes, dtype, side ? side : st);
  if (side) {
    // whatever happened above, `stream` ends behind everything the second
    // stream was given
    if (!(ok(hipEventRecord(ev_join, side)) && ok(hipStreamWaitEvent(st, ev_join, 0))) &&
        rc == DA_OK)
      rc = DA_ERR_LAUNCH;
    for (int i = 0; i < n_ev; ++i) (void)hipEventDestroy(ev[i]);
  }
  return rc;
}

// Device-side step metadata: the launch tables of one diffusion step built on
// the GPU from a device-resident table of per-sequence state, and the state
// machine advanced on the GPU, so that a whole denoising step (tables,
// forward, sampler, advance) can be replayed from a captured HIP graph with
// no host work.
//
// step_build_kernel restates, for every sequence of the batch:
//   * the per-sequence mode of _mixed_sparse_dense_attention
//     (dllmserve/layers/attention.py:168-265): no SparseConfig or cache
//     state 0 -> full attention over all N rows; state 1 -> full attention
//     plus selection of n_keep = min(max(1, int(Kc * ratio)), Kc) of the
//     Kc = N - bl non-block rows; state 2 -> the bl block rows against the
//     n_keep cached rows;
//   * the rows the runner feeds and their positions (model_runner.py:240-256);
//   * the slot lists (model_runner.py:257-273,287-302: slot r of a sequence
//     is page_table[r / 256] * 256 + r % 256, r < n_keep);
//   * the sampler's windows (model_runner.py:791-818,911-920).
// The table layout is the one the attention and sampler kernels take
// (cu_seqlens, segment-id lists, slot offsets, selection jobs, unmask
// parameters).  One workgroup of 1024 threads: one sequence per thread for
// the per-sequence values and the prefix sums, then all threads fill the
// per-row and per-slot arrays.
#include "common.h"

namespace dllm {

constexpr int kStepMaxSeq = 1024;
// P, N, sparse, block_len, block_idx, step_in_block, cache_state, delay, steps, cur, head_select, pool_k
constexpr int kStateCols = 12;
constexpr int kJobCols = 8;  // row0, n_tok, blk_start, blk_len, n_keep, slot_off, head_select, pool_k

struct StepBuildArgs {
  const int32_t* state;
  const double* ratio;
  const int32_t* pages;
  const int32_t* page_off;
  int n;
  int64_t tok_stride;
  int32_t* cu;          // [n+1]
  int32_t* dense_ids;   // [max(1, n)]
  int32_t* cached_ids;  // [max(1, n)]
  int32_t* slot_off;    // [n+1]
  int32_t* jobs;        // [max(1, n)][kJobCols]
  int32_t* slots;
  int slots_cap;
  int64_t* positions;
  int64_t* token_index;
  int rows_cap;
  int32_t* smp_params;  // [n][5]
  int64_t* smp_rows;
  int win_cap;
  int32_t* counts;      // [8]
};

__device__ __forceinline__ int keep_count(int kc, double ratio) {
  const long long f = (long long)((double)kc * ratio);  // int() truncates toward zero
  long long k = f > 1 ? f : 1;
  return (int)(k < kc ? k : kc);
}

// Exclusive prefix sums of N values per thread over the workgroup, all N
// scanned together (two barriers in all): ex[n] receives the thread's prefix
// of value n and tot[n] the workgroup's total.  lds holds 16 * N ints.
template <int N>
__device__ void block_exscan_n(const int (&v)[N], int (&ex)[N], int (&tot)[N], int* lds) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x[N];
#pragma unroll
  for (int n = 0; n < N; ++n) x[n] = wave_incl_scan(v[n]);
  if (lane == 63)
#pragma unroll
    for (int n = 0; n < N; ++n) lds[wave * N + n] = x[n];
  __syncthreads();
  const int nw = (int)(blockDim.x >> 6);
#pragma unroll
  for (int n = 0; n < N; ++n) {
    int base = 0, all = 0;
    for (int w = 0; w < nw; ++w) {
      const int s = lds[w * N + n];
      if (w < wave) base += s;
      all += s;
    }
    ex[n] = base + x[n] - v[n];
    tot[n] = all;
  }
  __syncthreads();  // lds may be reused
}

__global__ __launch_bounds__(1024) void step_build_kernel(StepBuildArgs a) {
  __shared__ int s_rows[kStepMaxSeq], s_start[kStepMaxSeq], s_cu[kStepMaxSeq];
  __shared__ int s_keep[kStepMaxSeq], s_sbase[kStepMaxSeq], s_pages[kStepMaxSeq];
  __shared__ int s_wlo[kStepMaxSeq], s_wn[kStepMaxSeq], s_woff[kStepMaxSeq];
  __shared__ int s_dense_rows[kStepMaxSeq];  // rows of a full-attention sequence, -1 otherwise
  __shared__ int s_npages[kStepMaxSeq];
  __shared__ int s_srange[kStepMaxSeq], s_sseq[kStepMaxSeq];  // slot ranges in slot order: start, sequence
  __shared__ int s_scan[16 * 8];
  const int i = threadIdx.x;
  const bool live = i < a.n;
  int mode = -1, rows = 0, start = 0, bs = 0, bl = 0, keep = 0, wlo = 0, wn = 0, sr = 0, first = 0, err = 0;
  int hsel = 0, pool = 1;
  if (live) {
    const int32_t* s = a.state + (int64_t)i * kStateCols;
    const int P = s[0], N = s[1], sparse = s[2], blen_cfg = s[3], bidx = s[4], sib = s[5], cs = s[6];
    const int steps = s[8], cur = s[9];
    hsel = s[10];
    pool = s[11];
    if (!sparse) {
      mode = 0;
      rows = N;
      wlo = P;
      wn = N - P;
      sr = steps - cur;
    } else {
      int b0, blen;  // compute_block_boundaries (state.py:42-62)
      if (N - P <= 0) {
        b0 = P;
        blen = 0;
      } else {
        b0 = P + bidx * blen_cfg;
        blen = min(blen_cfg, N - b0);
      }
      wlo = b0;
      wn = max(0, blen);
      sr = wn - sib;
      first = (cs == 0 && wn > 0) ? 1 : 0;
      if (cs == 0) {
        mode = 0;
        rows = N;
      } else if (cs == 1) {
        mode = 1;
        rows = N;
        bs = b0;
        bl = b0 < N ? max(0, min(max(0, blen), N - b0)) : 0;
        if (bl == 0) err = 2;
        keep = keep_count(N - bl, a.ratio[i]);
      } else if (cs == 2) {
        if (blen < 0) err = 3;
        mode = 2;
        rows = max(0, blen);
        start = b0;
        bs = b0;
        bl = rows;
        keep = keep_count(max(0, b0) + max(0, N - (b0 + blen)), a.ratio[i]);
      } else {
        err = 5;
        rows = N;
      }
    }
    if (sr == 0) err = err ? err : 4;
  }
  const int vals[8] = {rows, live && (mode == 0 || mode == 1), live && mode == 2, live && mode == 1,
                       mode == 2 ? keep : 0, mode == 1 ? keep : 0, wn, err != 0};
  int ex[8], tot[8];
  block_exscan_n<8>(vals, ex, tot, s_scan);
  const int cu0 = ex[0], c_at = ex[2], j_at = ex[3], ck = ex[4], jk = ex[5], woff = ex[6];
  const int tot_rows = tot[0], n_dense = tot[1], n_cached = tot[2], n_job = tot[3];
  const int tot_cached_keep = tot[4], tot_job_keep = tot[5], tot_win = tot[6], any_err = tot[7];
  // state-2 sequences' slots first, then state-1 sequences'
  const int sbase = mode == 2 ? ck : tot_cached_keep + jk;
  const int tot_slots = tot_cached_keep + tot_job_keep;
  const bool fits = tot_rows <= a.rows_cap && tot_slots <= a.slots_cap && tot_win <= a.win_cap;
  if (live) {
    s_rows[i] = rows;
    s_start[i] = start;
    s_cu[i] = cu0;
    s_keep[i] = (mode == 1 || mode == 2) ? keep : 0;
    s_sbase[i] = sbase;
    s_pages[i] = a.page_off[i];
    s_npages[i] = a.page_off[i + 1] - a.page_off[i];
    s_wlo[i] = wlo;
    s_wn[i] = wn;
    s_woff[i] = woff;
    a.cu[i] = cu0;
    s_dense_rows[i] = (mode == 0 || mode == 1) ? rows : -1;
    if (mode == 2) {
      a.cached_ids[c_at] = i;
      a.slot_off[c_at] = sbase;
      s_srange[c_at] = sbase;
      s_sseq[c_at] = i;
    }
    if (mode == 1) {
      s_srange[n_cached + j_at] = sbase;
      s_sseq[n_cached + j_at] = i;
    }
    if (mode == 1) {
      int32_t* j = a.jobs + kJobCols * (int64_t)j_at;
      j[0] = cu0;
      j[1] = rows;
      j[2] = bs;
      j[3] = bl;
      j[4] = keep;
      j[5] = sbase;
      j[6] = hsel;
      j[7] = pool;
    }
    int32_t* p = a.smp_params + 5 * (int64_t)i;
    p[0] = (int32_t)((int64_t)i * a.tok_stride + wlo);
    p[1] = wn;
    p[2] = woff;
    p[3] = sr;
    p[4] = first;
  }
  if (i == 0) {
    a.cu[a.n] = tot_rows;
    a.slot_off[n_cached] = tot_cached_keep;
    if (n_dense == 0) a.dense_ids[0] = 0;
    if (n_cached == 0) a.cached_ids[0] = 0;
    if (n_job == 0)
      for (int c = 0; c < kJobCols; ++c) a.jobs[c] = 0;
    a.counts[0] = tot_rows;
    a.counts[1] = n_dense;
    a.counts[2] = n_cached;
    a.counts[3] = n_job;
    a.counts[4] = tot_slots;
    a.counts[5] = tot_win;
    a.counts[6] = !fits ? 1 : 0;
    a.counts[7] = any_err;
  }
  __syncthreads();
  // full-attention sequences longest first, ties by index (the host's order)
  if (live && s_dense_rows[i] >= 0) {
    const int ri = s_dense_rows[i];
    int rank = 0;
    for (int j = 0; j < a.n; ++j) {
      const int rj = s_dense_rows[j];
      rank += (rj > ri || (rj == ri && j < i)) ? 1 : 0;
    }
    a.dense_ids[rank] = i;
  }
  if (!fits) return;  // uniform: the host sizes the buffers from the same state
  // Per-row, per-slot and per-window arrays, each flattened over the whole
  // batch: element e belongs to the last sequence (range) whose start is
  // <= e, found by binary search over the starts in LDS (all starts are in
  // ascending order; empty ranges are skipped by taking the last match).
  auto owner = [&](const int* starts, int n, int e) {
    int lo = 0, hi = n - 1;  // starts[0] <= e
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (starts[mid] <= e) lo = mid; else hi = mid - 1;
    }
    return lo;
  };
  for (int e = threadIdx.x; e < tot_rows; e += blockDim.x) {
    const int q = owner(s_cu, a.n, e);
    const int t = e - s_cu[q], st = s_start[q];
    a.positions[e] = st + t;
    a.token_index[e] = (int64_t)q * a.tok_stride + st + t;
  }
  const int n_ranges = n_cached + n_job;
  for (int e = threadIdx.x; e < tot_slots; e += blockDim.x) {
    const int k = owner(s_srange, n_ranges, e);
    const int q = s_sseq[k];
    const int r = e - s_srange[k];
    const int pg = r >> 8;
    a.slots[e] = pg < s_npages[q] ? a.pages[s_pages[q] + pg] * 256 + (r & 255) : -1;
  }
  for (int e = threadIdx.x; e < tot_win; e += blockDim.x) {
    const int q = owner(s_woff, a.n, e);
    a.smp_rows[e] = s_cu[q] + s_wlo[q] - s_start[q] + (e - s_woff[q]);
  }
}

// Sequence.advance + PerRequestSparseState.advance_step (state.py:77-104).
__global__ __launch_bounds__(256) void step_advance_kernel(int32_t* state, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int32_t* s = state + (int64_t)i * kStateCols;
  s[9] += 1;
  if (!s[2]) return;
  int sib = s[5] + 1;
  if (sib % s[3] == 0) {
    sib = 0;
    s[4] += 1;
  }
  s[5] = sib;
  const int d = s[7];
  int cs;
  if (d == 1)
    cs = sib == 0 ? 0 : (sib == 1 ? 1 : 2);
  else if (d == 0)
    cs = sib == 0 ? 1 : 2;
  else
    cs = sib < d ? 0 : (sib == d ? 1 : 2);
  s[6] = cs;
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_step_build(const int32_t* seq_state, const double* ratio, const int32_t* pages,
                               const int32_t* page_off, int n_seq, int64_t tok_stride, int32_t* cu,
                               int32_t* dense_ids, int32_t* cached_ids, int32_t* slot_off, int32_t* jobs,
                               int32_t* slots, int slots_cap, int64_t* positions, int64_t* token_index,
                               int rows_cap, int32_t* smp_params, int64_t* smp_rows, int win_cap, int32_t* counts,
                               void* stream) {
  static const char* name = "dllm_step_build";
  if (n_seq <= 0 || n_seq > kStepMaxSeq)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: %d sequences (1..%d supported)", name, n_seq, kStepMaxSeq);
  if (slots_cap < 0 || rows_cap < 0 || win_cap < 0 || tok_stride < 0)
    return fail(DLLM_ERR_INVALID_ARG, "%s: negative capacity or stride", name);
  if (!seq_state || !ratio || !page_off || !cu || !dense_ids || !cached_ids || !slot_off || !jobs || !smp_params ||
      !counts || (slots_cap && !slots) || (rows_cap && (!positions || !token_index)) || (win_cap && !smp_rows))
    return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  if ((int64_t)n_seq * tok_stride > INT32_MAX)
    return fail(DLLM_ERR_INVALID_ARG, "%s: token table exceeds int32 offsets", name);
  StepBuildArgs a;
  a.state = seq_state;
  a.ratio = ratio;
  a.pages = pages;
  a.page_off = page_off;
  a.n = n_seq;
  a.tok_stride = tok_stride;
  a.cu = cu;
  a.dense_ids = dense_ids;
  a.cached_ids = cached_ids;
  a.slot_off = slot_off;
  a.jobs = jobs;
  a.slots = slots;
  a.slots_cap = slots_cap;
  a.positions = positions;
  a.token_index = token_index;
  a.rows_cap = rows_cap;
  a.smp_params = smp_params;
  a.smp_rows = smp_rows;
  a.win_cap = win_cap;
  a.counts = counts;
  step_build_kernel<<<dim3(1), dim3(1024), 0, reinterpret_cast<hipStream_t>(stream)>>>(a);
  return check_launch(name);
}

extern "C" int dllm_step_advance(int32_t* seq_state, int n_seq, void* stream) {
  static const char* name = "dllm_step_advance";
  if (n_seq < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (n_seq == 0) return DLLM_OK;
  if (!seq_state) return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  step_advance_kernel<<<dim3((unsigned)((n_seq + 255) / 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      seq_state, n_seq);
  return check_launch(name);
}

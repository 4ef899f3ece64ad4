// K5 / K6: per-KV-head (head_select) or shared (token) top-k selection of the
// non-block K/V rows of a sequence, fused with the KV-cache scatter.  Each
// job (sequence) carries its own head_select and pool_kernel, so one launch
// serves a step whose sequences use different SparseConfigs.
//
// Four launches per call:
//   1. qbar_kernel   block mean of q per (job, query head): the block rows
//                    are staged through LDS and summed in f64, rows in
//                    order, one thread per two d.
//   2. score_kernel  per (job, KV head, 256 candidates): the candidates' K
//                    rows of that head are loaded coalesced into LDS, then
//                    each lane computes its candidate's dot products with
//                    the g query heads of the KV head (f64, d ascending):
//                    head_select -> the bf16 maximum over the g heads;
//                    token selection -> the f64 sum of the g dots.
//   3. topk_kernel   per (job, selection head): pool + scale into 16-bit
//                    order keys, a two-level byte histogram finds the
//                    threshold key of the n_keep-th best candidate, an
//                    index-order compaction takes every better candidate and
//                    the first ties, and a sort orders the n_keep selected
//                    rows (score descending, candidate index ascending):
//                    bitonic over unique 64-bit keys in LDS, or for more than
//                    kSortCap rows a stable two-pass radix sort in the
//                    workspace.  No limit on the candidate count.
//   4. sel_copy_kernel  copies every selected (rank, head) row piece, 16
//                    bytes per thread, into its cache slot.
// The arithmetic follows a fixed, order-defined rule (f64 sums in a stated
// order, explicit f32 / bf16 rounding points, ties to the lower candidate
// index), so the selected indices are reproducible bit for bit on the CPU.
#include "common.h"

#include <math.h>

namespace dllm {

constexpr int SHD = 128;           // the head dim these kernels handle
constexpr int kJobCols = 8;        // row0, n_tok, blk_start, blk_len, n_keep, slot_off, head_select, pool_k
constexpr int kScoreCands = 256;   // candidates per score workgroup
constexpr int kQbarRows = 64;      // block rows staged per qbar round
constexpr int kTopkThreads = 1024;
constexpr int kSortCap = 8192;     // selected rows sorted in LDS as 64-bit keys
constexpr int kMaxGroup = 64;      // query heads per KV head

struct SelArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t n_rows;
  int64_t q_stride, k_stride, v_stride;
  const int32_t* jobs;  // [n_job][kJobCols]
  int n_job, max_kc, max_keep;
  int Hq, Hkv, g;
  float sqrt_d;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t cache_slots;
  const int32_t* slots;
  int64_t n_slots;
  int64_t* idx_out;  // [n_job][Hkv][max_keep] or null
  // workspace
  uint16_t* qbar;    // [n_job][Hq][128] bf16 bits
  uint16_t* raw;     // [n_job][Hkv][max_kc] bf16 bits (head_select jobs)
  double* part;      // [n_job][Hkv][max_kc] per-KV-head sums (token-selection jobs)
  uint16_t* okey;    // [n_job][Hkv][max_kc] pooled order keys
  int32_t* sel;      // [n_job][Hkv][max_keep] selected candidates, best first
  uint16_t* ckey0;   // [n_job][Hkv][max_keep] x2: the large-sort ping-pong
  uint16_t* ckey1;
  int32_t* cidx0;
  int32_t* cidx1;
};

struct Job {
  int row0, n_tok, bs, bl, n_keep, slot_off, head_select, pool_k;
  int kc;  // candidates: n_tok - bl, clamped to the launch's max_kc
};

// The job as the kernels use it.  Its sizes are clamped to what the launch
// covers (kc <= max_kc, n_keep <= min(max_keep, kc)), and a job whose rows,
// block or slots fall outside the tensors selects nothing, so device-built
// tables that disagree with the host's launch sizes cannot write outside the
// workspace, the cache or the slot list.
__device__ __forceinline__ Job load_job(const SelArgs& a, int j) {
  const int32_t* p = a.jobs + (int64_t)kJobCols * j;
  Job jb{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], 0};
  const bool ok = jb.row0 >= 0 && jb.n_tok > 0 && (int64_t)jb.row0 + jb.n_tok <= a.n_rows && jb.bl > 0 &&
                  jb.bs >= 0 && jb.bs + jb.bl <= jb.n_tok && jb.slot_off >= 0;
  int kc = ok ? jb.n_tok - jb.bl : 0;
  kc = min(kc, a.max_kc);
  int nk = min(max(jb.n_keep, 0), min(a.max_keep, kc));
  if ((int64_t)jb.slot_off + nk > a.n_slots) nk = 0;
  jb.kc = nk > 0 ? kc : 0;
  jb.n_keep = nk;
  return jb;
}

// Candidate j (prefix rows, then suffix rows) -> row offset inside the sequence.
__device__ __forceinline__ int cand_row(const Job& jb, int j) { return j < jb.bs ? j : j + jb.bl; }

__device__ __forceinline__ float bf16_val(uint32_t b) { return bf16_bits_to_f32(b); }

// Order-preserving map of a bf16 pattern to an unsigned 16-bit key (-0 == +0).
__device__ __forceinline__ uint32_t bf16_order_key(uint32_t b) {
  if (b == 0x8000u) b = 0u;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

// Exclusive prefix count of `flag` over the workgroup (wavefronts in order);
// *total receives the workgroup's count.  Every thread must call it.
__device__ int block_excount(bool flag, int* wave_tot, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t m = __builtin_amdgcn_ballot_w64(flag);
  const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
  __syncthreads();
  if (lane == 0) wave_tot[wave] = __builtin_popcountll(m);
  __syncthreads();
  int base = 0, all = 0;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) {
    const int t = wave_tot[w];
    base += w < wave ? t : 0;
    all += t;
  }
  *total = all;
  return base + below;
}

// ---- 1. block mean of q ------------------------------------------------------
// grid (n_job, ceil(Hq / 4)), block 256 = 4 query heads x 64 threads:
// qbar[j][h][d] = bf16(f32(f64 sum_t q[bs+t][h][d] / bl)), t ascending.  The
// block rows of the 4 heads go through LDS kQbarRows at a time (every load of
// a round in flight together); thread (head, l) then sums d = 2l and 2l + 1
// row by row (64 lanes read 64 consecutive words: no bank conflicts).
constexpr int kQbarHeads = 4;
__global__ __launch_bounds__(256) void qbar_kernel(SelArgs a) {
  __shared__ uint32_t tile[kQbarRows * kQbarHeads * 64];  // [row][head][64 words]
  const int jid = blockIdx.x;
  const int h0 = blockIdx.y * kQbarHeads;
  const Job jb = load_job(a, jid);
  if (jb.n_keep <= 0) return;
  const int tid = threadIdx.x;
  const int hh = tid >> 6, l = tid & 63;
  const uint16_t* q0 = a.q + ((int64_t)jb.row0 + jb.bs) * a.q_stride + (int64_t)h0 * SHD;
  double s0 = 0.0, s1 = 0.0;
  for (int t0 = 0; t0 < jb.bl; t0 += kQbarRows) {
    const int n = min(kQbarRows, jb.bl - t0);
    // load: 16-byte chunk ch of (row r, head hl): 64 chunks per row, 4 rows per pass
    for (int i = tid; i < n * kQbarHeads * 16; i += blockDim.x) {
      const int r = i / (kQbarHeads * 16), rem = i - r * (kQbarHeads * 16);
      const int hl = rem >> 4, ch = rem & 15;
      if (h0 + hl < a.Hq)
        *reinterpret_cast<u32x4_t*>(tile + (r * kQbarHeads + hl) * 64 + ch * 4) =
            ld128(q0 + (int64_t)(t0 + r) * a.q_stride + hl * SHD + ch * 8);
    }
    __syncthreads();
    if (h0 + hh < a.Hq) {
      for (int r = 0; r < n; ++r) {
        const uint32_t w = tile[(r * kQbarHeads + hh) * 64 + l];
        s0 += (double)bf16_val(w & 0xffffu);
        s1 += (double)bf16_val(w >> 16);
      }
    }
    __syncthreads();
  }
  if (h0 + hh < a.Hq) {
    uint16_t* out = a.qbar + ((int64_t)jid * a.Hq + h0 + hh) * SHD + 2 * l;
    out[0] = (uint16_t)f64_to_bf16_bits_2step(s0 / (double)jb.bl);
    out[1] = (uint16_t)f64_to_bf16_bits_2step(s1 / (double)jb.bl);
  }
}

// ---- 2. scores ---------------------------------------------------------------
// grid (ceil(max_kc / 256), Hkv, n_job), block 256, dynamic LDS = 64 KiB of K
// rows + the g query heads' qbar as f32.  K rows: 16 lanes per 256-byte row,
// stored with 16-byte chunk c at c ^ (row & 15) so that the per-lane row reads
// afterwards (lane = row) spread over all banks.
// dot(h, j) = sum_d qbar[h][d] * k[j][kv][d] in f64, d ascending (each product
// of two bf16 values is exact in f64, so fma gives the same sums).
__global__ __launch_bounds__(256) void score_kernel(SelArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* kt = lds;
  float* qs = reinterpret_cast<float*>(lds + kScoreCands * 256);
  const int jid = blockIdx.z;
  const int kv = blockIdx.y;
  const Job jb = load_job(a, jid);
  const int c0 = blockIdx.x * kScoreCands;
  if (c0 >= jb.kc) return;
  const int g = a.g;
  const int tid = threadIdx.x;
  const int rsub = tid >> 4, ch = tid & 15;
  u32x4_t rows[kScoreCands / 16];
#pragma unroll
  for (int p = 0; p < kScoreCands / 16; ++p) {
    const int c = c0 + 16 * p + rsub;
    const int64_t row = (int64_t)jb.row0 + cand_row(jb, min(c, jb.kc - 1));
    rows[p] = ld128(a.k + row * a.k_stride + (int64_t)kv * SHD + ch * 8);
  }
  const uint16_t* qb = a.qbar + ((int64_t)jid * a.Hq + (int64_t)kv * g) * SHD;
  for (int i = tid; i < g * SHD; i += blockDim.x) qs[i] = bf16_val(qb[i]);
#pragma unroll
  for (int p = 0; p < kScoreCands / 16; ++p) {
    const int r = 16 * p + rsub;
    *reinterpret_cast<u32x4_t*>(kt + r * 256 + ((ch ^ (r & 15)) << 4)) = rows[p];
  }
  __syncthreads();
  const int c = c0 + tid;
  if (c >= jb.kc) return;
  // lane tid reads row tid; physical chunk cl ^ (tid & 15) (the 16 lanes of a
  // read group hit 16 different chunks)
  const uint8_t* krow = kt + tid * 256;
  const int sw = tid & 15;
  const int64_t out = ((int64_t)jid * a.Hkv + kv) * a.max_kc + c;
  float best = -INFINITY;
  double part = 0.0;
  for (int gi = 0; gi < g; ++gi) {
    const float* qq = qs + gi * SHD;
    double acc = 0.0;
#pragma unroll 4
    for (int cl = 0; cl < 16; ++cl) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(krow + ((cl ^ sw) << 4));
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        acc = __builtin_fma((double)qq[8 * cl + 2 * w], (double)bf16_val(x[w] & 0xffffu), acc);
        acc = __builtin_fma((double)qq[8 * cl + 2 * w + 1], (double)bf16_val(x[w] >> 16), acc);
      }
    }
    best = fmaxf(best, bf16_val(f64_to_bf16_bits_2step(acc)));
    part += acc;
  }
  if (jb.head_select)
    a.raw[out] = (uint16_t)(__float_as_uint(best) >> 16);
  else
    a.part[out] = part;
}

// ---- 3. top-k ------------------------------------------------------------------
// Bitonic sort, descending, of n (a power of two) unique 64-bit keys in LDS.
__device__ void bitonic_desc_u64(uint64_t* keys, int n) {
  for (int kk = 2; kk <= n; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int ixj = i ^ jj;
        if (ixj > i) {
          const uint64_t x = keys[i], y = keys[ixj];
          const bool desc = (i & kk) == 0;
          if (desc ? (x < y) : (x > y)) {
            keys[i] = y;
            keys[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Bitonic sort, ascending, of the workgroup's 1024 32-bit values (one per thread).
__device__ void bitonic_asc_1024(uint32_t* v) {
  for (int kk = 2; kk <= kTopkThreads; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      const int i = threadIdx.x;
      const int ixj = i ^ jj;
      if (ixj > i) {
        const uint32_t x = v[i], y = v[ixj];
        const bool asc = (i & kk) == 0;
        if (asc ? (x > y) : (x < y)) {
          v[i] = y;
          v[ixj] = x;
        }
      }
      __syncthreads();
    }
  }
}

struct TopkShared {
  uint32_t hist[256];
  int start[257];
  int running[256];
  int wave_tot[16];
  uint32_t chunk[kTopkThreads];
  int misc[4];  // threshold search results: high byte, count above it, low byte, count above T
};

// One stable counting pass of the large-sort path: elements [0, n) of
// (in_key, in_idx), in their current order, go to out (key, idx) ordered by
// the digit 255 - ((key >> shift) & 255) ascending, ties in input order.  The
// workgroup walks the input in chunks of 1024; inside a chunk each element's
// rank among equal digits comes from a bitonic sort of (digit, position)
// pairs.  out_key may be null (last pass).
__device__ void radix_pass(TopkShared& sh, const uint16_t* in_key, const int32_t* in_idx, uint16_t* out_key,
                           int32_t* out_idx, int n, int shift, int64_t* idx_out) {
  const int tid = threadIdx.x;
  for (int b = tid; b < 256; b += blockDim.x) sh.hist[b] = 0;
  __syncthreads();
  for (int e = tid; e < n; e += blockDim.x) atomicAdd(&sh.hist[255 - ((in_key[e] >> shift) & 255)], 1u);
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    for (int b = 0; b < 256; ++b) {
      sh.running[b] = s;
      s += (int)sh.hist[b];
    }
  }
  __syncthreads();
  for (int b0 = 0; b0 < n; b0 += kTopkThreads) {
    const int e = b0 + tid;
    const uint32_t d = e < n ? 255u - ((in_key[e] >> shift) & 255u) : 256u;
    sh.chunk[tid] = (d << 10) | (uint32_t)tid;
    __syncthreads();
    bitonic_asc_1024(sh.chunk);
    const uint32_t x = sh.chunk[tid];
    const int dx = (int)(x >> 10);
    const int dprev = tid > 0 ? (int)(sh.chunk[tid - 1] >> 10) : -1;
    if (dx != dprev) sh.start[dx] = tid;
    __syncthreads();
    const int rank = tid - sh.start[dx];
    if (dx < 256) {
      const int dest = sh.running[dx] + rank;
      const int src = b0 + (int)(x & 1023u);
      const int32_t ix = in_idx[src];
      if (out_key) out_key[dest] = in_key[src];
      out_idx[dest] = ix;
      if (idx_out) idx_out[dest] = ix;
    }
    __syncthreads();
    const int dnext = tid + 1 < kTopkThreads ? (int)(sh.chunk[tid + 1] >> 10) : 257;
    if (dx < 256 && dnext != dx) sh.running[dx] += rank + 1;
    __syncthreads();
  }
}

// Threshold bin of a 256-bin histogram: the bin b, scanning from 255 down,
// where cum0 + count(bins above b) < nk <= cum0 + count(bins >= b).  Wavefront
// 0 searches (lane l holds bins 255-4l .. 252-4l and a prefix scan over the
// lanes gives each its count above); out[0] = b, out[1] = cum0 + count above b.
// The caller must hold a barrier before (hist complete) and after (out read).
__device__ void find_bin(const uint32_t* hist, int nk, int cum0, int* out) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  int h[4], own = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = (int)hist[255 - 4 * lane - i];
    own += h[i];
  }
  int incl = own;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  int run = cum0 + incl - own, hit = -1, hit_run = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (hit < 0 && run + h[i] >= nk) {
      hit = 255 - 4 * lane - i;
      hit_run = run;
    }
    run += h[i];
  }
  const uint64_t m = __builtin_amdgcn_ballot_w64(hit >= 0);
  const int first = m ? __builtin_ctzll(m) : 63;   // the lane holding the highest such bin
  if (lane == first) {
    out[0] = hit >= 0 ? hit : 0;
    out[1] = hit >= 0 ? hit_run : cum0;
  }
}

// Bitonic sort, descending, of one 32-bit value per thread over the first n
// threads (n a power of two <= 1024; the other threads hold values sorted
// among themselves).  Strides below 64 exchange within the wavefront by
// lane permutes; larger ones go through `xchg` (1024 words of LDS).
__device__ uint32_t bitonic_desc_reg(uint32_t x, int n, uint32_t* xchg) {
  const int p = threadIdx.x;
  for (int kk = 2; kk <= n; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      uint32_t y;
      if (jj >= 64) {
        __syncthreads();
        xchg[p] = x;
        __syncthreads();
        y = xchg[p ^ jj];
      } else {
        y = (uint32_t)__shfl_xor((int)x, jj);
      }
      const bool low = (p & jj) == 0, desc = (p & kk) == 0;
      x = (low == desc) ? max(x, y) : min(x, y);
    }
  }
  return x;
}

constexpr int kLdsCand = 16384;  // candidates whose raw scores and order keys stay in LDS
constexpr int kRegSort = 1024;   // selected rows sorted one per thread in registers

// bf16 bits of the raw score of candidate u before the division by sqrt(D): the
// stored group maximum (head_select), or bf16 of the KV heads' partial sums added
// in head order (token selection)
__device__ __forceinline__ uint16_t raw_bits(const SelArgs& a, const Job& jb, int jid, int h, int u) {
  if (jb.head_select) return a.raw[((int64_t)jid * a.Hkv + h) * a.max_kc + u];
  double t = 0.0;
  const double* p = a.part + (int64_t)jid * a.Hkv * a.max_kc + u;
  for (int kv = 0; kv < a.Hkv; ++kv) t += p[(int64_t)kv * a.max_kc];
  return (uint16_t)f64_to_bf16_bits_2step(t);
}

// grid (Hkv, n_job), block 1024.  Token-selection jobs use selection head 0 only.
// LDS: 128 KiB pool (small path: raw bits, order keys and 32-bit sort keys of
// up to kLdsCand candidates; large path: kSortCap 64-bit sort keys) + the
// shared scratch.
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(SelArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t pool[128 * 1024];
  __shared__ TopkShared sh;
  const int h = blockIdx.x;
  const int jid = blockIdx.y;
  const Job jb = load_job(a, jid);
  if (!jb.head_select && h > 0) return;
  const int kc = jb.kc, nk = jb.n_keep;
  if (kc <= 0 || nk <= 0) return;
  const int tid = threadIdx.x;
  const int64_t base = ((int64_t)jid * a.Hkv + h) * a.max_kc;
  const int64_t sbase = ((int64_t)jid * a.Hkv + h) * a.max_keep;
  const int pk = jb.pool_k;
  const int pad = pk / 2;
  int64_t* io = a.idx_out ? a.idx_out + sbase : nullptr;
  int32_t* so = a.sel + sbase;
  for (int b = tid; b < 256; b += blockDim.x) sh.hist[b] = 0;

  if (kc <= kLdsCand) {
    // ---- small path: everything in LDS -------------------------------------
    uint16_t* rawl = reinterpret_cast<uint16_t*>(pool);
    uint16_t* okl = rawl + kLdsCand;
    uint32_t* skey = reinterpret_cast<uint32_t*>(pool + 64 * 1024);
    for (int c = tid; c < kc; c += blockDim.x) rawl[c] = raw_bits(a, jb, jid, h, c);
    __syncthreads();
    // pooled, scaled order keys (max over the window clipped to the
    // candidates, then bf16(f32 / f32(sqrt D)): monotone, so pooling before
    // or after the division gives the same value) and the high-byte histogram
    for (int c = tid; c < kc; c += blockDim.x) {
      const int lo = pk > 1 ? max(0, c - pad) : c;
      const int hi = pk > 1 ? min(kc - 1, c - pad + pk - 1) : c;
      float m = -INFINITY;
      for (int u = lo; u <= hi; ++u) m = fmaxf(m, bf16_val(rawl[u]));
      const uint32_t key = bf16_order_key(f32_to_bf16_bits(m / a.sqrt_d));
      okl[c] = (uint16_t)key;
      atomicAdd(&sh.hist[key >> 8], 1u);
    }
    __syncthreads();
    find_bin(sh.hist, nk, 0, sh.misc);
    __syncthreads();
    const uint32_t hb = (uint32_t)sh.misc[0];
    const int above_hb = sh.misc[1];
    for (int b = tid; b < 256; b += blockDim.x) sh.hist[b] = 0;
    __syncthreads();
    for (int c = tid; c < kc; c += blockDim.x) {
      const uint32_t key = okl[c];
      if ((key >> 8) == hb) atomicAdd(&sh.hist[key & 255], 1u);
    }
    __syncthreads();
    find_bin(sh.hist, nk, above_hb, sh.misc + 2);
    __syncthreads();
    const uint32_t T = (hb << 8) | (uint32_t)sh.misc[2];
    const int need_eq = nk - sh.misc[3];  // ties at T to take, lowest indices first
    // index-order compaction; unique keys: score key, then the complement of the candidate
    int run_eq = 0, run_pos = 0;
    for (int b0 = 0; b0 < kc; b0 += kTopkThreads) {
      const int c = b0 + tid;
      const uint32_t key = c < kc ? okl[c] : 0u;
      const bool gt = c < kc && key > T;
      const bool eq = c < kc && key == T;
      int eq_tot, sel_tot;
      const int er = block_excount(eq, sh.wave_tot, &eq_tot) + run_eq;
      const bool take = gt || (eq && er < need_eq);
      const int pos = block_excount(take, sh.wave_tot, &sel_tot) + run_pos;
      if (take) skey[pos] = (key << 16) | (uint32_t)(0xffff - c);
      run_eq += eq_tot;
      run_pos += sel_tot;
    }
    int P2 = 1;
    while (P2 < nk) P2 <<= 1;
    __syncthreads();
    if (P2 <= kRegSort) {
      uint32_t x = tid < nk ? skey[tid] : 0u;  // 0 sorts below every real key
      x = bitonic_desc_reg(x, P2, sh.chunk);
      if (tid < nk) {
        const int c = 0xffff - (int)(x & 0xffffu);
        so[tid] = c;
        if (io) io[tid] = c;
      }
    } else {
      for (int i = nk + tid; i < P2; i += blockDim.x) skey[i] = 0u;
      __syncthreads();
      for (int kk = 2; kk <= P2; kk <<= 1) {
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
          for (int i = tid; i < P2; i += blockDim.x) {
            const int ixj = i ^ jj;
            if (ixj > i) {
              const uint32_t x = skey[i], y = skey[ixj];
              const bool desc = (i & kk) == 0;
              if (desc ? (x < y) : (x > y)) {
                skey[i] = y;
                skey[ixj] = x;
              }
            }
          }
          __syncthreads();
        }
      }
      for (int r = tid; r < nk; r += blockDim.x) {
        const int c = 0xffff - (int)(skey[r] & 0xffffu);
        so[r] = c;
        if (io) io[r] = c;
      }
    }
    return;
  }

  // ---- large path: order keys in the workspace -------------------------------
  uint64_t* skey = reinterpret_cast<uint64_t*>(pool);
  uint16_t* ok = a.okey + base;
  __syncthreads();
  for (int c = tid; c < kc; c += blockDim.x) {
    const int lo = pk > 1 ? max(0, c - pad) : c;
    const int hi = pk > 1 ? min(kc - 1, c - pad + pk - 1) : c;
    float m = -INFINITY;
    for (int u = lo; u <= hi; ++u) m = fmaxf(m, bf16_val(raw_bits(a, jb, jid, h, u)));
    const uint32_t key = bf16_order_key(f32_to_bf16_bits(m / a.sqrt_d));
    ok[c] = (uint16_t)key;
    atomicAdd(&sh.hist[key >> 8], 1u);
  }
  __syncthreads();  // also makes the workgroup's own global writes visible to it
  find_bin(sh.hist, nk, 0, sh.misc);
  __syncthreads();
  const uint32_t hb = (uint32_t)sh.misc[0];
  const int above_hb = sh.misc[1];
  for (int b = tid; b < 256; b += blockDim.x) sh.hist[b] = 0;
  __syncthreads();
  for (int c = tid; c < kc; c += blockDim.x) {
    const uint32_t key = ok[c];
    if ((key >> 8) == hb) atomicAdd(&sh.hist[key & 255], 1u);
  }
  __syncthreads();
  find_bin(sh.hist, nk, above_hb, sh.misc + 2);
  __syncthreads();
  const uint32_t T = (hb << 8) | (uint32_t)sh.misc[2];
  const int need_eq = nk - sh.misc[3];
  const bool small = nk <= kSortCap;

  // index-order compaction of the selected candidates
  int run_eq = 0, run_pos = 0;
  for (int b0 = 0; b0 < kc; b0 += kTopkThreads) {
    const int c = b0 + tid;
    const uint32_t key = c < kc ? ok[c] : 0u;
    const bool gt = c < kc && key > T;
    const bool eq = c < kc && key == T;
    int eq_tot, sel_tot;
    const int er = block_excount(eq, sh.wave_tot, &eq_tot) + run_eq;
    const bool take = gt || (eq && er < need_eq);
    const int pos = block_excount(take, sh.wave_tot, &sel_tot) + run_pos;
    if (take) {
      if (small)
        skey[pos] = ((uint64_t)key << 32) | (uint64_t)(~(uint32_t)c);
      else {
        a.ckey0[sbase + pos] = (uint16_t)key;
        a.cidx0[sbase + pos] = c;
      }
    }
    run_eq += eq_tot;
    run_pos += sel_tot;
  }
  if (small) {
    int P2 = 1;
    while (P2 < nk) P2 <<= 1;
    for (int i = nk + tid; i < P2; i += blockDim.x) skey[i] = 0;  // below every real key
    __syncthreads();
    bitonic_desc_u64(skey, P2);
    for (int r = tid; r < nk; r += blockDim.x) {
      const int c = (int)(~(uint32_t)skey[r]);
      so[r] = c;
      if (io) io[r] = c;
    }
  } else {
    // the compacted list is in candidate order: two stable passes (low byte,
    // then high byte of the key, each descending) leave it ordered by score
    // descending, then candidate index ascending
    __syncthreads();
    radix_pass(sh, a.ckey0 + sbase, a.cidx0 + sbase, a.ckey1 + sbase, a.cidx1 + sbase, nk, 0, nullptr);
    radix_pass(sh, a.ckey1 + sbase, a.cidx1 + sbase, nullptr, so, nk, 8, io);
  }
}

// ---- 4. copy of the selected rows into their cache slots -------------------
// grid (ceil(max_keep * Hkv * 16 / 256), n_job), block 256: thread = one 16-byte
// chunk of one (rank r, KV head) piece; head_select jobs take each head's row
// from its own selection, token-selection jobs the same row for every head.
__global__ __launch_bounds__(256) void sel_copy_kernel(SelArgs a) {
  const int jid = blockIdx.y;
  const Job jb = load_job(a, jid);
  const int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t piece = x >> 4;
  const int ch = (int)(x & 15);
  const int r = (int)(piece / a.Hkv);
  const int h = (int)(piece - (int64_t)r * a.Hkv);
  if (r >= jb.n_keep) return;
  const int j = a.sel[((int64_t)jid * a.Hkv + (jb.head_select ? h : 0)) * a.max_keep + r];
  const int64_t slot = a.slots[jb.slot_off + r];
  if (slot < 0 || slot >= a.cache_slots || j < 0 || j >= jb.kc) return;
  const int64_t row = (int64_t)jb.row0 + cand_row(jb, j);
  const int64_t e = (int64_t)h * SHD + ch * 8;
  const int64_t row_elems = (int64_t)a.Hkv * SHD;
  st128(a.k_cache + slot * row_elems + e, ld128_stream(a.k + row * a.k_stride + e));
  st128(a.v_cache + slot * row_elems + e, ld128_stream(a.v + row * a.v_stride + e));
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct SelLayout {
  size_t qbar, raw, part, okey, sel, ckey, cidx, total;
};

static SelLayout sel_layout(int n_job, int max_kc, int Hq, int Hkv) {
  SelLayout L;
  const size_t nj = (size_t)n_job, kc = (size_t)max_kc, hk = (size_t)Hkv;
  L.qbar = align256(nj * Hq * SHD * 2);
  L.raw = align256(nj * hk * kc * 2);
  L.part = align256(nj * hk * kc * 8);
  L.okey = align256(nj * hk * kc * 2);
  L.sel = align256(nj * hk * kc * 4);  // max_keep <= max_kc
  const bool large = max_kc > kSortCap;
  L.ckey = large ? align256(nj * hk * kc * 2) : 0;
  L.cidx = large ? align256(nj * hk * kc * 4) : 0;
  L.total = L.qbar + L.raw + L.part + L.okey + L.sel + 2 * L.ckey + 2 * L.cidx;
  return L;
}

}  // namespace dllm

using namespace dllm;

extern "C" size_t dllm_select_kv_workspace_size(int n_job, int max_kc, int Hq, int Hkv, int D) {
  (void)D;
  if (n_job <= 0 || max_kc <= 0 || Hq <= 0 || Hkv <= 0) return 0;
  return sel_layout(n_job, max_kc, Hq, Hkv).total;
}

extern "C" int dllm_select_kv_store(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, int64_t n_rows,
                                    int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                                    const int32_t* jobs, int n_job, int max_kc, int max_keep, int Hq, int Hkv, int D,
                                    float sqrt_d, dllm_bf16* k_cache, dllm_bf16* v_cache, int64_t cache_slots,
                                    const int32_t* slots, int64_t n_slots, int64_t* idx_out, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  const char* name = "dllm_select_kv_store";
  set_error("");
  if (D != SHD) return fail(DLLM_ERR_UNSUPPORTED, "%s: head_dim %d not supported (the kernels handle 128)", name, D);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv) return fail(DLLM_ERR_INVALID_ARG, "%s: Hq=%d / Hkv=%d", name, Hq, Hkv);
  if (Hq / Hkv > kMaxGroup)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: %d query heads per KV head (at most %d)", name, Hq / Hkv, kMaxGroup);
  if (n_job < 0 || max_kc < 0 || max_keep < 0 || n_rows < 0 || n_slots < 0)
    return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (n_job == 0 || max_kc == 0 || max_keep == 0) return DLLM_OK;
  if (max_keep > max_kc) return fail(DLLM_ERR_INVALID_ARG, "%s: max_keep %d > max_kc %d", name, max_keep, max_kc);
  if ((int64_t)max_keep * Hkv * 16 / 256 + 1 >= ((int64_t)1 << 31) || (int64_t)max_kc / kScoreCands + 1 >= 65536 * 32)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: %d candidates / %d kept rows exceed the grid", name, max_kc, max_keep);
  if (!q || !k || !v || !jobs || !k_cache || !v_cache || !slots)
    return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache) ||
      q_stride_tok % 8 || k_stride_tok % 8 || v_stride_tok % 8)
    return fail(DLLM_ERR_INVALID_ARG, "%s: q/k/v/caches must be 16-byte aligned with strides multiple of 8", name);
  if (q_stride_tok < (int64_t)Hq * D || k_stride_tok < (int64_t)Hkv * D || v_stride_tok < (int64_t)Hkv * D)
    return fail(DLLM_ERR_INVALID_ARG, "%s: token stride smaller than a token row", name);
  if (!(sqrt_d > 0.f)) return fail(DLLM_ERR_INVALID_ARG, "%s: sqrt_d must be positive", name);
  const SelLayout L = sel_layout(n_job, max_kc, Hq, Hkv);
  if (!workspace || workspace_bytes < L.total)
    return fail(DLLM_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", name, L.total,
                workspace ? workspace_bytes : (size_t)0);
  if (!aligned16(workspace)) return fail(DLLM_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", name);
  SelArgs a = {};
  a.q = q; a.k = k; a.v = v; a.n_rows = n_rows;
  a.q_stride = q_stride_tok; a.k_stride = k_stride_tok; a.v_stride = v_stride_tok;
  a.jobs = jobs; a.n_job = n_job; a.max_kc = max_kc; a.max_keep = max_keep;
  a.Hq = Hq; a.Hkv = Hkv; a.g = Hq / Hkv;
  a.sqrt_d = sqrt_d;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slots = cache_slots;
  a.slots = slots; a.n_slots = n_slots; a.idx_out = idx_out;
  char* ws = reinterpret_cast<char*>(workspace);
  size_t o = 0;
  a.qbar = reinterpret_cast<uint16_t*>(ws + o); o += L.qbar;
  a.raw = reinterpret_cast<uint16_t*>(ws + o); o += L.raw;
  a.part = reinterpret_cast<double*>(ws + o); o += L.part;
  a.okey = reinterpret_cast<uint16_t*>(ws + o); o += L.okey;
  a.sel = reinterpret_cast<int32_t*>(ws + o); o += L.sel;
  if (L.ckey) {
    a.ckey0 = reinterpret_cast<uint16_t*>(ws + o); o += L.ckey;
    a.ckey1 = reinterpret_cast<uint16_t*>(ws + o); o += L.ckey;
    a.cidx0 = reinterpret_cast<int32_t*>(ws + o); o += L.cidx;
    a.cidx1 = reinterpret_cast<int32_t*>(ws + o); o += L.cidx;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  qbar_kernel<<<dim3(n_job, (Hq + kQbarHeads - 1) / kQbarHeads), dim3(256), 0, st>>>(a);
  int rc = check_launch(name);
  if (rc) return rc;
  const size_t score_lds = (size_t)kScoreCands * 256 + (size_t)a.g * SHD * sizeof(float);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(score_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)score_lds);
  if (e != hipSuccess) return fail(DLLM_ERR_HIP, "%s: hipFuncSetAttribute: %s", name, hipGetErrorString(e));
  score_kernel<<<dim3((max_kc + kScoreCands - 1) / kScoreCands, Hkv, n_job), dim3(256), score_lds, st>>>(a);
  if ((rc = check_launch(name))) return rc;
  topk_kernel<<<dim3(Hkv, n_job), dim3(kTopkThreads), 0, st>>>(a);
  if ((rc = check_launch(name))) return rc;
  const int64_t pieces = (int64_t)max_keep * Hkv * 16;
  sel_copy_kernel<<<dim3((unsigned)((pieces + 255) / 256), n_job), dim3(256), 0, st>>>(a);
  return check_launch(name);
}

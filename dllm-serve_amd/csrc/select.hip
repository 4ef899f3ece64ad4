// K5 / K6: per-KV-head (head_select) or shared (token) top-k selection of the
// non-block K/V rows of a sequence, fused with the KV-cache scatter.  Each
// job (sequence) carries its own head_select and pool_kernel, so one launch
// serves a step whose sequences use different SparseConfigs.
//
// Two launches per call:
//   1. score_kernel  per (job, KV head, 256 candidates): the block mean of q
//                    for the g query heads of the KV head (f64 sums, rows in
//                    order; every workgroup of the KV head computes it from
//                    the block rows, while its candidates' K rows are in
//                    flight), the K rows staged coalesced through LDS, then
//                    each lane's dot products with the g heads (f64, d
//                    ascending): head_select -> the bf16 maximum over the g
//                    heads; token selection -> the f64 sum of the g dots.
//   2. topk_kernel   per (job, KV head): pool + scale into 16-bit order
//                    keys, a two-level byte histogram finds the threshold key
//                    of the n_keep-th best candidate, an index-order
//                    compaction takes every better candidate and the first
//                    ties, and a sort orders the n_keep selected rows (score
//                    descending, candidate index ascending): in registers,
//                    bitonic over unique keys in LDS, or for more than
//                    kSortCap rows a stable two-pass radix sort in the
//                    workspace.  No limit on the candidate count.  The
//                    workgroup then copies its KV head's piece of every
//                    selected row into the row's cache slot.  Token-selection
//                    jobs make the same (shared) selection in every KV head's
//                    workgroup.
// The arithmetic follows a fixed, order-defined rule (f64 sums in a stated
// order, explicit f32 / bf16 rounding points, ties to the lower candidate
// index), so the selected indices are reproducible bit for bit on the CPU.
#include "common.h"

#include <math.h>

namespace dllm {

constexpr int SHD = 128;           // the head dim these kernels handle
constexpr int kJobCols = 8;        // row0, n_tok, blk_start, blk_len, n_keep, slot_off, head_select, pool_k
constexpr int kScoreCands = 256;   // candidates per score workgroup (one per thread)
constexpr int kScoreCandsMax = 304;  // per workgroup when that saves a second generation (see the launch)
constexpr int kQbarStage = 32768;  // bytes of block rows staged per qbar chunk (inside the K-tile area)
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
  int n_part;        // top-k workgroups per (job, KV head): each selects, then copies 1/n_part of the rows
  int score_cpw;     // candidates per score workgroup: a multiple of 16 in [kScoreCands, kScoreCandsMax]
  int q_dma;         // every q byte lies within 4 GiB of q: 32-bit buffer offsets reach every block row
  // workspace
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

// Exclusive prefix sums of two per-thread counts over the workgroup
// (wavefronts in order), both in one pass.  Every thread must call it.
__device__ void block_exscan2(int a, int b, int* wave_tot2, int* ex_a, int* ex_b) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int xa = wave_incl_scan(a), xb = wave_incl_scan(b);
  __syncthreads();
  if (lane == 63) {
    wave_tot2[2 * wave] = xa;
    wave_tot2[2 * wave + 1] = xb;
  }
  __syncthreads();
  int ba = 0, bb = 0;
  for (int w = 0; w < wave; ++w) {
    ba += wave_tot2[2 * w];
    bb += wave_tot2[2 * w + 1];
  }
  *ex_a = ba + xa - a;
  *ex_b = bb + xb - b;
}

// ---- 1. scores ---------------------------------------------------------------
// grid (ceil(max_kc / cpw), Hkv, n_job), block 256, dynamic LDS = cpw rows of
// K (256 bytes each; cpw = 256, or up to 304 with threads taking a second
// candidate) + the g query heads' qbar as f64 (padded to four heads when
// 1 < g <= 4, to a multiple of eight above).  K rows: 16 lanes per 256-byte row,
// stored with 16-byte chunk c at c ^ (row & 15) so that the per-lane row reads
// afterwards (lane = row) spread over all banks.
// qbar[h][d] = bf16(f32(f64 sum_t q[bs+t][h][d] / bl)), t ascending: the
// block rows of up to four query heads at a time go through LDS (the K-tile
// area, before the K rows are stored there) in chunks of 32 KiB, loaded
// while the K rows are in flight; thread (head slot tid / 64, pair l =
// tid % 64) then sums d = 2l and 2l + 1 row by row.
// dot(h, j) = sum_d qbar[h][d] * k[j][kv][d] in f64, d ascending (each product
// of two bf16 values is exact in f64, so fma gives the same sums).
// Dot products of one candidate's K row (LDS, chunk c at c ^ sw) with GW
// query heads' qbar (f64, [head][d]); heads gn..GW-1 read the padding of qbar
// and are not folded in.
template <int GW>
__device__ __forceinline__ void score_group(const uint8_t* krow, int sw, const double* qq, int gn, float& best,
                                            double& part) {
  double acc[GW];
#pragma unroll
  for (int u = 0; u < GW; ++u) acc[u] = 0.0;
#pragma unroll 2
  for (int cl = 0; cl < 16; ++cl) {
    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(krow + ((cl ^ sw) << 4));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const double k0 = (double)bf16_val(x[w] & 0xffffu), k1 = (double)bf16_val(x[w] >> 16);
#pragma unroll
      for (int u = 0; u < GW; ++u) {
        acc[u] = __builtin_fma(qq[u * SHD + 8 * cl + 2 * w], k0, acc[u]);
        acc[u] = __builtin_fma(qq[u * SHD + 8 * cl + 2 * w + 1], k1, acc[u]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    if (u < gn) {
      best = fmaxf(best, bf16_val(f64_to_bf16_bits_2step(acc[u])));
      part += acc[u];
    }
  }
}

// G1: the launch has one query head per KV head (a separate instantiation,
// so that the register allocation of the single-head path is its own).
template <bool G1>
__global__ __launch_bounds__(256) void score_kernel(SelArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* kt = lds;
  const int cpw = a.score_cpw;
  double* qs = reinterpret_cast<double*>(lds + cpw * 256);
  const int jid = blockIdx.z;
  const int kv = blockIdx.y;
  const Job jb = load_job(a, jid);
  const int c0 = blockIdx.x * cpw;
  if (c0 >= jb.kc) return;
  const int g = G1 ? 1 : a.g;
  const int tid = threadIdx.x;
  const int rsub = tid >> 4, ch = tid & 15;
  u32x4_t rows[kScoreCandsMax / 16];
#pragma unroll
  for (int p = 0; p < kScoreCandsMax / 16; ++p) {
    if (16 * p >= cpw) break;  // uniform
    const int c = c0 + 16 * p + rsub;
    const int64_t row = (int64_t)jb.row0 + cand_row(jb, min(c, jb.kc - 1));
    rows[p] = ld128(a.k + row * a.k_stride + (int64_t)kv * SHD + ch * 8);
  }
  {
    uint32_t* stage = reinterpret_cast<uint32_t*>(kt);  // [row][head of the pass][64 words]
    const int hs = tid >> 6, l = tid & 63;
    const uint16_t* qblk = a.q + ((int64_t)jb.row0 + jb.bs) * a.q_stride + (int64_t)kv * g * SHD;
    if (a.q_dma && ((int64_t)g * jb.bl + 3) / 4 * 4 <= cpw) {  // (then g * bl * 16 <= 304 * 16 fits an int)
      // The whole block fits the K-tile area: all its rows arrive at once by
      // buffer DMA, [head][row][16 chunks] (instruction j of wave j % 4 fills
      // 1 KiB = 64 pieces; pieces past the block read as zero), and the heads
      // are summed in rounds of four from LDS.
      const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
      const uint32_t qS = (uint32_t)(a.q_stride * 2);
      const uint32_t qbytes = (uint32_t)(jb.bl - 1) * qS + (uint32_t)(g * SHD * 2);
      const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qblk, qbytes);
      const int n_pieces = g * jb.bl * 16;
      for (int j = wave; j * 64 < n_pieces; j += 4) {
        const int i = j * 64 + l;
        const int hr = i >> 4, h = hr / jb.bl, r = hr - h * jb.bl;
        const uint32_t off = i < n_pieces ? (uint32_t)r * qS + (uint32_t)((h * SHD + (i & 15) * 8) * 2) : qbytes;
        dma16(qrs, kt + j * 1024, off);
      }
      vm_wait<0>();
      __syncthreads();
      for (int h = hs; h < g; h += 4) {
        const uint32_t* sp = stage + h * jb.bl * 64 + l;
        double s0 = 0.0, s1 = 0.0;
        int r = 0;
        for (; r + 16 <= jb.bl; r += 16) {
          uint32_t w[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) w[u] = sp[(r + u) * 64];
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            s0 += (double)bf16_val(w[u] & 0xffffu);
            s1 += (double)bf16_val(w[u] >> 16);
          }
        }
        for (; r < jb.bl; ++r) {
          const uint32_t w = sp[r * 64];
          s0 += (double)bf16_val(w & 0xffffu);
          s1 += (double)bf16_val(w >> 16);
        }
        qs[h * SHD + 2 * l] = (double)bf16_val(f64_to_bf16_bits_2step(s0 / (double)jb.bl));
        qs[h * SHD + 2 * l + 1] = (double)bf16_val(f64_to_bf16_bits_2step(s1 / (double)jb.bl));
      }
    } else {
      for (int h0 = 0; h0 < g; h0 += 4) {
        const int hp = min(4, g - h0);             // heads of this pass
        const int rows_per = kQbarStage / (hp * 256);  // block rows per chunk
        double s0 = 0.0, s1 = 0.0;
        for (int t0 = 0; t0 < jb.bl; t0 += rows_per) {
          const int n = min(rows_per, jb.bl - t0);
          const int items = n * hp * 16;  // 16-byte pieces of the chunk
          u32x4_t qv[kQbarStage / (256 * 16)];
#pragma unroll
          for (int u = 0; u < kQbarStage / (256 * 16); ++u) {
            const int i = u * 256 + tid;
            if (i < items) {
              const int r = i / (hp * 16), rem = i - r * (hp * 16);
              qv[u] = ld128(qblk + (int64_t)(t0 + r) * a.q_stride + (h0 + (rem >> 4)) * SHD + (rem & 15) * 8);
            }
          }
          __syncthreads();  // the previous chunk is summed (and the first: nothing reads the area yet)
#pragma unroll
          for (int u = 0; u < kQbarStage / (256 * 16); ++u) {
            const int i = u * 256 + tid;
            if (i < items) *reinterpret_cast<u32x4_t*>(stage + i * 4) = qv[u];
          }
          __syncthreads();
          if (hs < hp) {
            // 16 rows' words read together, then added in row order
            const uint32_t* sp = stage + hs * 64 + l;
            int r = 0;
            for (; r + 16 <= n; r += 16) {
              uint32_t w[16];
#pragma unroll
              for (int u = 0; u < 16; ++u) w[u] = sp[(r + u) * hp * 64];
#pragma unroll
              for (int u = 0; u < 16; ++u) {
                s0 += (double)bf16_val(w[u] & 0xffffu);
                s1 += (double)bf16_val(w[u] >> 16);
              }
            }
            for (; r < n; ++r) {
              const uint32_t w = sp[r * hp * 64];
              s0 += (double)bf16_val(w & 0xffffu);
              s1 += (double)bf16_val(w >> 16);
            }
          }
        }
        if (hs < hp) {
          qs[(h0 + hs) * SHD + 2 * l] = (double)bf16_val(f64_to_bf16_bits_2step(s0 / (double)jb.bl));
          qs[(h0 + hs) * SHD + 2 * l + 1] = (double)bf16_val(f64_to_bf16_bits_2step(s1 / (double)jb.bl));
        }
      }
    }
    __syncthreads();  // the stage area becomes the K tile
  }
#pragma unroll
  for (int p = 0; p < kScoreCandsMax / 16; ++p) {
    if (16 * p >= cpw) break;
    const int r = 16 * p + rsub;
    *reinterpret_cast<u32x4_t*>(kt + r * 256 + ((ch ^ (r & 15)) << 4)) = rows[p];
  }
  __syncthreads();
  if constexpr (G1) {
    // thread tid scores candidate tid and, in a workgroup of more than 256,
    // candidate tid + 256: a wavefront with any second candidate runs the two
    // dependent f64 chains interleaved (each still d ascending; lanes without
    // a second candidate run a discarded copy on a valid row).  Lane reads row
    // r at physical chunk cl ^ (r & 15): the 16 lanes of a read group hit 16
    // different chunks.
    const int cb = tid + 256;
    const bool has_a = c0 + tid < jb.kc;
    const bool has_b = cb < cpw && c0 + cb < jb.kc;
    const uint8_t* ka = kt + tid * 256;
    const int swa = tid & 15;
    double acc_a = 0.0, acc_b = 0.0;
    if (__builtin_amdgcn_ballot_w64(has_b)) {
      const int rb = min(cb, cpw - 1);
      const uint8_t* kb = kt + rb * 256;
      const int swb = rb & 15;
#pragma unroll 4
      for (int cl = 0; cl < 16; ++cl) {
        const u32x4_t xa = *reinterpret_cast<const u32x4_t*>(ka + ((cl ^ swa) << 4));
        const u32x4_t xb = *reinterpret_cast<const u32x4_t*>(kb + ((cl ^ swb) << 4));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const double q0 = qs[8 * cl + 2 * w], q1 = qs[8 * cl + 2 * w + 1];
          acc_a = __builtin_fma(q0, (double)bf16_val(xa[w] & 0xffffu), acc_a);
          acc_b = __builtin_fma(q0, (double)bf16_val(xb[w] & 0xffffu), acc_b);
          acc_a = __builtin_fma(q1, (double)bf16_val(xa[w] >> 16), acc_a);
          acc_b = __builtin_fma(q1, (double)bf16_val(xb[w] >> 16), acc_b);
        }
      }
    } else if (has_a) {
#pragma unroll 4
      for (int cl = 0; cl < 16; ++cl) {
        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(ka + ((cl ^ swa) << 4));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          acc_a = __builtin_fma(qs[8 * cl + 2 * w], (double)bf16_val(x[w] & 0xffffu), acc_a);
          acc_a = __builtin_fma(qs[8 * cl + 2 * w + 1], (double)bf16_val(x[w] >> 16), acc_a);
        }
      }
    }
    const int64_t out = ((int64_t)jid * a.Hkv + kv) * a.max_kc + c0 + tid;
    if (has_a) {
      if (jb.head_select)
        a.raw[out] = (uint16_t)(f64_to_bf16_bits_2step(acc_a));
      else
        a.part[out] = acc_a;
    }
    if (has_b) {
      if (jb.head_select)
        a.raw[out + 256] = (uint16_t)(f64_to_bf16_bits_2step(acc_b));
      else
        a.part[out + 256] = acc_b;
    }
    return;
  }
  // g > 1: thread tid scores candidates tid and tid + 256 (the latter when cpw > 256)
  for (int cl0 = tid; cl0 < cpw; cl0 += 256) {
  const int c = c0 + cl0;
  if (c >= jb.kc) return;
  // lane reads row cl0; physical chunk cl ^ (cl0 & 15) (the 16 lanes of a
  // read group hit 16 different chunks)
  const uint8_t* krow = kt + cl0 * 256;
  const int sw = cl0 & 15;
  const int64_t out = ((int64_t)jid * a.Hkv + kv) * a.max_kc + c;
  float best = -INFINITY;
  double part = 0.0;
  // GW query heads at a time (4, or 8 when g > 4), their dependent f64
  // chains interleaved (each head still sums d ascending) and every K element
  // converted once for the group; the heads of the group below g are folded
  // into best / part in ascending order
  if (g == 7) {  // Dream-7B's 28 / 4 heads: the exact group, no padded head
    score_group<7>(krow, sw, qs, 7, best, part);
  } else if (g > 4) {
    for (int g0 = 0; g0 < g; g0 += 8) score_group<8>(krow, sw, qs + g0 * SHD, min(8, g - g0), best, part);
  } else {
    score_group<4>(krow, sw, qs, g, best, part);
  }
  if (jb.head_select)
    a.raw[out] = (uint16_t)(__float_as_uint(best) >> 16);
  else
    a.part[out] = part;
  }
}

// ---- 2. top-k and copy ------------------------------------------------------------------
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
  int wave_tot2[2 * 16];
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
  const int incl = wave_incl_scan(own);
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

// The rank of key x among the first NR descending runs of 64 keys in `runs`:
// its lane in its own run plus, for each other run, the number of its keys
// that are larger.  The keys > x form a prefix of a run: its length is built
// from the bits 32 .. 1 (at most 63), then the last key decides 64; the NR
// searches advance in lockstep.
template <int NR>
__device__ __forceinline__ int rank_search(uint32_t x, const uint32_t* runs, int lane, int wave) {
  int cnt[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) cnt[r] = 0;
#pragma unroll
  for (int b = 32; b >= 1; b >>= 1)
#pragma unroll
    for (int r = 0; r < NR; ++r) cnt[r] += runs[r * 64 + cnt[r] + b - 1] > x ? b : 0;
  int rank = lane;
#pragma unroll
  for (int r = 0; r < NR; ++r) rank += r == wave ? 0 : cnt[r] + (runs[r * 64 + 63] > x ? 1 : 0);
  return rank;
}

// Rank of every key among up to 1024 unique 32-bit keys, one per thread
// (threads without a key hold 0, which ranks below every real key): each
// wavefront sorts its 64 keys descending with DPP / permlane moves (21
// stages), the sorted runs go to `runs` (1024 words of LDS), and
// rank_search counts, for every other run, its keys above the thread's.  The
// real keys are the first n_keys threads' (ceil(n_keys / 64) runs): the
// later runs hold only zeros and count nothing, so the search stops at the
// next multiple of four runs, and wavefronts without a real key return at
// once.  Returns the rank of the key the thread holds after the wave sort
// (its position in the descending order; meaningful only for a real key);
// *key receives that key.
__device__ int rank_sort_desc(uint32_t x, int n_keys, uint32_t* runs, uint32_t* key) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int kk = 2; kk <= 64; kk <<= 1) {
#pragma unroll
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      const uint32_t y = lane_xor(x, jj);
      const bool low = (lane & jj) == 0, desc = (lane & kk) == 0;
      x = (low == desc) ? max(x, y) : min(x, y);
    }
  }
  runs[threadIdx.x] = x;
  lds_barrier();  // global loads in flight (the copy's preloaded rows) stay in flight
  *key = x;
  constexpr int kRuns = kTopkThreads / 64;
  const int nruns = (n_keys + 63) >> 6;  // wave-uniform
  if (wave >= nruns) return 0;
  // the search covers the first NR runs, NR the multiple of four at or above
  // nruns (the runs between hold only zeros)
  if (nruns <= 4) return rank_search<4>(x, runs, lane, wave);
  if (nruns <= 8) return rank_search<8>(x, runs, lane, wave);
  if (nruns <= 12) return rank_search<12>(x, runs, lane, wave);
  return rank_search<kRuns>(x, runs, lane, wave);
}

constexpr int kLdsCand = 16384;  // candidates whose raw scores and order keys stay in LDS
constexpr int kRegSort = 1024;   // selected rows ranked one per thread (rank_sort_desc)

// bf16 bits of the raw score of candidate u before the division by sqrt(D): the
// stored group maximum (head_select), or bf16 of the KV heads' partial sums added
// in head order (token selection)
__device__ __forceinline__ uint16_t raw_bits(const SelArgs& a, const Job& jb, int jid, int h, int u) {
  if (jb.head_select) return a.raw[((int64_t)jid * a.Hkv + h) * a.max_kc + u];
  double t = 0.0;
  const double* p = a.part + (int64_t)jid * a.Hkv * a.max_kc + u;
  int kv = 0;
  for (; kv + 16 <= a.Hkv; kv += 16) {  // 16 loads in flight, added in head order
    double x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = p[(int64_t)(kv + i) * a.max_kc];
#pragma unroll
    for (int i = 0; i < 16; ++i) t += x[i];
  }
  for (; kv < a.Hkv; ++kv) t += p[(int64_t)kv * a.max_kc];
  return (uint16_t)f64_to_bf16_bits_2step(t);
}

// The copy of the selected rows of ranks [r0, r1) -- their KV-head-h pieces
// -- into their cache slots by the whole workgroup: item i = (rank r0 + i / 16,
// 16-byte chunk i % 16), eight items per thread in flight.  cand(r) gives the
// candidate of rank r.
template <typename CandFn>
__device__ __forceinline__ void copy_selected(const SelArgs& a, const Job& jb, int h, int r0, int r1, CandFn cand) {
  const int64_t row_elems = (int64_t)a.Hkv * SHD;
  const int n_items = (r1 - r0) * 16;
  constexpr int kPer = 8;
  for (int i0 = 0; i0 < n_items; i0 += kPer * kTopkThreads) {
    u32x4_t kx[kPer], vx[kPer];
    int64_t slot[kPer];
    int64_t e[kPer];
    // the source rows depend only on the ranks in LDS, the destinations on
    // the slot list: both loads are issued before either is waited for
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = i0 + u * kTopkThreads + (int)threadIdx.x;
      slot[u] = -1;
      if (i < n_items) {
        const int r = r0 + (i >> 4), chk = i & 15;
        const int j = cand(r);
        if (j >= 0 && j < jb.kc) {
          const int64_t row = (int64_t)jb.row0 + cand_row(jb, j);
          e[u] = (int64_t)h * SHD + chk * 8;
          kx[u] = ld128_stream(a.k + row * a.k_stride + e[u]);
          vx[u] = ld128_stream(a.v + row * a.v_stride + e[u]);
          slot[u] = a.slots[jb.slot_off + r];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if (slot[u] >= 0 && slot[u] < a.cache_slots) {
        st128(a.k_cache + slot[u] * row_elems + e[u], kx[u]);
        st128(a.v_cache + slot[u] * row_elems + e[u], vx[u]);
      }
  }
}

// grid (Hkv, n_job, n_part), block 1024.  Each of the n_part workgroups of
// (job, KV head) makes the selection and copies one contiguous share of the
// ranks (part 0 writes idx_out); token-selection jobs: every KV head's
// workgroups make the same selection (from the summed partial dots) and
// copy their own head's pieces, and only head 0 writes idx_out.  Beyond
// kLdsCand candidates (the sort then goes through the workspace, one buffer
// per (job, head)) part 0 alone selects and copies every rank.
// LDS: 128 KiB pool (small path: raw bits, order keys and 32-bit sort keys of
// up to kLdsCand candidates, then the selected candidates in rank order;
// large path: kSortCap 64-bit sort keys) + the shared scratch.
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(SelArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t pool[128 * 1024];
  __shared__ TopkShared sh;
  const int h = blockIdx.x;
  const int jid = blockIdx.y;
  const int part = blockIdx.z;
  const Job jb = load_job(a, jid);
  const int kc = jb.kc, nk = jb.n_keep;
  if (kc <= 0 || nk <= 0) return;
  if (part > 0 && kc > kLdsCand) return;
  const int tid = threadIdx.x;
  const int64_t base = ((int64_t)jid * a.Hkv + h) * a.max_kc;
  const int64_t sbase = ((int64_t)jid * a.Hkv + h) * a.max_keep;
  const int pk = jb.pool_k;
  const int pad = pk / 2;
  int64_t* io = a.idx_out && part == 0 && (jb.head_select || h == 0) ? a.idx_out + sbase : nullptr;
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
    // or after the division gives the same value) and the high-byte histogram.
    // When every candidate is kept (n_keep == kc) there is no threshold: the
    // sort keys go straight to position c, the compaction's index order.
    const bool keep_all = nk >= kc;
    for (int c = tid; c < kc; c += blockDim.x) {
      const int lo = pk > 1 ? max(0, c - pad) : c;
      const int hi = pk > 1 ? min(kc - 1, c - pad + pk - 1) : c;
      float m = -INFINITY;
      for (int u = lo; u <= hi; ++u) m = fmaxf(m, bf16_val(rawl[u]));
      const uint32_t key = bf16_order_key(f32_to_bf16_bits(m / a.sqrt_d));
      if (keep_all) {
        skey[c] = (key << 16) | (uint32_t)(0xffff - c);
      } else {
        okl[c] = (uint16_t)key;
        atomicAdd(&sh.hist[key >> 8], 1u);
      }
    }
    if (!keep_all) {
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
      // Index-order compaction (unique keys: score key, then the complement of
      // the candidate).  Thread t owns the E consecutive candidates from E t;
      // one scan gives the counts of better (> T) and tied (== T) candidates
      // before them, and a kept candidate goes to position
      // (better before it) + min(tied before it, need_eq).
      const int E = (kc + kTopkThreads - 1) / kTopkThreads;
      const int c0 = tid * E;
      int ngt = 0, neq = 0;
      for (int e = 0; e < E; ++e) {
        const int c = c0 + e;
        if (c < kc) {
          const uint32_t key = okl[c];
          ngt += key > T;
          neq += key == T;
        }
      }
      int gt_before, eq_before;
      block_exscan2(ngt, neq, sh.wave_tot2, &gt_before, &eq_before);
      for (int e = 0; e < E; ++e) {
        const int c = c0 + e;
        if (c >= kc) break;
        const uint32_t key = okl[c];
        const bool gt = key > T, eq = key == T;
        if (gt || (eq && eq_before < need_eq))
          skey[gt_before + min(eq_before, need_eq)] = (key << 16) | (uint32_t)(0xffff - c);
        gt_before += gt;
        eq_before += eq;
      }
    }
    int P2 = 1;
    while (P2 < nk) P2 <<= 1;
    __syncthreads();
    int32_t* selc = reinterpret_cast<int32_t*>(pool);  // rank -> candidate (raw bits / keys are dead)
    if (P2 <= kRegSort) {
      // Part p copies compaction positions [p0, p1) (each selected row once
      // over the parts).  Its first kPre items per thread are loaded before
      // the ranks are known, so that their latency overlaps the rank sort,
      // whose barriers wait on LDS only; a destination needs the row's rank
      // (rank_of, by candidate) and the rank's slot (slot_l).
      uint16_t* rank_of = reinterpret_cast<uint16_t*>(pool + 32 * 1024);  // the order keys are dead
      int32_t* slot_l = selc;                                              // the raw bits are dead
      const int p0 = (int)((int64_t)nk * part / a.n_part), p1 = (int)((int64_t)nk * (part + 1) / a.n_part);
      const int n_items = (p1 - p0) * 16;
      constexpr int kPre = 6;
      // the slot of rank tid (n_keep <= 1024 here), issued before the rows so
      // that waiting for it leaves the rows in flight
      const int32_t my_slot = tid < nk ? a.slots[jb.slot_off + tid] : -1;
      u32x4_t pk[kPre], pv[kPre];
      int pc[kPre];
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int i = u * kTopkThreads + tid;
        pc[u] = -1;
        if (i < n_items) {
          const int j = 0xffff - (int)(skey[p0 + (i >> 4)] & 0xffffu);
          const int64_t row = (int64_t)jb.row0 + cand_row(jb, j);
          const int64_t e = (int64_t)h * SHD + (i & 15) * 8;
          pk[u] = ld128_stream(a.k + row * a.k_stride + e);
          pv[u] = ld128_stream(a.v + row * a.v_stride + e);
          pc[u] = j;
        }
      }
      uint32_t x;
      const int rank = rank_sort_desc(tid < nk ? skey[tid] : 0u, nk, sh.chunk, &x);  // 0 ranks below every real key
      if (x != 0u) {  // exactly the nk real keys
        const int c = 0xffff - (int)(x & 0xffffu);
        rank_of[c] = (uint16_t)rank;
        if (io) io[rank] = c;
      }
      if (tid < nk) slot_l[tid] = my_slot;
      lds_barrier();
      const int64_t row_elems = (int64_t)a.Hkv * SHD;
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        if (pc[u] >= 0) {
          const int64_t slot = slot_l[rank_of[pc[u]]];
          const int64_t e = (int64_t)h * SHD + ((u * kTopkThreads + tid) & 15) * 8;
          if (slot >= 0 && slot < a.cache_slots) {
            st128(a.k_cache + slot * row_elems + e, pk[u]);
            st128(a.v_cache + slot * row_elems + e, pv[u]);
          }
        }
      }
      // the rest of the share, eight items per thread in flight
      constexpr int kPer = 8;
      for (int i0 = kPre * kTopkThreads; i0 < n_items; i0 += kPer * kTopkThreads) {
        u32x4_t kx[kPer], vx[kPer];
        int64_t slot[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int i = i0 + u * kTopkThreads + tid;
          slot[u] = -1;
          if (i < n_items) {
            const int j = 0xffff - (int)(skey[p0 + (i >> 4)] & 0xffffu);
            const int64_t row = (int64_t)jb.row0 + cand_row(jb, j);
            const int64_t e = (int64_t)h * SHD + (i & 15) * 8;
            kx[u] = ld128_stream(a.k + row * a.k_stride + e);
            vx[u] = ld128_stream(a.v + row * a.v_stride + e);
            slot[u] = slot_l[rank_of[j]];
          }
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int i = i0 + u * kTopkThreads + tid;
          if (slot[u] >= 0 && slot[u] < a.cache_slots) {
            const int64_t e = (int64_t)h * SHD + (i & 15) * 8;
            st128(a.k_cache + slot[u] * row_elems + e, kx[u]);
            st128(a.v_cache + slot[u] * row_elems + e, vx[u]);
          }
        }
      }
      return;
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
      // selc overlaps only the raw bits / order keys, skey lies behind them
      for (int r = tid; r < nk; r += blockDim.x) {
        const int c = 0xffff - (int)(skey[r] & 0xffffu);
        selc[r] = c;
        if (io) io[r] = c;
      }
    }
    __syncthreads();
    const int r0 = (int)((int64_t)nk * part / a.n_part), r1 = (int)((int64_t)nk * (part + 1) / a.n_part);
    copy_selected(a, jb, h, r0, r1, [&](int r) { return selc[r]; });
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
  __syncthreads();  // the workgroup's writes of so are visible to it
  copy_selected(a, jb, h, 0, nk, [&](int r) { return so[r]; });
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct SelLayout {
  size_t raw, part, okey, sel, ckey, cidx, total;
};

static SelLayout sel_layout(int n_job, int max_kc, int Hq, int Hkv) {
  SelLayout L;
  const size_t nj = (size_t)n_job, kc = (size_t)max_kc, hk = (size_t)Hkv;
  L.raw = align256(nj * hk * kc * 2);
  L.part = align256(nj * hk * kc * 8);
  L.okey = align256(nj * hk * kc * 2);
  L.sel = align256(nj * hk * kc * 4);  // max_keep <= max_kc
  const bool large = max_kc > kSortCap;
  L.ckey = large ? align256(nj * hk * kc * 2) : 0;
  L.cidx = large ? align256(nj * hk * kc * 4) : 0;
  L.total = L.raw + L.part + L.okey + L.sel + 2 * L.ckey + 2 * L.cidx;
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
  if ((int64_t)max_kc / kScoreCands + 1 >= ((int64_t)1 << 31) || n_job > 65535 || Hkv > 65535)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: %d jobs / %d candidates / %d KV heads exceed the grid", name, n_job, max_kc,
                Hkv);
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
  a.q_dma = n_rows <= ((((int64_t)1 << 32) - 1) / (q_stride_tok * 2)) ? 1 : 0;  // q_stride_tok >= Hq * D > 0 here
  a.jobs = jobs; a.n_job = n_job; a.max_kc = max_kc; a.max_keep = max_keep;
  a.Hq = Hq; a.Hkv = Hkv; a.g = Hq / Hkv;
  a.sqrt_d = sqrt_d;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slots = cache_slots;
  a.slots = slots; a.n_slots = n_slots; a.idx_out = idx_out;
  char* ws = reinterpret_cast<char*>(workspace);
  size_t o = 0;
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
  // Two score workgroups fit per CU (VGPRs, and LDS up to 80 KiB each): when
  // 256 candidates per workgroup need more than one such generation on the
  // 256 CUs and up to 304 fit in one, take the larger workgroups (4 x 1280
  // tokens, 32 KV heads: 640 -> 512 workgroups; the last 128 ran as a second
  // generation).
  // qbar of g heads as f64, padded to four heads (g <= 4) or to a multiple of eight (the dot products'
  // head groups)
  const size_t qs_bytes = (size_t)(a.g == 1 ? 1 : a.g > 4 ? (a.g + 7) / 8 * 8 : 4) * SHD * sizeof(double);
  const int64_t heads = (int64_t)Hkv * n_job;
  a.score_cpw = kScoreCands;
  {
    const int64_t n1 = (max_kc + kScoreCands - 1) / kScoreCands;
    const int64_t n2 = (max_kc + kScoreCandsMax - 1) / kScoreCandsMax;
    if (n1 * heads > 512 && n2 < n1 && n2 * heads <= 512) {
      const int cpw = (int)(((max_kc + n2 - 1) / n2 + 15) / 16 * 16);
      if ((size_t)cpw * 256 + qs_bytes <= 80 * 1024) a.score_cpw = cpw;
    }
  }
  const size_t score_lds = (size_t)a.score_cpw * 256 + qs_bytes;
  auto score = a.g == 1 ? score_kernel<true> : score_kernel<false>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(score), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)score_lds);
  if (e != hipSuccess) return fail(DLLM_ERR_HIP, "%s: hipFuncSetAttribute: %s", name, hipGetErrorString(e));
  score<<<dim3((unsigned)((max_kc + a.score_cpw - 1) / a.score_cpw), Hkv, n_job), dim3(256), score_lds, st>>>(a);
  int rc = check_launch(name);
  if (rc) return rc;
  // enough top-k workgroups to give every CU one (256 CUs), at most four per (job, KV head)
  const int64_t pairs = (int64_t)n_job * Hkv;
  a.n_part = (int)max((int64_t)1, min((int64_t)4, 256 / pairs));
  topk_kernel<<<dim3(Hkv, n_job, a.n_part), dim3(kTopkThreads), 0, st>>>(a);
  return check_launch(name);
}

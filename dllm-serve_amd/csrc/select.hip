// K5 / K6: per-KV-head (head_select) or shared (token) top-k selection of the
// non-block K/V rows of a sequence, fused with the KV-cache scatter.
//
// Three launches per call:
//   1. qbar_kernel    q-mean over the block rows          (n_job x Hq x 128)
//   2. score_kernel   raw bf16 scores per candidate        (n_job x n_sel x Kc)
//   3. topk_store_kernel  pool + scale + exact top-n_keep by bitonic sort in
//      LDS, then copies the selected K/V rows into their cache slots.
// The arithmetic follows a fixed, order-defined rule (sequential fp64 sums,
// explicit f32 / bf16 rounding points, ties to the lower candidate index) so
// the selected indices are reproducible bit for bit on the CPU.
#include "common.h"

#include <math.h>

namespace dllm {

constexpr int SHD = 128;         // the head dim these kernels handle
constexpr int MAX_KC = 8192;     // candidates per sequence handled in LDS
constexpr int TOPK_THREADS = 1024;

struct SelArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, k_stride, v_stride;
  const int32_t* jobs;  // [n_job][6]
  int n_job, max_kc, max_keep;
  int Hq, Hkv, g, head_select, pool_k;
  float sqrt_d;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t cache_slots;
  const int32_t* slots;
  int64_t* idx_out;
  uint16_t* qbar;    // [n_job][Hq][128] bf16 bits
  uint16_t* scores;  // [n_job][n_sel][max_kc] bf16 bits
};

struct Job {
  int row0, n_tok, bs, bl, n_keep, slot_off;
};

__device__ __forceinline__ Job load_job(const int32_t* jobs, int j) {
  const int32_t* p = jobs + 6 * j;
  return Job{p[0], p[1], p[2], p[3], p[4], p[5]};
}

// Candidate j (prefix rows, then suffix rows) -> row offset inside the sequence.
__device__ __forceinline__ int cand_row(const Job& jb, int j) { return j < jb.bs ? j : j + jb.bl; }

// f64 -> f32 (round to nearest even) -> bf16 (round to nearest even)
__device__ __forceinline__ uint32_t f64_to_bf16_bits(double x) { return f64_to_bf16_bits_2step(x); }

// grid (n_job, Hq), block 128: qbar[h][d] = bf16(f32(sum_t q[bs+t][h][d] / bl))
__global__ __launch_bounds__(128) void qbar_kernel(SelArgs a) {
  const int jid = blockIdx.x;
  const int h = blockIdx.y;
  const int d = threadIdx.x;
  const Job jb = load_job(a.jobs, jid);
  double sum = 0.0;
  const uint16_t* qp = a.q + (int64_t)(jb.row0 + jb.bs) * a.q_stride + h * SHD + d;
  for (int t = 0; t < jb.bl; ++t) sum += (double)bf16_bits_to_f32(qp[(int64_t)t * a.q_stride]);
  const double mean = jb.bl > 0 ? sum / (double)jb.bl : 0.0;
  a.qbar[((int64_t)jid * a.Hq + h) * SHD + d] = (uint16_t)f64_to_bf16_bits(mean);
}

// grid (ceil(max_kc/256), n_sel, n_job), block 256: one candidate per thread.
__global__ __launch_bounds__(256) void score_kernel(SelArgs a) {
  extern __shared__ float qs[];  // qbar of the heads this block needs, as f32
  const int jid = blockIdx.z;
  const int hs = blockIdx.y;
  const Job jb = load_job(a.jobs, jid);
  const int Kc = jb.n_tok - jb.bl;
  const int nh = a.head_select ? a.g : a.Hq;  // query heads feeding this selection head
  const int h0 = a.head_select ? hs * a.g : 0;
  const uint16_t* qb = a.qbar + ((int64_t)jid * a.Hq + h0) * SHD;
  for (int i = threadIdx.x; i < nh * SHD; i += blockDim.x) qs[i] = bf16_bits_to_f32(qb[i]);
  __syncthreads();
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= Kc) return;
  const uint16_t* krow = a.k + (int64_t)(jb.row0 + cand_row(jb, j)) * a.k_stride;
  float best = -INFINITY;
  if (a.head_select) {
    const uint16_t* kp = krow + hs * SHD;
    for (int gi = 0; gi < nh; ++gi) {
      const float* qq = qs + gi * SHD;
      double acc = 0.0;
      for (int c = 0; c < SHD / 8; ++c) {
        const u32x4_t kv = ld128(kp + c * 8);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          acc += (double)qq[c * 8 + 2 * w] * (double)bf16_bits_to_f32(kv[w] & 0xffffu);
          acc += (double)qq[c * 8 + 2 * w + 1] * (double)bf16_bits_to_f32(kv[w] >> 16);
        }
      }
      best = fmaxf(best, bf16_bits_to_f32(f64_to_bf16_bits(acc)));
    }
  } else {
    double acc = 0.0;
    for (int h = 0; h < nh; ++h) {
      const uint16_t* kp = krow + (h / a.g) * SHD;
      const float* qq = qs + h * SHD;
      for (int c = 0; c < SHD / 8; ++c) {
        const u32x4_t kv = ld128(kp + c * 8);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          acc += (double)qq[c * 8 + 2 * w] * (double)bf16_bits_to_f32(kv[w] & 0xffffu);
          acc += (double)qq[c * 8 + 2 * w + 1] * (double)bf16_bits_to_f32(kv[w] >> 16);
        }
      }
    }
    best = bf16_bits_to_f32(f64_to_bf16_bits(acc));
  }
  a.scores[((int64_t)jid * gridDim.y + hs) * a.max_kc + j] = (uint16_t)(__float_as_uint(best) >> 16);
}

// Order-preserving map of a bf16 pattern to an unsigned 16-bit key (-0 == +0).
__device__ __forceinline__ uint32_t bf16_order_key(uint32_t b) {
  if (b == 0x8000u) b = 0u;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

// grid (n_sel, n_job), block 1024.
__global__ __launch_bounds__(TOPK_THREADS) void topk_store_kernel(SelArgs a) {
  __shared__ uint32_t keys[MAX_KC];
  __shared__ float sc[MAX_KC];
  const int hs = blockIdx.x;
  const int n_sel = gridDim.x;
  const int jid = blockIdx.y;
  const Job jb = load_job(a.jobs, jid);
  const int Kc = jb.n_tok - jb.bl;
  if (Kc <= 0 || jb.n_keep <= 0) return;
  const int tid = threadIdx.x;
  const uint16_t* raw = a.scores + ((int64_t)jid * n_sel + hs) * a.max_kc;
  for (int j = tid; j < Kc; j += TOPK_THREADS) sc[j] = bf16_bits_to_f32(raw[j]);
  int P2 = 1;
  while (P2 < Kc) P2 <<= 1;
  __syncthreads();
  const int pk = a.pool_k;
  const int pad = pk / 2;
  for (int j = tid; j < P2; j += TOPK_THREADS) {
    uint32_t key = 0u;  // below every real key
    if (j < Kc) {
      float m = sc[j];
      if (pk > 1) {
        const int lo = max(0, j - pad);
        const int hi = min(Kc - 1, j - pad + pk - 1);
        m = -INFINITY;
        for (int u = lo; u <= hi; ++u) m = fmaxf(m, sc[u]);
      }
      const uint32_t sb = f32_to_bf16_bits(m / a.sqrt_d);
      key = (bf16_order_key(sb) << 16) | (uint32_t)(0xffff - j);
    }
    keys[j] = key;
  }
  __syncthreads();
  // Bitonic sort, descending.  Keys are unique, so the order is total.
  for (int kk = 2; kk <= P2; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int i = tid; i < P2; i += TOPK_THREADS) {
        const int ixj = i ^ jj;
        if (ixj > i) {
          const uint32_t x = keys[i], y = keys[ixj];
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
  const int n_keep = jb.n_keep;
  if (a.idx_out) {
    int64_t* io = a.idx_out + ((int64_t)jid * n_sel + hs) * a.max_keep;
    for (int r = tid; r < n_keep; r += TOPK_THREADS) io[r] = 0xffff - (int)(keys[r] & 0xffffu);
  }
  // Copy selected rows into their cache slots (16 bytes per thread).
  const int row_elems = a.Hkv * SHD;
  const int heads = a.head_select ? 1 : a.Hkv;     // heads copied per selected row
  const int h_first = a.head_select ? hs : 0;
  const int chunks = heads * (SHD / 8);
  const int64_t total = (int64_t)n_keep * chunks;
  for (int64_t c = tid; c < total; c += TOPK_THREADS) {
    const int r = (int)(c / chunks);
    const int e = (int)(c - (int64_t)r * chunks) * 8 + h_first * SHD;
    const int64_t slot = a.slots[jb.slot_off + r];
    if (slot < 0 || slot >= a.cache_slots) continue;
    const int j = 0xffff - (int)(keys[r] & 0xffffu);
    const int64_t row = jb.row0 + cand_row(jb, j);
    st128(a.k_cache + slot * row_elems + e, ld128(a.k + row * a.k_stride + e));
    st128(a.v_cache + slot * row_elems + e, ld128(a.v + row * a.v_stride + e));
  }
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace dllm

using namespace dllm;

extern "C" size_t dllm_select_kv_workspace_size(int n_job, int max_kc, int Hq, int Hkv, int D, int head_select) {
  (void)D;
  if (n_job <= 0 || max_kc <= 0 || Hq <= 0 || Hkv <= 0) return 0;
  const int n_sel = head_select ? Hkv : 1;
  return align256((size_t)n_job * Hq * SHD * 2) + align256((size_t)n_job * n_sel * max_kc * 2);
}

extern "C" int dllm_select_kv_store(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v,
                                    int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                                    const int32_t* jobs, int n_job, int max_kc, int max_keep, int max_blk,
                                    int Hq, int Hkv, int D, int head_select, int pool_k, float sqrt_d,
                                    dllm_bf16* k_cache, dllm_bf16* v_cache, int64_t cache_slots,
                                    const int32_t* slots, int64_t* idx_out, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  const char* name = "dllm_select_kv_store";
  (void)max_blk;
  set_error("");
  if (D != SHD) return fail(DLLM_ERR_UNSUPPORTED, "%s: head_dim %d not supported (the kernels handle 128)", name, D);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv) return fail(DLLM_ERR_INVALID_ARG, "%s: Hq=%d / Hkv=%d", name, Hq, Hkv);
  if (n_job < 0 || max_kc < 0 || max_keep < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (n_job == 0 || max_kc == 0 || max_keep == 0) return DLLM_OK;
  if (max_kc > MAX_KC) return fail(DLLM_ERR_UNSUPPORTED, "%s: %d candidates exceed %d", name, max_kc, MAX_KC);
  if (max_keep > max_kc) return fail(DLLM_ERR_INVALID_ARG, "%s: max_keep %d > max_kc %d", name, max_keep, max_kc);
  if (!q || !k || !v || !jobs || !k_cache || !v_cache || !slots)
    return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!aligned16(k) || !aligned16(v) || !aligned16(k_cache) || !aligned16(v_cache) || k_stride_tok % 8 ||
      v_stride_tok % 8)
    return fail(DLLM_ERR_INVALID_ARG, "%s: k/v/caches must be 16-byte aligned with strides multiple of 8", name);
  if (!(sqrt_d > 0.f)) return fail(DLLM_ERR_INVALID_ARG, "%s: sqrt_d must be positive", name);
  const size_t need = dllm_select_kv_workspace_size(n_job, max_kc, Hq, Hkv, D, head_select);
  if (!workspace || workspace_bytes < need)
    return fail(DLLM_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", name, need,
                workspace ? workspace_bytes : (size_t)0);
  SelArgs a = {};
  a.q = q; a.k = k; a.v = v;
  a.q_stride = q_stride_tok; a.k_stride = k_stride_tok; a.v_stride = v_stride_tok;
  a.jobs = jobs; a.n_job = n_job; a.max_kc = max_kc; a.max_keep = max_keep;
  a.Hq = Hq; a.Hkv = Hkv; a.g = Hq / Hkv; a.head_select = head_select ? 1 : 0; a.pool_k = pool_k;
  a.sqrt_d = sqrt_d;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slots = cache_slots; a.slots = slots; a.idx_out = idx_out;
  char* ws = reinterpret_cast<char*>(workspace);
  a.qbar = reinterpret_cast<uint16_t*>(ws);
  a.scores = reinterpret_cast<uint16_t*>(ws + align256((size_t)n_job * Hq * SHD * 2));
  const int n_sel = a.head_select ? Hkv : 1;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  qbar_kernel<<<dim3(n_job, Hq), dim3(128), 0, st>>>(a);
  int rc = check_launch(name);
  if (rc) return rc;
  const int nh = a.head_select ? a.g : Hq;
  const size_t lds = (size_t)nh * SHD * sizeof(float);
  if (lds > 64 * 1024) return fail(DLLM_ERR_UNSUPPORTED, "%s: %d query heads per selection head too many", name, nh);
  score_kernel<<<dim3((max_kc + 255) / 256, n_sel, n_job), dim3(256), lds, st>>>(a);
  if ((rc = check_launch(name))) return rc;
  topk_store_kernel<<<dim3(n_sel, n_job), dim3(TOPK_THREADS), 0, st>>>(a);
  return check_launch(name);
}

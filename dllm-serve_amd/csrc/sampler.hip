// K8 / K9: the low-confidence remasking sampler of the diffusion runner.
//
// K8 (smx_row_kernel) reduces each row of bf16 logits
// [M, V] to what `x0_p, x0 = torch.max(F.softmax(logits, -1), -1)` returns
// (dllmserve/engine/model_runner.py:862-863,886-887):
//   m  = max_j l_j,  s = sum_j exp(l_j - m)                      (f32)
//   P_j = bf16(exp(l_j - m) / s)                                  (the bf16 probabilities)
//   x0_p = max_j P_j = bf16(1 / s),  x0 = min { j : P_j == x0_p }
// in one read of the logits.  A probability can only round to x0_p when its
// logit is within 2^-6 of m, and bf16 logits below m are that close to it
// only when |m| <= 2; so x0 is the first index of the maximal logit unless
// |m| <= 2, in which case the columns before that index are rescanned for an
// earlier one whose rounded probability ties.
//
// Layout: one workgroup per row (1024 threads when there are at most 512
// rows, else 256); each thread streams every NT-th 16-byte chunk with four
// loads in flight and keeps a record {m, s, first index of m}; the records
// are merged across the workgroup and one wavefront finishes the row (the
// tie rescan included).  HBM-bound: 2 V bytes per row, read once.
//
// With a per-row temperature T > 0 the row is first transformed as the
// reference's add_gumbel_noise does (model_runner.py:592-600):
//   v_j = bf16(exp(f64 l_j) / (-log u_j)^T),   u_j uniform in [0, 1) (f64)
// and the softmax-max runs over v.  u_j comes from a counter-based generator
// (SplitMix64 of seed + (c + 1) * 0x9E3779B97F4A7C15, c = (row_base + row) *
// V + j, top 53 bits), so a row's draws do not depend on how rows are
// grouped into launches; torch's own generator stream is not reproduced.
//
// K9 (lowconf_unmask_kernel) is the per-sequence unmasking step that follows
// (model_runner.py:895-949): in the sequence's window of token positions,
// count the masked ones, unmask k = min(ceil(nmask / steps_remain), nmask) of
// them -- the window's first position first when the first-token rule
// applies -- and the rest in order of confidence (descending, ties to the
// lower position, which is the set torch.topk returns).  One workgroup per
// sequence; the k-th largest (confidence, position) key is found by a
// bitwise search over keys held in LDS.
#include "common.h"

#include <limits.h>

namespace dllm {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kUnmaskMaxWin = 8192;  // SamplingParams caps gen_length at 8192

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Merge partial (m2, s2, i2) into (m, s, i).  An empty partial is
// (-inf, 0, INT_MAX).  Symmetric, so butterfly reductions agree on all lanes.
__device__ __forceinline__ void smx_merge(float& m, float& s, int& i, float m2, float s2, int i2) {
  const float mn = fmaxf(m, m2);
  const float a = (m == mn) ? s : s * fexp2((m - mn) * kLog2e);
  const float b = (m2 == mn) ? s2 : s2 * fexp2((m2 - mn) * kLog2e);
  i = (m > m2) ? i : (m2 > m) ? i2 : min(i, i2);
  s = a + b;
  m = mn;
}

__device__ __forceinline__ void smx_wave_reduce(float& m, float& s, int& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __uint_as_float(lane_xor(__float_as_uint(m), off));
    const float s2 = __uint_as_float(lane_xor(__float_as_uint(s), off));
    const int i2 = (int)lane_xor((uint32_t)i, off);
    smx_merge(m, s, i, m2, s2, i2);
  }
}

__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t c) {
  uint64_t z = seed + (c + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// exp(l) / (-log u)^T in f64, rounded to f32 and then to bf16 (the value the
// reference stores back into its bf16 logits), returned as f32.
__device__ __forceinline__ float gumbel_value(float l, double T, uint64_t seed, uint64_t c) {
  const double u = (double)(splitmix64_at(seed, c) >> 11) * 0x1.0p-53;
  const double nl = -log(u);
  const double g = T == 1.0 ? nl : pow(nl, T);
  const double v = exp((double)l) / g;
  return bf16_bits_to_f32(f64_to_bf16_bits_2step(v));
}

// Fold 8 logits (one 16-byte chunk starting at column e0) into the running
// (m, s, i).  A thread's chunks arrive in increasing column order, so a tie
// with the running max keeps the earlier index.
template <bool GUMBEL>
__device__ __forceinline__ void smx_chunk(u32x4_t v, int e0, float& m, float& s, int& i, double T = 0.0,
                                          uint64_t seed = 0, uint64_t c0 = 0) {
  float f[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    f[2 * w] = __uint_as_float(v[w] << 16);
    f[2 * w + 1] = __uint_as_float(v[w] & 0xffff0000u);
  }
  if (GUMBEL) {
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = gumbel_value(f[k], T, seed, c0 + (uint64_t)k);
  }
  const float cm = fmaxf(fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3])), fmaxf(fmaxf(f[4], f[5]), fmaxf(f[6], f[7])));
  if (cm > m) {
    int k = 7;
#pragma unroll
    for (int kk = 6; kk >= 0; --kk)
      if (f[kk] == cm) k = kk;
    s *= fexp2((m - cm) * kLog2e);
    m = cm;
    i = e0 + k;
  }
  if (m != -INFINITY) {
    float e[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) e[k] = fexp2((f[k] - m) * kLog2e);
    s += ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
  }
}

struct SmxArgs {
  const uint16_t* logits;
  int64_t ld;       // elements between rows
  int M;
  int V;
  int chunks;       // V / 8
  int64_t* x0;
  uint16_t* x0p;
  const double* temp;  // per-row temperature (nullable: no transform)
  uint64_t seed;
  int64_t row_base;
};

// Fold columns [8 c0, 8 c1) of one row into the thread's running (m, s, i):
// thread t takes chunks c0 + t, c0 + t + NT, ..., four 16-byte loads in flight.
template <bool GUMBEL, int NT>
__device__ __forceinline__ void smx_scan(const SmxArgs& a, int row, int c0, int c1, float& m, float& s, int& idx) {
  const uint16_t* base = a.logits + (int64_t)row * a.ld;
  const u32x4_t ninf = {0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u};
  const double T = GUMBEL ? a.temp[row] : 0.0;
  const uint64_t rc = GUMBEL ? (uint64_t)(a.row_base + row) * (uint64_t)a.V : 0;
  for (int c = c0 + (int)threadIdx.x; c < c1; c += 4 * NT) {
    u32x4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int cc = c + u * NT;
      v[u] = cc < c1 ? ld128_stream(base + 8 * (int64_t)cc) : ninf;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e0 = 8 * (c + u * NT);
      if (GUMBEL && T > 0.0 && c + u * NT < c1)  // padding chunks stay -inf
        smx_chunk<true>(v[u], e0, m, s, idx, T, a.seed, rc + (uint64_t)e0);
      else
        smx_chunk<false>(v[u], e0, m, s, idx);
    }
  }
}

// Merge the workgroup's per-thread records; every thread returns the result.
template <int NT>
__device__ __forceinline__ void smx_block_reduce(float& m, float& s, int& idx) {
  __shared__ float red_m[NT / 64];
  __shared__ float red_s[NT / 64];
  __shared__ int red_i[NT / 64];
  smx_wave_reduce(m, s, idx);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
    red_i[wave] = idx;
  }
  __syncthreads();
  m = -INFINITY;
  s = 0.f;
  idx = INT_MAX;
  if (lane < NT / 64) {
    m = red_m[lane];
    s = red_s[lane];
    idx = red_i[lane];
  }
  smx_wave_reduce(m, s, idx);
}

// x0 / x0_p of one row from its merged (m, s, first index of m), by one
// wavefront: the probability of the maximum is bf16(1/s); when |m| <= 2 an
// earlier column may round to the same probability, so the columns before
// the first maximum are rescanned for the earliest such one.
__device__ void smx_finish(const SmxArgs& a, int row, float m, float s, int idx) {
  const int lane = threadIdx.x & 63;
  const uint32_t P = f32_to_bf16_bits(1.0f / s);
  int best = idx;
  if (fabsf(m) <= 2.0f && idx != INT_MAX && idx > 0) {
    // earliest column j < idx with bf16(exp(v_j - m) / s) == P
    const uint16_t* base = a.logits + (int64_t)row * a.ld;
    const float thr = m - 0.015625f;
    int found = INT_MAX;
    const int nch = (idx + 7) >> 3;
    const double T = a.temp ? a.temp[row] : 0.0;
    const uint64_t rc = (uint64_t)(a.row_base + row) * (uint64_t)a.V;
    for (int c = lane; c < nch; c += 64) {
      const u32x4_t v = ld128(base + 8 * (int64_t)c);
#pragma unroll
      for (int k = 7; k >= 0; --k) {
        const uint32_t w = v[k >> 1];
        float f = (k & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
        if (T > 0.0) f = gumbel_value(f, T, a.seed, rc + (uint64_t)(8 * c + k));
        const int j = 8 * c + k;
        if (j < idx && f >= thr && f32_to_bf16_bits(expf(f - m) / s) == P) found = min(found, j);
      }
    }
    found = min(found, (int)lane_xor((uint32_t)found, 32));
    found = min(found, (int)lane_xor((uint32_t)found, 16));
    found = min(found, (int)lane_xor((uint32_t)found, 8));
    found = min(found, (int)lane_xor((uint32_t)found, 4));
    found = min(found, (int)lane_xor((uint32_t)found, 2));
    found = min(found, (int)lane_xor((uint32_t)found, 1));
    best = min(best, found);
  }
  if (lane == 0) {
    a.x0[row] = best == INT_MAX ? 0 : best;
    a.x0p[row] = (uint16_t)P;
  }
}

// One workgroup per row: scan, merge and finish in one launch.
template <bool GUMBEL, int NT>
__global__ __launch_bounds__(NT) void smx_row_kernel(SmxArgs a) {
  const int row = blockIdx.x;
  float m = -INFINITY, s = 0.f;
  int idx = INT_MAX;
  smx_scan<GUMBEL, NT>(a, row, 0, a.chunks, m, s, idx);
  smx_block_reduce<NT>(m, s, idx);
  if ((threadIdx.x >> 6) == 0) smx_finish(a, row, m, s, idx);
}

// ---- K9 ---------------------------------------------------------------------

struct UnmaskArgs {
  int64_t* tokens;
  int64_t n_tokens;       // elements of tokens (bounds guard)
  const int32_t* params;  // [n_seq][5]: tok_off, win_len, row_off, steps_remain, first_rule
  const int64_t* x0;
  const uint16_t* conf;
  int64_t n_rows;         // rows of x0 / conf (bounds guard)
  int64_t mask_id;
  int max_win;
  int32_t* n_unmasked;    // nullable
};

// Order-preserving map of bf16 bits to 16-bit unsigned (-0 equals +0).
__device__ __forceinline__ uint32_t conf_order(uint32_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

__device__ __forceinline__ int block_sum(int v, int* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += (int)lane_xor((uint32_t)v, off);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void lowconf_unmask_kernel(UnmaskArgs a) {
  __shared__ uint32_t keys[kUnmaskMaxWin];
  __shared__ int red[4];
  const int b = blockIdx.x;
  const int32_t* p = a.params + 5 * (int64_t)b;
  const int64_t tok_off = p[0];
  const int n = min(min(p[1], a.max_win), kUnmaskMaxWin);
  const int64_t r0 = p[2];
  const int sr = p[3];
  const bool first_rule = p[4] != 0;
  const int tid = threadIdx.x;
  const bool valid = n > 0 && tok_off >= 0 && tok_off + n <= a.n_tokens && r0 >= 0 && r0 + n <= a.n_rows;
  if (!valid) {  // uniform per workgroup
    if (a.n_unmasked && tid == 0) a.n_unmasked[b] = 0;
    return;
  }
  int64_t* tok = a.tokens + tok_off;
  int cnt = 0;
  for (int j = tid; j < n; j += 256) {
    const bool masked = tok[j] == a.mask_id;
    keys[j] = masked ? ((conf_order(a.conf[r0 + j]) << 16) | (0xffffu - (uint32_t)j)) : 0u;
    cnt += masked;
  }
  const int nmask = block_sum(cnt, red);  // its barriers also publish keys[]
  // steps_remain <= 0: nothing is unmasked (the reference divides by it)
  int k = sr > 0 ? min((nmask + sr - 1) / sr, nmask) : 0;
  const int k_total = k;
  if (first_rule && k > 0 && keys[0] != 0u) {
    __syncthreads();  // every thread has read keys[0]
    if (tid == 0) {
      tok[0] = a.x0[r0];
      keys[0] = 0u;
    }
    --k;
    __syncthreads();
  }
  if (k > 0) {
    uint32_t T = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = T | (1u << bit);
      int c = 0;
      for (int j = tid; j < n; j += 256) c += keys[j] >= cand;
      if (block_sum(c, red) >= k) T = cand;
    }
    // keys are distinct and the k-th largest is non-zero: exactly k pass
    for (int j = tid; j < n; j += 256)
      if (keys[j] >= T) tok[j] = a.x0[r0 + j];
  }
  if (a.n_unmasked && tid == 0) a.n_unmasked[b] = k_total;
}

}  // namespace dllm

using namespace dllm;

extern "C" size_t dllm_softmax_max_workspace_size(int M, int V) {
  (void)M;
  (void)V;
  return 0;  // one workgroup per row: no partial records
}

static int softmax_max_launch(const char* name, const uint16_t* logits, int64_t ld, int M, int V,
                              const double* row_temperature, uint64_t seed, int64_t row_base, int64_t* x0,
                              uint16_t* x0_p, void* stream) {
  if (M < 0 || V < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (M == 0) return DLLM_OK;
  if (V == 0 || V % 8 != 0)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: vocabulary size %d must be a positive multiple of 8", name, V);
  if (!logits || !x0 || !x0_p) return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  if (!aligned16(logits) || ld % 8 != 0 || ld < V)
    return fail(DLLM_ERR_INVALID_ARG, "%s: logits must be 16-byte aligned with a row stride >= V and a multiple of 8",
                name);
  SmxArgs a;
  a.logits = logits;
  a.ld = ld;
  a.M = M;
  a.V = V;
  a.chunks = V / 8;
  a.x0 = x0;
  a.x0p = x0_p;
  a.temp = row_temperature;
  a.seed = seed;
  a.row_base = row_base;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)M);
  // few rows: 1024 threads per row keep enough loads in flight per CU
  if (M <= 512) {
    if (row_temperature)
      smx_row_kernel<true, 1024><<<grid, dim3(1024), 0, st>>>(a);
    else
      smx_row_kernel<false, 1024><<<grid, dim3(1024), 0, st>>>(a);
  } else {
    if (row_temperature)
      smx_row_kernel<true, 256><<<grid, dim3(256), 0, st>>>(a);
    else
      smx_row_kernel<false, 256><<<grid, dim3(256), 0, st>>>(a);
  }
  return check_launch(name);
}

extern "C" int dllm_softmax_max(const uint16_t* logits, int64_t ld, int M, int V, int64_t* x0, uint16_t* x0_p,
                                void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return softmax_max_launch("dllm_softmax_max", logits, ld, M, V, nullptr, 0, 0, x0, x0_p, stream);
}

extern "C" int dllm_softmax_max_sample(const uint16_t* logits, int64_t ld, int M, int V,
                                       const double* row_temperature, uint64_t seed, int64_t row_base, int64_t* x0,
                                       uint16_t* x0_p, void* workspace, size_t workspace_bytes, void* stream) {
  if (row_base < 0) return fail(DLLM_ERR_INVALID_ARG, "dllm_softmax_max_sample: negative row_base");
  (void)workspace;
  (void)workspace_bytes;
  return softmax_max_launch("dllm_softmax_max_sample", logits, ld, M, V, row_temperature, seed, row_base, x0, x0_p,
                            stream);
}

extern "C" int dllm_lowconf_unmask(int64_t* tokens, int64_t n_tokens, const int32_t* seq_params, int n_seq,
                                   int max_win, const int64_t* x0, const uint16_t* conf, int64_t n_rows,
                                   int64_t mask_id, int32_t* n_unmasked, void* stream) {
  static const char* name = "dllm_lowconf_unmask";
  if (n_seq < 0 || max_win < 0 || n_tokens < 0 || n_rows < 0)
    return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (n_seq == 0) return DLLM_OK;
  if (max_win > kUnmaskMaxWin)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: window of %d positions exceeds %d", name, max_win, kUnmaskMaxWin);
  if (!tokens || !seq_params || (n_rows > 0 && (!x0 || !conf)))
    return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  UnmaskArgs a;
  a.tokens = tokens;
  a.n_tokens = n_tokens;
  a.params = seq_params;
  a.x0 = x0;
  a.conf = conf;
  a.n_rows = n_rows;
  a.mask_id = mask_id;
  a.max_win = max_win;
  a.n_unmasked = n_unmasked;
  lowconf_unmask_kernel<<<dim3((unsigned)n_seq), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(a);
  return check_launch(name);
}

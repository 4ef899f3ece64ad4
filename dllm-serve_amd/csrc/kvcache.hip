// K1 / K2: KV-cache scatter and gather by slot mapping, plus the library's
// error-reporting helpers.
//
// Layout: the cache is a flat array of rows of row_elems = Hkv*D bf16
// elements (slot stride row_elems); token rows of key/value have an element
// stride key_stride_tok.  One thread moves one 16-byte chunk (8 bf16), so a
// wavefront moves 1 KiB of contiguous row data per instruction; the slot
// index is re-read per chunk from L1/L2 (4 bytes per 16 moved).
#include "common.h"

#include <stdarg.h>
#include <stdio.h>

namespace dllm {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return DLLM_OK;
}

// ---- vectorised row copy: one wavefront per row, 16 bytes per lane ---------
// DIR == 0: store (token rows -> cache rows); DIR == 1: load (cache -> tokens).
template <int DIR>
__global__ __launch_bounds__(256) void kv_copy_vec(const uint16_t* __restrict__ src_k, const uint16_t* __restrict__ src_v,
                                                   uint16_t* __restrict__ dst_k, uint16_t* __restrict__ dst_v,
                                                   const int32_t* __restrict__ slot, int64_t k_stride,
                                                   int64_t v_stride, int64_t cache_slots, int n_tok,
                                                   int chunks_per_row) {
  const int lane = threadIdx.x & 63;
  const int waves_total = gridDim.x * (blockDim.x >> 6);
  const int64_t row_elems = (int64_t)chunks_per_row * 8;
  for (int i = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); i < n_tok; i += waves_total) {
    const int64_t s = slot[i];
    if (s < 0 || s >= cache_slots) continue;
    const uint16_t* ks;
    const uint16_t* vs;
    uint16_t* kd;
    uint16_t* vd;
    if (DIR == 0) {
      ks = src_k + (int64_t)i * k_stride;
      vs = src_v + (int64_t)i * v_stride;
      kd = dst_k + s * row_elems;
      vd = dst_v + s * row_elems;
    } else {
      ks = src_k + s * row_elems;
      vs = src_v + s * row_elems;
      kd = dst_k + (int64_t)i * k_stride;
      vd = dst_v + (int64_t)i * v_stride;
    }
    for (int c = lane; c < chunks_per_row; c += 64) {
      const u32x4_t a = ld128(ks + c * 8);
      const u32x4_t b = ld128(vs + c * 8);
      st128(kd + c * 8, a);
      st128(vd + c * 8, b);
    }
  }
}

// Scalar fallback for unaligned pointers / odd row sizes (2 bytes per thread).
template <int DIR>
__global__ __launch_bounds__(256) void kv_copy_scalar(const uint16_t* __restrict__ src_k, const uint16_t* __restrict__ src_v,
                                                      uint16_t* __restrict__ dst_k, uint16_t* __restrict__ dst_v,
                                                      const int32_t* __restrict__ slot, int64_t k_stride,
                                                      int64_t v_stride, int64_t cache_slots, int n_tok, int row_elems) {
  const int64_t total = (int64_t)n_tok * row_elems;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < total; c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = c / row_elems;
    const int64_t e = c - i * row_elems;
    const int64_t s = slot[i];
    if (s < 0 || s >= cache_slots) continue;
    const int64_t cache_off = s * row_elems + e;
    if (DIR == 0) {
      dst_k[cache_off] = src_k[i * k_stride + e];
      dst_v[cache_off] = src_v[i * v_stride + e];
    } else {
      dst_k[i * k_stride + e] = src_k[cache_off];
      dst_v[i * v_stride + e] = src_v[cache_off];
    }
  }
}

template <int DIR>
static int kv_copy(const uint16_t* sk, const uint16_t* sv, uint16_t* dk, uint16_t* dv, const int32_t* slot,
                   int64_t k_stride, int64_t v_stride, int64_t cache_slots, int n_tok, int row_elems,
                   void* stream, const char* name) {
  if (n_tok < 0 || row_elems <= 0 || cache_slots < 0)
    return fail(DLLM_ERR_INVALID_ARG, "%s: bad sizes n_tok=%d row_elems=%d cache_slots=%lld", name, n_tok, row_elems,
                (long long)cache_slots);
  if (n_tok == 0) return DLLM_OK;
  if (!sk || !sv || !dk || !dv || !slot) return fail(DLLM_ERR_INVALID_ARG, "%s: null pointer", name);
  if (k_stride < row_elems || v_stride < row_elems)
    return fail(DLLM_ERR_INVALID_ARG, "%s: token stride (%lld, %lld) smaller than row_elems %d", name,
                (long long)k_stride, (long long)v_stride, row_elems);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = (row_elems % 8 == 0) && (k_stride % 8 == 0) && (v_stride % 8 == 0) && aligned16(sk) &&
                   aligned16(sv) && aligned16(dk) && aligned16(dv);
  if (vec) {
    const int chunks = row_elems / 8;
    int64_t blocks = ((int64_t)n_tok + 3) / 4;  // four rows (wavefronts) per block
    if (blocks > 8192) blocks = 8192;
    kv_copy_vec<DIR><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(sk, sv, dk, dv, slot, k_stride, v_stride,
                                                                   cache_slots, n_tok, chunks);
  } else {
    const int64_t total = (int64_t)n_tok * row_elems;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    kv_copy_scalar<DIR><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(sk, sv, dk, dv, slot, k_stride, v_stride,
                                                                      cache_slots, n_tok, row_elems);
  }
  return check_launch(name);
}

}  // namespace dllm

extern "C" const char* dllm_last_error(void) { return dllm::g_err; }

extern "C" int dllm_abi_version(void) { return 200; }

extern "C" int dllm_store_kvcache(const dllm_bf16* key, int64_t key_stride_tok, const dllm_bf16* value,
                                  int64_t value_stride_tok, dllm_bf16* k_cache, dllm_bf16* v_cache,
                                  int64_t cache_slots, const int32_t* slot_mapping, int n_tok, int row_elems,
                                  void* stream) {
  dllm::g_err[0] = 0;
  return dllm::kv_copy<0>(key, value, k_cache, v_cache, slot_mapping, key_stride_tok, value_stride_tok, cache_slots,
                          n_tok, row_elems, stream, "dllm_store_kvcache");
}

extern "C" int dllm_load_kvcache(dllm_bf16* key, int64_t key_stride_tok, dllm_bf16* value, int64_t value_stride_tok,
                                 const dllm_bf16* k_cache, const dllm_bf16* v_cache, int64_t cache_slots,
                                 const int32_t* slot_mapping, int n_tok, int row_elems, void* stream) {
  dllm::g_err[0] = 0;
  return dllm::kv_copy<1>(k_cache, v_cache, key, value, slot_mapping, key_stride_tok, value_stride_tok, cache_slots,
                          n_tok, row_elems, stream, "dllm_load_kvcache");
}

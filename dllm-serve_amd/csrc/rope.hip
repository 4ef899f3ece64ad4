// K7: NeoX rotary embedding of q and k in one launch (gfx950).
//
// For token i (position p = positions[i]), head h and j in [0, D/2):
//   x1 = x[i, h, j], x2 = x[i, h, j + D/2]                      (bf16 -> f32)
//   c = cos_sin[p, j], s = cos_sin[p, D/2 + j]                  (f32 table)
//   y[i, h, j]       = bf16(x1*c - x2*s)
//   y[i, h, j + D/2] = bf16(x2*c + x1*s)
// Every product and the sum are rounded to f32 separately (no fused
// multiply-add), which is what the reference's f32 tensor expression
// computes op by op (dllmserve/layers/rotary_embedding.py:6-17).
//
// Thread = one 16-byte chunk pair (elements [8c, 8c+8) of both halves) of
// one head of one token, so the 8 lanes of a D = 128 head read and write
// 2 x 128 contiguous bytes; grid.x = token, grid.y covers the (Hq + Hkv)
// heads x D/16 chunk pairs of a token.  Memory bound: per token
// 4 (Hq + Hkv) D bytes of q/k traffic plus one 4D-byte table row (L2).
#include "common.h"

namespace dllm {

struct RopeArgs {
  const uint16_t* q_in;
  uint16_t* q_out;
  const uint16_t* k_in;
  uint16_t* k_out;
  int64_t qi_stride, qo_stride, ki_stride, ko_stride;
  const int64_t* positions;
  const float* cos_sin;
  int64_t max_position;
  int Hq, Hkv, D;
};

__device__ __forceinline__ float rot_first(float x1, float x2, float c, float s) {
#pragma clang fp contract(off)
  return x1 * c - x2 * s;
}
__device__ __forceinline__ float rot_second(float x1, float x2, float c, float s) {
#pragma clang fp contract(off)
  return x2 * c + x1 * s;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int i = blockIdx.x;
  const int cpr = a.D >> 4;  // chunk pairs per head
  const int r = blockIdx.y * 256 + threadIdx.x;
  if (r >= (a.Hq + a.Hkv) * cpr) return;
  const int64_t p = a.positions[i];
  if (p < 0 || p >= a.max_position) return;
  const int h = r / cpr;
  const int c = r - h * cpr;
  const int half = a.D >> 1;
  const uint16_t* src;
  uint16_t* dst;
  if (h < a.Hq) {
    src = a.q_in + (int64_t)i * a.qi_stride + h * a.D;
    dst = a.q_out + (int64_t)i * a.qo_stride + h * a.D;
  } else {
    src = a.k_in + (int64_t)i * a.ki_stride + (h - a.Hq) * a.D;
    dst = a.k_out + (int64_t)i * a.ko_stride + (h - a.Hq) * a.D;
  }
  const u32x4_t x1 = ld128_stream(src + 8 * c);
  const u32x4_t x2 = ld128_stream(src + half + 8 * c);
  const float* row = a.cos_sin + p * a.D;
  const f32x4_t c0 = *reinterpret_cast<const f32x4_t*>(row + 8 * c);
  const f32x4_t c1 = *reinterpret_cast<const f32x4_t*>(row + 8 * c + 4);
  const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(row + half + 8 * c);
  const f32x4_t s1 = *reinterpret_cast<const f32x4_t*>(row + half + 8 * c + 4);
  const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  u32x4_t y1, y2;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float a0 = bf16_lo(x1[w]), a1 = bf16_hi(x1[w]);
    const float b0 = bf16_lo(x2[w]), b1 = bf16_hi(x2[w]);
    y1[w] = cvt_pk_bf16(rot_first(a0, b0, cs[2 * w], sn[2 * w]), rot_first(a1, b1, cs[2 * w + 1], sn[2 * w + 1]));
    y2[w] = cvt_pk_bf16(rot_second(a0, b0, cs[2 * w], sn[2 * w]), rot_second(a1, b1, cs[2 * w + 1], sn[2 * w + 1]));
  }
  st128(dst + 8 * c, y1);
  st128(dst + half + 8 * c, y2);
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_rope_neox(const uint16_t* q_in, int64_t q_in_stride, uint16_t* q_out, int64_t q_out_stride,
                              const uint16_t* k_in, int64_t k_in_stride, uint16_t* k_out, int64_t k_out_stride,
                              const int64_t* positions, const float* cos_sin_cache, int64_t max_position,
                              int n_tok, int Hq, int Hkv, int D, void* stream) {
  static const char* name = "dllm_rope_neox";
  if (n_tok < 0 || Hq < 0 || Hkv < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (D <= 0 || D % 16 != 0 || D > 512)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: head_dim %d must be a multiple of 16 and at most 512", name, D);
  if (n_tok == 0 || Hq + Hkv == 0) return DLLM_OK;
  if (!positions || !cos_sin_cache || max_position <= 0)
    return fail(DLLM_ERR_INVALID_ARG, "%s: positions / cos_sin_cache / max_position missing", name);
  if (Hq > 0 && (!q_in || !q_out)) return fail(DLLM_ERR_INVALID_ARG, "%s: q pointers missing", name);
  if (Hkv > 0 && (!k_in || !k_out)) return fail(DLLM_ERR_INVALID_ARG, "%s: k pointers missing", name);
  const void* ptrs[] = {q_in, q_out, k_in, k_out, cos_sin_cache};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(DLLM_ERR_INVALID_ARG, "%s: pointers must be 16-byte aligned", name);
  if ((Hq > 0 && (q_in_stride < (int64_t)Hq * D || q_out_stride < (int64_t)Hq * D || q_in_stride % 8 ||
                  q_out_stride % 8)) ||
      (Hkv > 0 && (k_in_stride < (int64_t)Hkv * D || k_out_stride < (int64_t)Hkv * D || k_in_stride % 8 ||
                   k_out_stride % 8)))
    return fail(DLLM_ERR_INVALID_ARG, "%s: token strides must be >= H*D and multiples of 8 elements", name);
  const int64_t per_tok = (int64_t)(Hq + Hkv) * (D / 16);
  if (per_tok > (int64_t)256 * 65535) return fail(DLLM_ERR_INVALID_ARG, "%s: too many heads", name);
  RopeArgs a;
  a.q_in = q_in; a.q_out = q_out; a.k_in = k_in; a.k_out = k_out;
  a.qi_stride = q_in_stride; a.qo_stride = q_out_stride; a.ki_stride = k_in_stride; a.ko_stride = k_out_stride;
  a.positions = positions; a.cos_sin = cos_sin_cache; a.max_position = max_position;
  a.Hq = Hq; a.Hkv = Hkv; a.D = D;
  const dim3 grid((unsigned)n_tok, (unsigned)((per_tok + 255) / 256));
  rope_kernel<<<grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(a);
  return check_launch(name);
}

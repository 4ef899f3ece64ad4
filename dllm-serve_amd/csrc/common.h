// Shared device helpers for the gfx950 kernels: vector types, bf16 bit
// conversions, the thread-local error string and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "dllm_attn.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

namespace dllm {

// ---- host-side error reporting -------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- bf16 <-> f32 (bit exact) ---------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
// Round-to-nearest-even f32 -> bf16 bits (NaN kept quiet).  Same rule the
// oracle implements with integer arithmetic.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
// f64 -> f32 (round to nearest even) -> bf16 (round to nearest even): two
// roundings, as torch's double -> bfloat16 conversion does.  The empty asm
// keeps the compiler from merging the two conversions into a single
// double -> bf16 rounding (which it lowers through round-to-odd); the two
// differ when the f32 value lands exactly on a bf16 midpoint.
__device__ __forceinline__ uint32_t f64_to_bf16_bits_2step(double x) {
  float f = (float)x;
  asm volatile("" : "+v"(f));
  return f32_to_bf16_bits(f);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// Two f32 -> packed bf16x2 (round to nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  const f32x2_t x = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// acc + lo + hi of a packed bf16 pair, exactly the values an MFMA B operand
// holds (one v_dot2_f32_bf16 against (1, 1)).
__device__ __forceinline__ float add_bf16x2(uint32_t pk, float acc) {
  const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk), one, acc, false);
}

// Combine a value across the lane pair (l, l ^ 32) with v_permlane32_swap
// (gfx950): after the swap one operand holds lanes 0..31 of x in both halves
// and the other lanes 32..63.  Every lane of the wavefront must be active.
// pair_max32 takes the maximum with one v_max_f32: fmaxf on the swap's
// outputs would first quieten both operands (two more VALU instructions),
// which the callers' NaN-free inputs never need.
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"((uint32_t)r[0]), "v"((uint32_t)r[1]));
  return m;
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Cross-lane moves inside the LDS-free VALU datapath (DPP and the gfx950
// permlane swaps) instead of ds_bpermute round trips; every lane of the
// wavefront must be active.  Lane semantics (checked on the device): row_shl:n
// gives lane l the value of lane l + n of its 16-lane row, row_shr:n of lane
// l - n (0 past the row start with bound_ctrl), row_ror:8 of lane l ^ 8,
// row_bcast:15 / :31 of lane 15 / 31 to the rows selected by the row mask;
// permlane16_swap(x, x) returns rows (0, 0, 2, 2) and (1, 1, 3, 3) of x,
// permlane32_swap(x, x) halves (0, 0) and (1, 1).
__device__ __forceinline__ uint32_t lane_xor(uint32_t x, int j) {
  const int lane = threadIdx.x & 63;
  switch (j) {
    case 1:
      return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    case 2:
      return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    case 4: {
      const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x104, 0xF, 0xF, false);  // l + 4
      const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x114, 0xF, 0xF, false);  // l - 4
      return (lane & 4) ? dn : up;
    }
    case 8:
      return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x128, 0xF, 0xF, false);  // row_ror:8
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
      return (lane & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
      return (lane & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
    }
  }
}

// Inclusive prefix sum over the 64 lanes: sums within 16-lane rows
// (row_shr 1, 2, 4, 8), then the row totals carried by row_bcast.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
  return x;
}

// Workgroup barrier that orders LDS only: each wavefront waits for its own
// LDS operations, then all meet.  Global loads still in flight stay in flight
// (the attention kernels' DMA waited for with vm_wait, the selection copy's
// preloaded rows).  Between wavefronts that each waited for their own DMA
// (vm_wait) and finished their own LDS reads: the wait on LDS reads plus
// s_barrier is all the ordering needed.  __syncthreads() in a kernel that
// fills LDS with global_load_lds makes the compiler wait for vmcnt(0) before
// the barrier, which would also retire the DMA of the next tile.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Buffer resource over [base, base + bytes): loads at offsets >= bytes return
// zero, which is how rows past the end of a segment read as zero without any
// per-lane clamping.  The whole offset is passed in the VGPR operand (the
// scalar offset is kept 0 so the range check covers it); offsets are 32-bit
// byte offsets from base, which the host checks cannot overflow.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// s_waitcnt vmcnt(N), expcnt / lgkmcnt untouched (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
// The waitcnt intrinsic is not a memory operation for the compiler, so an
// empty asm with a memory clobber follows it: no LDS read of the tile being
// waited for can be hoisted above the wait.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
  asm volatile("" ::: "memory");
}

// AUX = 2: non-temporal (streaming) policy, for bytes that one workgroup reads once.
template <int AUX = 0>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16, (int)voff, 0, 0,
                                           AUX);
}

// Plain 128-bit global load / store.
__device__ __forceinline__ u32x4_t ld128(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// Cache-policy bits of the load builtins: 2 = nt (streaming: the line is
// read once and need not stay in L2 ahead of reused data).
constexpr int kStreamAux = 2;
// 128-bit load of data read exactly once, with the nt hint.
__device__ __forceinline__ u32x4_t ld128_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ void st128(void* p, u32x4_t v) { *reinterpret_cast<u32x4_t*>(p) = v; }

}  // namespace dllm

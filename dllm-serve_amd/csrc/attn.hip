// K3a / K3b: bidirectional attention on gfx950 bf16 MFMA.
//
// One kernel template serves both paths:
//   * K3a (dense varlen, modes 0/1): a workgroup of 4 wavefronts owns 128
//     "M rows" of one segment and one KV head and streams the segment's keys
//     through LDS in tiles of 64; each wavefront owns 32 M rows.
//   * K3b (generation block vs cached KV, mode 2): a workgroup owns 32 M
//     rows; its 4 wavefronts split every 128-key tile (32 keys each) and are
//     merged in LDS at the end; long key ranges are also split across
//     workgroups (partials in a workspace, merged by attn_combine_kernel).
//
// "M rows" pack the Hq/Hkv query heads that share a KV head: M row m of a
// segment is token m / g, query head hkv*g + m % g (g = Hq/Hkv), so every
// K/V byte brought into LDS serves all g heads.
//
// Per wavefront and key block of 32 the math is
//   S^T[32 keys x 32 rows] = K[32 x 128] . Q^T[128 x 32]   (8 x mfma 32x32x16)
//   online softmax over keys (rows live in lanes: lane%32 = M row)
//   O^T[128 x 32] += V^T[128 x 32 keys] . P^T[32 keys x 32] (8 x mfma 32x32x16)
// Computing the transposed products keeps the softmax statistics and the
// O^T accumulator of an M row in the same lane, so P^T goes straight from
// the S^T accumulator registers into the B operand of the second product.
// The key order inside each group of 16 is permuted consistently in the V^T
// LDS tile and in P^T (a contraction is invariant under a permutation of its
// summation index), which makes every operand fetch one 16-byte LDS read.
#include "common.h"

#include <math.h>

#include <type_traits>

namespace dllm {

constexpr int HD = 128;       // head dim handled by this build
constexpr int KSTR = HD + 8;  // LDS row stride (elements) of the K tile: 272 B, conflict-free 16 B reads

template <int WM, int WK, int KBW>
struct Cfg {
  static constexpr int NKT = 32 * KBW * WK;  // keys per workgroup tile
  static constexpr int VSTR = NKT + 8;       // LDS row stride (elements) of the V^T tile
  static constexpr int K_ELEMS = NKT * KSTR;
  static constexpr int V_ELEMS = HD * VSTR;
  static constexpr int BUF_ELEMS = K_ELEMS + V_ELEMS;
  static constexpr int BM = 32 * WM;               // M rows per workgroup
  static constexpr int KCH = NKT / 16;             // 16-byte K chunks per thread per tile
  static constexpr int VGR = NKT / 64;             // (4 keys x 8 d) V groups per thread per tile
  static constexpr int LDS_BYTES = 2 * BUF_ELEMS * 2;
};

struct SegDesc {
  int qrow0;     // first q / o row of the segment
  int Lq;        // q rows (tokens)
  int krow0;     // first contiguous k / v row
  int Lkb;       // contiguous k / v rows
  int n_c;       // cached rows in front of the contiguous ones (K3b)
  int slot_base; // offset of this segment's slots
};

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* seg_ids;
  const int32_t* slots;
  const int32_t* slot_off;
  float* ws;          // split partials (K3b, n_split > 1)
  int64_t q_stride, k_stride, v_stride, o_stride;
  int64_t cache_slots;
  int n_seg, Hkv, g, mtiles, n_split, keys_per_split;
  int logical_blocks;
  float scale_log2;
};

__device__ __forceinline__ int xcd_remap(int b, int nb) {
  // Work-groups are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous range of logical tiles so the tiles of one (segment, head),
  // which read the same K/V, share that XCD's L2.
  const int per = nb >> 3;
  return (b & 7) * per + (b >> 3);
}

__device__ __forceinline__ u32x4_t zero_unless(u32x4_t v, bool ok) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = ok ? v[i] : 0u;
  return r;
}

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

// Where each thread's 16-byte pieces of a key tile go:
//   K: rows (tid >> 4) + 16 i, chunk tid & 15               (i < KCH)
//   V: 4 rows 4 kg + e of the 8-element column chunk dc      (i < VGR)
//      with idx = tid + 256 i, kg = idx % (NKT/4), dc = idx / (NKT/4)
template <int WM, int WK, int KBW>
struct TileRegs {
  using C = Cfg<WM, WK, KBW>;
  u32x4_t kr[C::KCH];
  u32x4_t vr[C::VGR][4];

  __device__ __forceinline__ void store(uint16_t* buf) const {
    const int tid = threadIdx.x;
    uint16_t* Ks = buf;
    uint16_t* Vt = buf + C::K_ELEMS;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int row = (tid >> 4) + 16 * i;
      const int ch = tid & 15;
      *reinterpret_cast<u32x4_t*>(Ks + row * KSTR + ch * 8) = kr[i];
    }
#pragma unroll
    for (int i = 0; i < C::VGR; ++i) {
      const int idx = tid + 256 * i;
      const int kg = idx % (C::NKT / 4);
      const int dc = idx / (C::NKT / 4);
      const int j = kg & 3;
      // Keys 4kg..4kg+3 sit at positions pos..pos+3 of the permuted order:
      // inside a group of 16 keys, position 8h + i holds key 4h + (i%4) + 8(i/4).
      const int pos = 16 * (kg >> 2) + 8 * (j & 1) + 4 * (j >> 1);
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // word w holds d = dc*8 + 2w (low half), 2w+1 (high half)
        const uint32_t a0 = vr[i][0][w], a1 = vr[i][1][w], a2 = vr[i][2][w], a3 = vr[i][3][w];
        u32x2_t lo, hi;
        lo[0] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
        lo[1] = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
        hi[0] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
        hi[1] = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
        const int d = dc * 8 + 2 * w;
        *reinterpret_cast<u32x2_t*>(Vt + d * C::VSTR + pos) = lo;
        *reinterpret_cast<u32x2_t*>(Vt + (d + 1) * C::VSTR + pos) = hi;
      }
    }
  }
};

// Dense segments: K/V rows are contiguous token rows of the segment.  All
// address arithmetic is scalar except one 32-bit base offset per piece.
template <int WM, int WK, int KBW>
struct DenseLoader : TileRegs<WM, WK, KBW> {
  using C = Cfg<WM, WK, KBW>;
  __amdgpu_buffer_rsrc_t krs, vrs;
  uint32_t kS, vS;               // token stride in bytes
  uint32_t k_off;                // this thread's K piece offset for tile row 0
  uint32_t v_off[C::VGR];        // this thread's V piece offsets for tile row 0

  __device__ __forceinline__ void init(const AttnArgs& a, const SegDesc& sd, int hkv) {
    const int tid = threadIdx.x;
    kS = (uint32_t)(a.k_stride * 2);
    vS = (uint32_t)(a.v_stride * 2);
    const uint16_t* kb = a.k + (int64_t)sd.krow0 * a.k_stride + hkv * HD;
    const uint16_t* vb = a.v + (int64_t)sd.krow0 * a.v_stride + hkv * HD;
    const int Lk = sd.Lkb;
    krs = make_rsrc(kb, Lk > 0 ? (uint32_t)(Lk - 1) * kS + HD * 2 : 0u);
    vrs = make_rsrc(vb, Lk > 0 ? (uint32_t)(Lk - 1) * vS + HD * 2 : 0u);
    k_off = (uint32_t)(tid >> 4) * kS + (uint32_t)(tid & 15) * 16u;
#pragma unroll
    for (int i = 0; i < C::VGR; ++i) {
      const int idx = tid + 256 * i;
      const int kg = idx % (C::NKT / 4);
      const int dc = idx / (C::NKT / 4);
      v_off[i] = (uint32_t)(kg * 4) * vS + (uint32_t)dc * 16u;
    }
  }

  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) this->kr[i] = bload(krs, k_off + (uint32_t)(k0 + 16 * i) * kS, 0u);
#pragma unroll
    for (int i = 0; i < C::VGR; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) this->vr[i][e] = bload(vrs, v_off[i] + (uint32_t)(k0 + e) * vS, 0u);
  }
};

// Cached segments (mode 2): key index kidx < n_c reads cache row
// slots[slot_base + kidx]; n_c <= kidx < n_c + Lkb reads block row kidx - n_c.
// The slots of the next-but-one tile are fetched while the next tile's rows
// are loaded, so no tile waits on its own slot indirection.
template <int WM, int WK, int KBW>
struct CachedLoader : TileRegs<WM, WK, KBW> {
  using C = Cfg<WM, WK, KBW>;
  const AttnArgs* ap;
  const int32_t* sp;   // this segment's slots (a valid dummy when it has none)
  int hkv, kend, n_c, krow0, Lkb;
  int sk[C::KCH];      // slots of this thread's K rows of the pending tile
  int sv[C::VGR][4];   // slots of this thread's V rows of the pending tile

  __device__ __forceinline__ void init(const AttnArgs& a, const SegDesc& sd, int hkv_, int kend_) {
    ap = &a;
    hkv = hkv_;
    kend = kend_;
    n_c = sd.n_c;
    krow0 = sd.krow0;
    Lkb = sd.Lkb;
    sp = n_c > 0 ? a.slots + sd.slot_base : a.slot_off;
  }

  // Slot of cached row kidx; the index is clamped into the segment's slot
  // list so the (unconditional) load is always in bounds.
  __device__ __forceinline__ int slot_at(int kidx) const { return sp[min(max(kidx, 0), max(n_c - 1, 0))]; }

  __device__ __forceinline__ void fetch_slots(int k0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) sk[i] = slot_at(k0 + (tid >> 4) + 16 * i);
#pragma unroll
    for (int i = 0; i < C::VGR; ++i) {
      const int kg = (tid + 256 * i) % (C::NKT / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[i][e] = slot_at(k0 + kg * 4 + e);
    }
  }

  __device__ __forceinline__ u32x4_t row_piece(const uint16_t* cache, const uint16_t* blk, int64_t stride, int slot,
                                               int kidx, int col) const {
    const AttnArgs& a = *ap;
    const bool in_range = kidx < kend;
    const bool cached = kidx < n_c;
    const bool slot_ok = slot >= 0 && (int64_t)slot < a.cache_slots;
    const uint16_t* p;
    if (cached)
      p = cache + (int64_t)(slot_ok ? slot : 0) * (a.Hkv * HD) + hkv * HD;
    else
      p = blk + (int64_t)(krow0 + min(max(kidx - n_c, 0), Lkb - 1)) * stride + hkv * HD;
    return zero_unless(ld128(p + col), in_range && (!cached || slot_ok));
  }

  __device__ __forceinline__ void load(int k0) {
    const AttnArgs& a = *ap;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i)
      this->kr[i] = row_piece(a.k_cache, a.k, a.k_stride, sk[i], k0 + (tid >> 4) + 16 * i, (tid & 15) * 8);
#pragma unroll
    for (int i = 0; i < C::VGR; ++i) {
      const int idx = tid + 256 * i;
      const int kg = idx % (C::NKT / 4);
      const int dc = idx / (C::NKT / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        this->vr[i][e] = row_piece(a.v_cache, a.v, a.v_stride, sv[i][e], k0 + kg * 4 + e, dc * 8);
    }
  }
};

// Running softmax state of one wavefront (M row = lane % 32).  The reference
// maximum m_run (log2 domain) is only raised when a new score exceeds it by
// more than kLazy, so most tiles skip rescaling O; probabilities then stay
// below 2^kLazy, well inside the bf16 / fp32 range.
constexpr float kLazy = 8.0f;

template <int KBW>
struct WaveState {
  f32x16_t oacc[4];
  float m_run;  // reference maximum, log2 domain
  float l_run;  // this lane's half of the row sum
};

// One key tile for one wavefront: S^T = K Q^T, online softmax, O^T += V^T P^T.
template <int WM, int WK, int KBW, bool MASK>
__device__ __forceinline__ void tile_compute(const uint16_t* Ks, const uint16_t* Vt, const bf16x8_t (&qf)[8],
                                             WaveState<KBW>& st, float c, int k_valid) {
  using C = Cfg<WM, WK, KBW>;
  const int lane = threadIdx.x & 63;
  const int lrow = lane & 31;
  const int hl = lane >> 5;
  const int wk = (threadIdx.x >> 6) / WM;

  f32x16_t sacc[KBW];
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sacc[b][i] = 0.f;
    const int kb = wk * KBW + b;
    const uint16_t* kp = Ks + (kb * 32 + lrow) * KSTR + hl * 8;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8_t af = as_bf16x8(*reinterpret_cast<const u32x4_t*>(kp + kk * 16));
      sacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[kk], sacc[b], 0, 0, 0);
    }
  }

  float mx = -INFINITY;
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
    const int kb = wk * KBW + b;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (MASK) {
        const int key = kb * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (key >= k_valid) sacc[b][i] = -INFINITY;
      }
      mx = fmaxf(mx, sacc[b][i]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32)) * c;  // c > 0: scaling commutes with max
  const bool need = mx > st.m_run + kLazy;
  if (__builtin_amdgcn_ballot_w64(need)) {
    const float m_new = need ? mx : st.m_run;
    const float alpha = (st.m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(st.m_run - m_new);
    st.l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) st.oacc[db][i] *= alpha;
    st.m_run = m_new;
  }
  const float neg_m = (st.m_run == -INFINITY) ? 0.f : -st.m_run;

  float psum = 0.f;
  bf16x8_t pf[2 * KBW];
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4_t pk;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][8 * j + 2 * w], c, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][8 * j + 2 * w + 1], c, neg_m));
        psum += p0 + p1;
        pk[w] = cvt_pk_bf16(p0, p1);
      }
      pf[2 * b + j] = as_bf16x8(pk);
    }
  }
  st.l_run += psum;

#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const uint16_t* vp = Vt + (db * 32 + lrow) * C::VSTR + wk * KBW * 32 + hl * 8;
#pragma unroll
    for (int cch = 0; cch < 2 * KBW; ++cch) {
      const bf16x8_t af = as_bf16x8(*reinterpret_cast<const u32x4_t*>(vp + cch * 16));
      st.oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, pf[cch], st.oacc[db], 0, 0, 0);
    }
  }
}

template <int WM, int WK, int KBW, bool CACHED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WK == 1 ? 2 : 1, WK == 1 ? 2 : 1))) void attn_fwd_kernel(AttnArgs a) {
  using C = Cfg<WM, WK, KBW>;
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  if (L >= a.logical_blocks) return;

  int r = L;
  int split = 0;
  if (CACHED) {
    split = r % a.n_split;
    r /= a.n_split;
  }
  const int mt = r % a.mtiles;
  r /= a.mtiles;
  const int hkv = r % a.Hkv;
  const int s = r / a.Hkv;
  const int sid = a.seg_ids ? a.seg_ids[s] : s;

  SegDesc sd;
  sd.qrow0 = a.cu_q[sid];
  sd.Lq = a.cu_q[sid + 1] - sd.qrow0;
  if (CACHED) {
    sd.krow0 = sd.qrow0;
    sd.Lkb = sd.Lq;
    sd.slot_base = a.slot_off[s];
    sd.n_c = a.slot_off[s + 1] - sd.slot_base;
  } else {
    sd.krow0 = a.cu_k[sid];
    sd.Lkb = a.cu_k[sid + 1] - sd.krow0;
    sd.n_c = 0;
    sd.slot_base = 0;
  }
  const int g = a.g;
  const int M = sd.Lq * g;
  const int m_base = mt * C::BM;
  if (m_base >= M) return;
  const int Lk = sd.n_c + sd.Lkb;
  int kbeg = 0, kend = Lk;
  if (CACHED) {
    kbeg = split * a.keys_per_split;
    kend = min(Lk, kbeg + a.keys_per_split);
    if (kbeg > kend) kbeg = kend;
  }

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lrow = lane & 31;
  const int hl = lane >> 5;
  const int wm = wave % WM;
  const int wk = wave / WM;

  // ---- Q^T fragments (B operand of S^T = K Q^T), resident for the whole loop.
  // Rows past the segment (M tail) read as zero through the buffer bound.
  const int m = m_base + wm * 32 + lrow;
  const bool m_ok = m < M;
  const int tok = m_ok ? m / g : 0;
  const int head = hkv * g + (m_ok ? m - tok * g : 0);
  bf16x8_t qf[8];
  {
    const uint32_t qS = (uint32_t)(a.q_stride * 2);
    const __amdgpu_buffer_rsrc_t qrs =
        make_rsrc(a.q + (int64_t)sd.qrow0 * a.q_stride, sd.Lq > 0 ? (uint32_t)sd.Lq * qS : 0u);

    const uint32_t qbytes = sd.Lq > 0 ? (uint32_t)sd.Lq * qS : 0u;
    const uint32_t qoff = m_ok ? (uint32_t)tok * qS + (uint32_t)(head * HD + hl * 8) * 2u : qbytes;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = as_bf16x8(bload(qrs, qoff + (uint32_t)kk * 32u, 0u));
  }

  WaveState<KBW> st;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) st.oacc[db][i] = 0.f;
  st.m_run = -INFINITY;
  st.l_run = 0.f;
  const float c = a.scale_log2;

  const int ntiles = (kend - kbeg + C::NKT - 1) / C::NKT;
  using Loader = typename std::conditional<CACHED, CachedLoader<WM, WK, KBW>, DenseLoader<WM, WK, KBW>>::type;
  Loader io;
  if constexpr (CACHED) {
    io.init(a, sd, hkv, kend);
    io.fetch_slots(kbeg);
  } else {
    io.init(a, sd, hkv);
  }
  if (ntiles > 0) {
    io.load(kbeg);
    if constexpr (CACHED) io.fetch_slots(kbeg + C::NKT);
    io.store(smem);
  }
  __syncthreads();

  // Full tiles with the next tile's loads in flight; the last (possibly
  // partial) tile is peeled off and masked.
  for (int t = 0; t + 1 < ntiles; ++t) {
    const int k0 = kbeg + t * C::NKT;
    io.load(k0 + C::NKT);
    if constexpr (CACHED) io.fetch_slots(k0 + 2 * C::NKT);
    const uint16_t* Ks = smem + (t & 1) * C::BUF_ELEMS;
    tile_compute<WM, WK, KBW, false>(Ks, Ks + C::K_ELEMS, qf, st, c, C::NKT);
    io.store(smem + ((t + 1) & 1) * C::BUF_ELEMS);
    __syncthreads();
  }
  if (ntiles > 0) {
    const int t = ntiles - 1;
    const int k_valid = kend - (kbeg + t * C::NKT);
    const uint16_t* Ks = smem + (t & 1) * C::BUF_ELEMS;
    if (k_valid < C::NKT)
      tile_compute<WM, WK, KBW, true>(Ks, Ks + C::K_ELEMS, qf, st, c, k_valid);
    else
      tile_compute<WM, WK, KBW, false>(Ks, Ks + C::K_ELEMS, qf, st, c, C::NKT);
  }
  __syncthreads();

  const float m_run = st.m_run;
  const float l_tot = st.l_run + __shfl_xor(st.l_run, 32);
  f32x16_t (&oacc)[4] = st.oacc;

  if constexpr (WK == 1) {
    // ---- direct epilogue: normalise and store bf16
    if (m_ok) {
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      uint16_t* op = a.o + (int64_t)(sd.qrow0 + tok) * a.o_stride + head * HD;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = db * 32 + 8 * rq + 4 * hl;
          u32x2_t w;
          w[0] = pack_bf16x2(oacc[db][4 * rq + 0] * inv, oacc[db][4 * rq + 1] * inv);
          w[1] = pack_bf16x2(oacc[db][4 * rq + 2] * inv, oacc[db][4 * rq + 3] * inv);
          *reinterpret_cast<u32x2_t*>(op + d) = w;
        }
    }
  } else {
    // ---- merge the WK wavefronts' partial softmax states in LDS
    float* red = reinterpret_cast<float*>(smem);
    float* red_m = red;                 // [WK][32]
    float* red_l = red + WK * 32;       // [WK][32]
    float* ored = red + 2 * WK * 32;    // [WK][128][32]
    if (hl == 0) {
      red_m[wk * 32 + lrow] = m_run;
      red_l[wk * 32 + lrow] = l_tot;
    }
    __syncthreads();
    float m_all = -INFINITY;
#pragma unroll
    for (int w = 0; w < WK; ++w) m_all = fmaxf(m_all, red_m[w * 32 + lrow]);
    const float m_all_use = (m_all == -INFINITY) ? 0.f : m_all;
    const float fac = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_all_use);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = db * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        ored[(wk * HD + d) * 32 + lrow] = oacc[db][i] * fac;
      }
    __syncthreads();
    // 256 threads: row q = tid / 8, 16 consecutive d per thread.
    const int q = tid >> 3;
    const int d0 = (tid & 7) * 16;
    float mq = -INFINITY;
#pragma unroll
    for (int w = 0; w < WK; ++w) mq = fmaxf(mq, red_m[w * 32 + q]);
    const float mq_use = (mq == -INFINITY) ? 0.f : mq;
    float lq = 0.f;
#pragma unroll
    for (int w = 0; w < WK; ++w) {
      const float mw = red_m[w * 32 + q];
      lq += (mw == -INFINITY) ? 0.f : red_l[w * 32 + q] * __builtin_amdgcn_exp2f(mw - mq_use);
    }
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < WK; ++w) sum += ored[(w * HD + d0 + i) * 32 + q];
      acc[i] = sum;
    }
    const int mrow = m_base + q;
    if (mrow < M) {
      const int tq = mrow / g;
      const int hq = hkv * g + (mrow - tq * g);
      if (a.n_split == 1) {
        const float inv = lq > 0.f ? 1.f / lq : 0.f;
        uint16_t* op = a.o + (int64_t)(sd.qrow0 + tq) * a.o_stride + hq * HD + d0;
        u32x4_t w0, w1;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          w0[w] = pack_bf16x2(acc[2 * w] * inv, acc[2 * w + 1] * inv);
          w1[w] = pack_bf16x2(acc[8 + 2 * w] * inv, acc[8 + 2 * w + 1] * inv);
        }
        st128(op, w0);
        st128(op + 8, w1);
      } else {
        // partial record P = ((s*Hkv + hkv)*mtiles + mt)*n_split + split, 32 rows each
        const int64_t P = (((int64_t)s * a.Hkv + hkv) * a.mtiles + mt) * a.n_split + split;
        float* po = a.ws + (P * 32 + q) * HD + d0;
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
          f32x4_t v4 = {acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
          *reinterpret_cast<f32x4_t*>(po + i) = v4;
        }
        if ((tid & 7) == 0) {
          const int64_t nrec = (int64_t)a.n_seg * a.Hkv * a.mtiles * a.n_split;
          float* pml = a.ws + nrec * 32 * HD + (P * 32 + q) * 2;
          pml[0] = mq;
          pml[1] = lq;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K3a, dense varlen attention: K and V tiles go HBM -> LDS by buffer DMA
// (buffer_load_dwordx4 ... lds, no VGPR staging); the V^T MFMA operand is
// read with the transposing LDS read ds_read_b64_tr_b16.
//
// LDS per stage (2 stages): K [64 keys][256 B] then V [64 keys][256 B], no
// padding; 16-byte chunks are XOR-swizzled inside a row so the MFMA operand
// reads are bank-conflict free:
//   K: physical chunk = logical chunk ^ (row & 15)
//   V: physical chunk = logical chunk ^ (4 * (row & 3))
// One DMA instruction writes 1 KiB = 4 rows; lane L of it carries row
// 4q + L/16, physical chunk L%16.
//
// ds_read_b64_tr_b16 (gfx950): in each group of 16 lanes, lane 4k+c supplies
// 8 bytes = elements [4c, 4c+4) of row k of a 4 x 16 block; lane n receives
// column n (rows 0..3).  With rows = keys and columns = head-dim positions
// this yields 4 consecutive keys of one d: half of a V^T A-operand fragment.
constexpr int DK_TILE = 64;                    // keys per tile
constexpr int DK_STAGE_BYTES = 2 * DK_TILE * 256;  // K + V

// s_waitcnt vmcnt(N), expcnt / lgkmcnt untouched (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16, (int)voff, 0, 0, 0);
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2_t ds_read_tr16(const uint8_t* p) {
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4_t*)(const_cast<uint8_t*>(p)));
  return __builtin_bit_cast(u32x2_t, v);
}

// Per-lane LDS / DMA offsets.  The swizzles make every per-kk (K) and per-db
// (V) read offset a XOR of one base with a compile-time constant:
//   K read, kk:  lrow*256 + ((2kk + hl) ^ (lrow & 15))*16 = kbase ^ (32 kk)
//   V read, db:  (4hl + k)*256 + (4(db ^ k) + 2 dhalf + c/2)*16 + 8(c&1) = vbase ^ (64 db)
// A DMA instruction q writes tile rows R = 4q + L/16 (L = lane), physical
// chunk P = L % 16, i.e. global chunk P ^ (R & 15) (K) or P ^ 4(R & 3) (V):
//   K: (L/16)*kS + ((P ^ (L/16)) * 16 ^ 64 (q & 3))      V: (L/16)*vS + (P ^ 4(L/16))*16
struct DenseAddr {
  uint32_t kbase, vbase;
  uint32_t kdma, vdma;
};

__device__ __forceinline__ void dense_addr(DenseAddr& ad, int lane, uint32_t kS, uint32_t vS) {
  const int rl = lane >> 4, P = lane & 15;
  ad.kdma = (uint32_t)rl * kS + (uint32_t)((P ^ rl) * 16);
  ad.vdma = (uint32_t)rl * vS + (uint32_t)((P ^ (4 * rl)) * 16);
  const int lrow = lane & 31, hl = lane >> 5;
  ad.kbase = (uint32_t)(lrow * 256 + ((hl ^ (lrow & 15)) * 16));
  const int dhalf = (lane >> 4) & 1, k = (lane & 15) >> 2, c = lane & 3;
  ad.vbase = (uint32_t)((4 * hl + k) * 256 + (4 * k + 2 * dhalf + (c >> 1)) * 16 + 8 * (c & 1));
}

// Softmax state of NQ query blocks (32 M rows each) of one wavefront.
template <int NQ>
struct DenseState {
  f32x16_t oacc[NQ][4];
  float m_run[NQ];
  float l_run[NQ];
};

// Online-softmax update of one query block from its two S^T key blocks;
// returns the packed P^T fragments (B operands of O^T += V^T P^T).
template <bool MASK>
__device__ __forceinline__ void dense_softmax(f32x16_t (&sacc)[2], f32x16_t (&oacc)[4], float& m_run, float& l_run,
                                              bf16x8_t (&pf)[4], float c, int k_valid, int hl) {
  float mx = -INFINITY;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (MASK) {
        const int key = b * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (key >= k_valid) sacc[b][i] = -INFINITY;
      }
      mx = fmaxf(mx, sacc[b][i]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32)) * c;
  const bool need = mx > m_run + kLazy;
  if (__builtin_amdgcn_ballot_w64(need)) {
    const float m_new = need ? mx : m_run;
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
    m_run = m_new;
  }
  const float neg_m = (m_run == -INFINITY) ? 0.f : -m_run;
  float psum = 0.f;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4_t pk;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][8 * j + 2 * w], c, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][8 * j + 2 * w + 1], c, neg_m));
        psum += p0 + p1;
        pk[w] = cvt_pk_bf16(p0, p1);
      }
      pf[2 * b + j] = as_bf16x8(pk);
    }
  l_run += psum;
}

// One 64-key tile for one wavefront owning NQ query blocks: every K and V^T
// operand fragment read from LDS feeds NQ MFMAs.
template <int NQ, bool MASK>
__device__ __forceinline__ void dense_tile(const uint8_t* Ks, const uint8_t* Vs, const DenseAddr& ad,
                                           const bf16x8_t (&qf)[NQ][8], DenseState<NQ>& st, float c, int k_valid) {
  const int lane = threadIdx.x & 63;
  const int hl = lane >> 5;
  // kk outer, key block inner: the 2*NQ accumulators form independent MFMA
  // chains that interleave instead of one chain waiting on itself.
  f32x16_t sacc[NQ][2];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[q][b][i] = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const bf16x8_t af =
          as_bf16x8(*reinterpret_cast<const u32x4_t*>(Ks + b * 32 * 256 + (ad.kbase ^ (uint32_t)(32 * kk))));
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        sacc[q][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[q][kk], sacc[q][b], 0, 0, 0);
    }
  }
  bf16x8_t pf[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q) dense_softmax<MASK>(sacc[q], st.oacc[q], st.m_run[q], st.l_run[q], pf[q], c, k_valid, hl);
  // key chunk outer, d block inner: 4*NQ independent accumulator chains.
#pragma unroll
  for (int cch = 0; cch < 4; ++cch) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const uint8_t* vp = Vs + (ad.vbase ^ (uint32_t)(64 * db)) + cch * 16 * 256;
      const u32x2_t lo = ds_read_tr16(vp);
      const u32x2_t hi = ds_read_tr16(vp + 8 * 256);
      u32x4_t a4 = {lo[0], lo[1], hi[0], hi[1]};
      const bf16x8_t af = as_bf16x8(a4);
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        st.oacc[q][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, pf[q][cch], st.oacc[q][db], 0, 0, 0);
    }
  }
}

// NW wavefronts x NQ query blocks of 32 M rows = 32*NW*NQ rows per
// workgroup; ST LDS stages (ST-1 tiles in flight while one is computed).
template <int NW, int NQ, int ST>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NQ == 1 ? 2 : 1, NQ == 1 ? 2 : 1))) void attn_dense_kernel(AttnArgs a) {
  constexpr int BM = 32 * NW * NQ;
  constexpr int DMA_PER_WAVE = DK_TILE * 256 / 1024 / NW;  // 1 KiB DMA instructions per wave, K (same for V)
  constexpr int DMA_TILE = 2 * DMA_PER_WAVE;               // this wave's DMA instructions per tile
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  if (L >= a.logical_blocks) return;
  int r = L;
  const int mt = r % a.mtiles;
  r /= a.mtiles;
  const int hkv = r % a.Hkv;
  const int s = r / a.Hkv;
  const int sid = a.seg_ids ? a.seg_ids[s] : s;
  const int qrow0 = a.cu_q[sid];
  const int Lq = a.cu_q[sid + 1] - qrow0;
  const int krow0 = a.cu_k[sid];
  const int Lk = a.cu_k[sid + 1] - krow0;
  const int g = a.g;
  const int M = Lq * g;
  const int m_base = mt * BM;
  if (m_base >= M) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lrow = lane & 31;
  const int hl = lane >> 5;

  const uint32_t kS = (uint32_t)(a.k_stride * 2), vS = (uint32_t)(a.v_stride * 2);
  const __amdgpu_buffer_rsrc_t krs =
      make_rsrc(a.k + (int64_t)krow0 * a.k_stride + hkv * HD, Lk > 0 ? (uint32_t)(Lk - 1) * kS + HD * 2 : 0u);
  const __amdgpu_buffer_rsrc_t vrs =
      make_rsrc(a.v + (int64_t)krow0 * a.v_stride + hkv * HD, Lk > 0 ? (uint32_t)(Lk - 1) * vS + HD * 2 : 0u);
  DenseAddr ad;
  dense_addr(ad, lane, kS, vS);

  // DMA instruction j (global index q = DMA_PER_WAVE*wave + j) covers tile rows 4q..4q+3.
  auto issue = [&](uint8_t* stage, int k0) {
#pragma unroll
    for (int j = 0; j < DMA_PER_WAVE; ++j) {
      const int q = DMA_PER_WAVE * wave + j;
      const uint32_t row = (uint32_t)(k0 + 4 * q);
      dma16(krs, stage + q * 1024, row * kS + (ad.kdma ^ (uint32_t)(64 * (q & 3))));
      dma16(vrs, stage + DK_TILE * 256 + q * 1024, row * vS + ad.vdma);
    }
  };

  const int ntiles = (Lk + DK_TILE - 1) / DK_TILE;
#pragma unroll
  for (int j = 0; j < ST - 1; ++j)
    if (j < ntiles) issue(lds + j * DK_STAGE_BYTES, j * DK_TILE);

  // Q^T fragments; rows past the segment read as zero through the buffer bound.
  bf16x8_t qf[NQ][8];
  int tokq[NQ], headq[NQ];
  bool okq[NQ];
  {
    const uint32_t qS = (uint32_t)(a.q_stride * 2);
    const uint32_t qbytes = Lq > 0 ? (uint32_t)Lq * qS : 0u;
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(a.q + (int64_t)qrow0 * a.q_stride, qbytes);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int m = m_base + (wave * NQ + q) * 32 + lrow;
      okq[q] = m < M;
      tokq[q] = okq[q] ? m / g : 0;
      headq[q] = hkv * g + (okq[q] ? m - tokq[q] * g : 0);
      const uint32_t qoff = okq[q] ? (uint32_t)tokq[q] * qS + (uint32_t)(headq[q] * HD + hl * 8) * 2u : qbytes;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) qf[q][kk] = as_bf16x8(bload(qrs, qoff + (uint32_t)kk * 32u, 0u));
    }
  }

  DenseState<NQ> st;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) st.oacc[q][db][i] = 0.f;
    st.m_run[q] = -INFINITY;
    st.l_run[q] = 0.f;
  }
  const float c = a.scale_log2;

  // Full tiles, the next tile's DMA in flight; the last tile is peeled off
  // (masked) so the loop body holds a single tile variant.
  // Tile t lives in stage t % ST.  At the top of iteration t this wave's DMA
  // of tiles t+1 .. t+ST-2 may still be in flight (ST-2 tiles of DMA_TILE
  // instructions); the barrier then makes everyone's DMA of tile t visible
  // and frees stage (t-1) % ST, which receives tile t+ST-1.
  for (int t = 0; t + 1 < ntiles; ++t) {
    if (t + ST - 2 < ntiles) vm_wait<(ST - 2) * DMA_TILE>(); else vm_wait<0>();
    __syncthreads();
    uint8_t* cur = lds + (t % ST) * DK_STAGE_BYTES;
    if (t + ST - 1 < ntiles) issue(lds + ((t + ST - 1) % ST) * DK_STAGE_BYTES, (t + ST - 1) * DK_TILE);
    dense_tile<NQ, false>(cur, cur + DK_TILE * 256, ad, qf, st, c, DK_TILE);
  }
  if (ntiles > 0) {
    const int t = ntiles - 1;
    vm_wait<0>();
    __syncthreads();
    uint8_t* cur = lds + (t % ST) * DK_STAGE_BYTES;
    dense_tile<NQ, true>(cur, cur + DK_TILE * 256, ad, qf, st, c, Lk - t * DK_TILE);
  }

#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const float l_tot = st.l_run[q] + __shfl_xor(st.l_run[q], 32);
    if (okq[q]) {
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      uint16_t* op = a.o + (int64_t)(qrow0 + tokq[q]) * a.o_stride + headq[q] * HD;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = db * 32 + 8 * rq + 4 * hl;
          u32x2_t w;
          w[0] = cvt_pk_bf16(st.oacc[q][db][4 * rq + 0] * inv, st.oacc[q][db][4 * rq + 1] * inv);
          w[1] = cvt_pk_bf16(st.oacc[q][db][4 * rq + 2] * inv, st.oacc[q][db][4 * rq + 3] * inv);
          *reinterpret_cast<u32x2_t*>(op + d) = w;
        }
    }
  }
}

// Merge the n_split partial records of every (segment, head, M row).
// grid: (n_seg*Hkv*mtiles*32) rows / 2 per block; block 256 = 2 rows x 128 d.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int row_rec = blockIdx.x * 2 + (threadIdx.x >> 7);  // (s, hkv, mt, q) flattened
  const int d = threadIdx.x & 127;
  const int total_rows = a.n_seg * a.Hkv * a.mtiles * 32;
  if (row_rec >= total_rows) return;
  const int q = row_rec & 31;
  int r = row_rec >> 5;
  const int mt = r % a.mtiles;
  r /= a.mtiles;
  const int hkv = r % a.Hkv;
  const int s = r / a.Hkv;
  const int sid = a.seg_ids ? a.seg_ids[s] : s;
  const int qrow0 = a.cu_q[sid];
  const int Lq = a.cu_q[sid + 1] - qrow0;
  const int g = a.g;
  const int mrow = mt * 32 + q;
  if (mrow >= Lq * g) return;
  const int64_t nrec = (int64_t)a.n_seg * a.Hkv * a.mtiles * a.n_split;
  const int64_t P0 = (((int64_t)s * a.Hkv + hkv) * a.mtiles + mt) * a.n_split;
  const float* ml = a.ws + nrec * 32 * HD;
  float mx = -INFINITY;
  for (int sp = 0; sp < a.n_split; ++sp) mx = fmaxf(mx, ml[((P0 + sp) * 32 + q) * 2]);
  const float mu = (mx == -INFINITY) ? 0.f : mx;
  float l = 0.f, acc = 0.f;
  for (int sp = 0; sp < a.n_split; ++sp) {
    const float* rec = ml + ((P0 + sp) * 32 + q) * 2;
    const float w = (rec[0] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(rec[0] - mu);
    l += rec[1] * w;
    acc += a.ws[((P0 + sp) * 32 + q) * HD + d] * w;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int tq = mrow / g;
  const int hq = hkv * g + (mrow - tq * g);
  a.o[(int64_t)(qrow0 + tq) * a.o_stride + hq * HD + d] = (uint16_t)f32_to_bf16_bits(acc * inv);
}

static const float kLog2e = 1.4426950408889634f;

// K3a launch shapes (one query block of 32 rows per wavefront, two LDS
// stages): 4 wavefronts (128 M rows) for short segments, 8 wavefronts
// (256 M rows sharing each K/V tile) once a segment has >= 1024 M rows.
constexpr int DENSE_ST = 2;
constexpr int DENSE_LONG_M = 1024;
// K3b: 1 x 32 M rows, 128-key tiles split over 4 wavefronts.
using CachedCfg = Cfg<1, 4, 1>;

static int common_checks(const char* name, const void* q, const void* k, const void* v, const void* o, int Hq,
                         int Hkv, int D, int64_t qs, int64_t ks, int64_t vs, int64_t os) {
  if (D != HD) return fail(DLLM_ERR_UNSUPPORTED, "%s: head_dim %d not supported (this build handles 128)", name, D);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
    return fail(DLLM_ERR_INVALID_ARG, "%s: Hq=%d must be a positive multiple of Hkv=%d", name, Hq, Hkv);
  if (!q || !k || !v || !o) return fail(DLLM_ERR_INVALID_ARG, "%s: null tensor pointer", name);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(DLLM_ERR_INVALID_ARG, "%s: q/k/v/o must be 16-byte aligned", name);
  if (qs % 8 || ks % 8 || vs % 8 || os % 8)
    return fail(DLLM_ERR_INVALID_ARG, "%s: token strides must be multiples of 8 elements", name);
  if (qs < (int64_t)Hq * D || os < (int64_t)Hq * D || ks < (int64_t)Hkv * D || vs < (int64_t)Hkv * D)
    return fail(DLLM_ERR_INVALID_ARG, "%s: token stride smaller than a token row", name);
  return DLLM_OK;
}

// Raise a kernel's dynamic-LDS limit (once per kernel and device).
template <typename KernelFn>
static int set_lds(KernelFn fn, int bytes, const char* name) {
  static thread_local const void* done[16];
  static thread_local int done_dev[16];
  static thread_local int n_done = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const void* key = reinterpret_cast<const void*>(fn);
  for (int i = 0; i < n_done; ++i)
    if (done[i] == key && done_dev[i] == dev) return DLLM_OK;
  hipError_t e = hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return fail(DLLM_ERR_HIP, "%s: hipFuncSetAttribute(LDS %d B): %s", name, bytes, hipGetErrorString(e));
  if (n_done < 16) {
    done[n_done] = key;
    done_dev[n_done] = dev;
    ++n_done;
  }
  return DLLM_OK;
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_attn_varlen_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                                    const int32_t* cu_q, const int32_t* cu_k, const int32_t* seg_ids, int n_seg,
                                    int max_seqlen_q, int max_seqlen_k, int Hq, int Hkv, int D, int64_t q_stride_tok,
                                    int64_t k_stride_tok, int64_t v_stride_tok, int64_t o_stride_tok,
                                    float softmax_scale, void* stream) {
  const char* name = "dllm_attn_varlen_fwd";
  int rc = common_checks(name, q, k, v, o, Hq, Hkv, D, q_stride_tok, k_stride_tok, v_stride_tok, o_stride_tok);
  if (rc) return rc;
  if (n_seg < 0 || max_seqlen_q < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative n_seg / max_seqlen_q", name);
  if (n_seg == 0 || max_seqlen_q == 0) return DLLM_OK;
  if (!cu_q || !cu_k) return fail(DLLM_ERR_INVALID_ARG, "%s: null cu_seqlens", name);
  if (max_seqlen_k < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative max_seqlen_k", name);
  {
    // per-segment byte offsets are 32-bit (buffer loads)
    const int64_t kvs = k_stride_tok > v_stride_tok ? k_stride_tok : v_stride_tok;
    if ((int64_t)max_seqlen_k * kvs * 2 + 4096 >= ((int64_t)1 << 32) ||
        (int64_t)max_seqlen_q * q_stride_tok * 2 + 4096 >= ((int64_t)1 << 32))
      return fail(DLLM_ERR_UNSUPPORTED, "%s: a segment spans more than 4 GiB of q/k/v", name);
  }
  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.cu_q = cu_q; a.cu_k = cu_k; a.seg_ids = seg_ids;
  a.q_stride = q_stride_tok; a.k_stride = k_stride_tok; a.v_stride = v_stride_tok; a.o_stride = o_stride_tok;
  a.n_seg = n_seg; a.Hkv = Hkv; a.g = Hq / Hkv;
  const bool wide = (int64_t)max_seqlen_q * a.g >= DENSE_LONG_M;
  const int nw = wide ? 8 : 4;
  const int bm = 32 * nw;
  a.mtiles = (int)(((int64_t)max_seqlen_q * a.g + bm - 1) / bm);
  a.n_split = 1;
  const int64_t logical = (int64_t)a.mtiles * Hkv * n_seg;
  if (logical > (int64_t)1 << 30) return fail(DLLM_ERR_INVALID_ARG, "%s: problem too large", name);
  a.logical_blocks = (int)logical;
  a.scale_log2 = softmax_scale * kLog2e;
  auto kern = wide ? attn_dense_kernel<8, 1, DENSE_ST> : attn_dense_kernel<4, 1, DENSE_ST>;
  constexpr int lds_bytes = DENSE_ST * DK_STAGE_BYTES;
  if ((rc = set_lds(kern, lds_bytes, name))) return rc;
  const int nb = (int)((logical + 7) / 8 * 8);
  kern<<<dim3(nb), dim3(64 * nw), lds_bytes, reinterpret_cast<hipStream_t>(stream)>>>(a);
  return check_launch(name);
}

static int block_cached_plan(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int& mtiles, int& n_split,
                             int& keys_per_split) {
  const int g = Hq / Hkv;
  mtiles = (max_q * g + 31) / 32;
  const int64_t pairs = (int64_t)n_seg * Hkv * mtiles;
  // Aim for >= 2 workgroups per CU (256 CUs) with at least two 128-key tiles per split.
  int64_t want = pairs > 0 ? (512 + pairs - 1) / pairs : 1;
  const int max_split = max_keys > 0 ? (max_keys + 255) / 256 : 1;
  if (want > max_split) want = max_split;
  if (want < 1) want = 1;
  n_split = (int)want;
  const int tiles = (max_keys + CachedCfg::NKT - 1) / CachedCfg::NKT;
  const int tiles_per_split = (tiles + n_split - 1) / n_split;
  keys_per_split = tiles_per_split * CachedCfg::NKT;
  if (keys_per_split <= 0) keys_per_split = CachedCfg::NKT;
  n_split = max_keys > 0 ? (max_keys + keys_per_split - 1) / keys_per_split : 1;
  return 0;
}

extern "C" size_t dllm_attn_block_cached_workspace_size(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int D) {
  (void)D;
  if (n_seg <= 0 || max_q <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv) return 0;
  int mtiles, n_split, kps;
  block_cached_plan(n_seg, max_q, max_keys, Hq, Hkv, mtiles, n_split, kps);
  if (n_split <= 1) return 0;
  const size_t nrec = (size_t)n_seg * Hkv * mtiles * n_split;
  return nrec * 32 * (HD + 2) * sizeof(float);
}

extern "C" int dllm_attn_block_cached_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                                          const int32_t* cu, const int32_t* seg_ids, int n_seg, int max_q,
                                          int max_keys, const dllm_bf16* k_cache, const dllm_bf16* v_cache,
                                          int64_t cache_slots, const int32_t* slots, const int32_t* slot_off,
                                          int Hq, int Hkv, int D, int64_t q_stride_tok, int64_t k_stride_tok,
                                          int64_t v_stride_tok, int64_t o_stride_tok, float softmax_scale,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  const char* name = "dllm_attn_block_cached_fwd";
  int rc = common_checks(name, q, k, v, o, Hq, Hkv, D, q_stride_tok, k_stride_tok, v_stride_tok, o_stride_tok);
  if (rc) return rc;
  if (n_seg < 0 || max_q < 0 || max_keys < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (n_seg == 0 || max_q == 0) return DLLM_OK;
  if (!cu || !slot_off) return fail(DLLM_ERR_INVALID_ARG, "%s: null cu / slot_off", name);
  if ((int64_t)max_q * q_stride_tok * 2 + 4096 >= ((int64_t)1 << 32))
    return fail(DLLM_ERR_UNSUPPORTED, "%s: a block spans more than 4 GiB of q", name);
  if (cache_slots > 0 && (!k_cache || !v_cache || !slots))
    return fail(DLLM_ERR_INVALID_ARG, "%s: null cache / slots", name);
  if (cache_slots > 0 && (!aligned16(k_cache) || !aligned16(v_cache)))
    return fail(DLLM_ERR_INVALID_ARG, "%s: caches must be 16-byte aligned", name);
  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slots = cache_slots;
  a.cu_q = cu; a.cu_k = cu; a.seg_ids = seg_ids; a.slots = slots; a.slot_off = slot_off;
  a.q_stride = q_stride_tok; a.k_stride = k_stride_tok; a.v_stride = v_stride_tok; a.o_stride = o_stride_tok;
  a.n_seg = n_seg; a.Hkv = Hkv; a.g = Hq / Hkv;
  int mtiles, n_split, kps;
  block_cached_plan(n_seg, max_q, max_keys, Hq, Hkv, mtiles, n_split, kps);
  a.mtiles = mtiles; a.n_split = n_split; a.keys_per_split = kps;
  if (n_split > 1) {
    const size_t need = dllm_attn_block_cached_workspace_size(n_seg, max_q, max_keys, Hq, Hkv, D);
    if (!workspace || workspace_bytes < need)
      return fail(DLLM_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", name, need,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(DLLM_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", name);
    a.ws = reinterpret_cast<float*>(workspace);
  }
  const int64_t logical = (int64_t)n_split * mtiles * Hkv * n_seg;
  if (logical > (int64_t)1 << 30) return fail(DLLM_ERR_INVALID_ARG, "%s: problem too large", name);
  a.logical_blocks = (int)logical;
  a.scale_log2 = softmax_scale * kLog2e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto kern = attn_fwd_kernel<1, 4, 1, true>;
  if ((rc = set_lds(kern, CachedCfg::LDS_BYTES, name))) return rc;
  const int nb = (int)((logical + 7) / 8 * 8);
  kern<<<dim3(nb), dim3(256), CachedCfg::LDS_BYTES, st>>>(a);
  if ((rc = check_launch(name))) return rc;
  if (n_split > 1) {
    const int64_t rows = (int64_t)n_seg * Hkv * mtiles * 32;
    attn_combine_kernel<<<dim3((unsigned)((rows + 1) / 2)), dim3(256), 0, st>>>(a);
    if ((rc = check_launch(name))) return rc;
  }
  return DLLM_OK;
}

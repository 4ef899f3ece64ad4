// K3a / K3b: bidirectional attention on gfx950 bf16 MFMA.
//
//   * K3a attn_dense_kernel (dense varlen, cache states 0/1): a workgroup of
//     NW wavefronts owns NW*32 "M rows" of one segment and one KV head and
//     streams the segment's keys through LDS in tiles.
//   * K3b attn_cached_kernel (generation block vs cached KV, state 2): a
//     workgroup owns 32 M rows; each of its 4 wavefronts takes 32 keys of
//     every 128-key tile and the four states are merged in LDS at the end;
//     long key ranges are also split across workgroups (partials in a
//     workspace, merged by attn_combine_kernel).
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
// operand and in P^T (a contraction is invariant under a permutation of its
// summation index), which makes every operand fetch a single LDS read.
#include "common.h"

#include <math.h>

#include <mutex>
#include <type_traits>

namespace dllm {

constexpr int HD = 128;       // the head dim these kernels handle

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
  int xcd_chunk;      // logical blocks per chunk of the XCD interleave (grid = multiple of 8 * xcd_chunk)
  float scale_log2;
};

// Work-groups are dispatched round-robin over the 8 XCDs (XCD = b % 8), and
// each XCD has its own L2.  Logical blocks are dealt to the XCDs in chunks of
// `ch` consecutive ones, chunk j to XCD j % 8, so the blocks of a chunk (the
// m-tiles of one (segment, head), which read the same K/V) share an L2, while
// every XCD gets an even share of every part of the batch.  Handing each XCD
// one contiguous eighth instead left ragged batches unbalanced: with 16
// segments of 410..1245 tokens the busiest XCD held 1.6x the mean work
// (those 16 segments, 28 query / 4 KV heads: 226 -> 172 us with chunks of
// 4).  The grid must be a multiple of 8 * ch; the map is then a bijection
// onto [0, grid).
__device__ __forceinline__ int xcd_remap(int b, int ch) {
  const int x = b & 7, i = b >> 3;
  const int j = i / ch;
  return (j * 8 + x) * ch + (i - j * ch);
}


// Running softmax state of one wavefront (M row = lane % 32).  The reference
// maximum m_run (log2 domain) is only raised when a new score exceeds it by
// more than kLazy, so most tiles skip rescaling O; probabilities then stay
// below 2^kLazy, well inside the bf16 / fp32 range.
constexpr float kLazy = 8.0f;

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
// (the XOR acts on the chunk offset alone, the row offset is added after it)
struct DenseAddr {
  uint32_t kbase, vbase;
  uint32_t kdma_row, kdma_chunk, vdma;
};

__device__ __forceinline__ void dense_addr(DenseAddr& ad, int lane, uint32_t kS, uint32_t vS) {
  const int rl = lane >> 4, P = lane & 15;
  ad.kdma_row = (uint32_t)rl * kS;
  ad.kdma_chunk = (uint32_t)((P ^ rl) * 16);
  ad.vdma = (uint32_t)rl * vS + (uint32_t)((P ^ (4 * rl)) * 16);
  const int lrow = lane & 31, hl = lane >> 5;
  ad.kbase = (uint32_t)(lrow * 256 + ((hl ^ (lrow & 15)) * 16));
  const int dhalf = (lane >> 4) & 1, k = (lane & 15) >> 2, c = lane & 3;
  ad.vbase = (uint32_t)((4 * hl + k) * 256 + (4 * k + 2 * dhalf + (c >> 1)) * 16 + 8 * (c & 1));
}

// Softmax state of NQ query blocks (32 M rows each) of one wavefront.
// thr = m_run + kLazy and neg_m = -m_run (0 while m_run is -inf) change only
// when m_run does, so the per-tile test and exponent need no extra VALU work.
template <int NQ>
struct DenseState {
  f32x16_t oacc[NQ][4];
  float m_run[NQ];
  float l_run[NQ];
  float thr[NQ];
  float neg_m[NQ];
};

template <int NQ>
__device__ __forceinline__ void dense_state_init(DenseState<NQ>& st) {
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) st.oacc[q][db][i] = 0.f;
    st.m_run[q] = -INFINITY;
    st.l_run[q] = 0.f;
    st.thr[q] = -INFINITY;
    st.neg_m[q] = 0.f;
  }
}

// Online-softmax update of one query block from its two S^T key blocks;
// returns the packed P^T fragments (B operands of O^T += V^T P^T).
template <int KB, bool MASK>
__device__ __forceinline__ void dense_softmax(f32x16_t (&sacc)[KB], f32x16_t (&oacc)[4], float& m_run, float& l_run,
                                              float& thr, float& neg_m, bf16x8_t (&pf)[2 * KB], float c, int k_valid,
                                              uint64_t bad, int hl) {
  float mx = -INFINITY;
#pragma unroll
  for (int b = 0; b < KB; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (MASK) {
        const int key = b * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (key >= k_valid || ((bad >> key) & 1ull)) sacc[b][i] = -INFINITY;
      }
      mx = fmaxf(mx, sacc[b][i]);
    }
  mx = pair_max32(mx) * c;
  const bool need = mx > thr;
  if (__builtin_amdgcn_ballot_w64(need)) {
    const float m_new = need ? mx : m_run;
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
    m_run = m_new;
    thr = m_run + kLazy;
    neg_m = (m_run == -INFINITY) ? 0.f : -m_run;
  }
  // The row sum adds the bf16-rounded numerators, the same values the O^T
  // product consumes; two partial sums (one starting from l_run) keep the
  // dependent chain short.
  float psum[2] = {l_run, 0.f};
#pragma unroll
  for (int b = 0; b < KB; ++b)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4_t pk;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][8 * j + 2 * w], c, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[b][8 * j + 2 * w + 1], c, neg_m));
        pk[w] = cvt_pk_bf16(p0, p1);
        psum[w & 1] = add_bf16x2(pk[w], psum[w & 1]);
      }
      pf[2 * b + j] = as_bf16x8(pk);
    }
  l_run = psum[0] + psum[1];
}

// One key tile (TK keys) for one wavefront owning NQ query blocks: every K
// and V^T operand fragment read from LDS feeds NQ MFMAs.
// V^T operands of one 32-key block for callers whose tiles arrive by
// global_load_lds: the compiler makes every transposing-read builtin wait for
// all such DMA still in flight (it cannot tell the tiles apart), which would
// drain the next tile's prefetch.  The 16 reads are one asm block that ends
// with its own lgkmcnt(0) wait, so its outputs are complete when it returns.
// Read (c, d, h) -- key chunk c, d block d, half h -- is at
// vbase ^ 64 d + 4096 c + 2048 h; output index (4 c + d) * 2 + h.
__device__ __forceinline__ void v_operands_untracked(const uint8_t* Vs, const DenseAddr& ad, u32x2_t (&r)[16]) {
  uint32_t b[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    b[d] = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)(Vs + (ad.vbase ^ (uint32_t)(64 * d)));
  asm volatile(
      "ds_read_b64_tr_b16 %0, %16\n"
      "ds_read_b64_tr_b16 %1, %16 offset:2048\n"
      "ds_read_b64_tr_b16 %2, %17\n"
      "ds_read_b64_tr_b16 %3, %17 offset:2048\n"
      "ds_read_b64_tr_b16 %4, %18\n"
      "ds_read_b64_tr_b16 %5, %18 offset:2048\n"
      "ds_read_b64_tr_b16 %6, %19\n"
      "ds_read_b64_tr_b16 %7, %19 offset:2048\n"
      "ds_read_b64_tr_b16 %8, %16 offset:4096\n"
      "ds_read_b64_tr_b16 %9, %16 offset:6144\n"
      "ds_read_b64_tr_b16 %10, %17 offset:4096\n"
      "ds_read_b64_tr_b16 %11, %17 offset:6144\n"
      "ds_read_b64_tr_b16 %12, %18 offset:4096\n"
      "ds_read_b64_tr_b16 %13, %18 offset:6144\n"
      "ds_read_b64_tr_b16 %14, %19 offset:4096\n"
      "ds_read_b64_tr_b16 %15, %19 offset:6144\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7]),
        "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]), "=&v"(r[12]), "=&v"(r[13]), "=&v"(r[14]),
        "=&v"(r[15])
      : "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3])
      : "memory");
}

template <int NQ, int TK, bool MASK, bool UNTRACKED_V = false>
__device__ __forceinline__ void dense_tile(const uint8_t* Ks, const uint8_t* Vs, const DenseAddr& ad,
                                           const bf16x8_t (&qf)[NQ][8], DenseState<NQ>& st, float c, int k_valid,
                                           uint64_t bad = 0) {
  constexpr int KB = TK / 32;  // key blocks of 32 per tile
  const int lane = threadIdx.x & 63;
  const int hl = lane >> 5;
  // kk outer, key block inner: the KB*NQ accumulators form independent MFMA
  // chains that interleave instead of one chain waiting on itself.  Each
  // S^T block is one chain over the head dimension: the wavefronts sharing
  // a SIMD interleave their chains, and splitting the reduction over two
  // partial accumulators (to lengthen the chain count) costs 16 VALU adds per
  // tile to merge them -- 2-5 % slower at every measured shape, since the
  // softmax VALU work rivals the MFMA work.
  f32x16_t sacc[NQ][KB];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[q][b][i] = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      const bf16x8_t af =
          as_bf16x8(*reinterpret_cast<const u32x4_t*>(Ks + b * 32 * 256 + (ad.kbase ^ (uint32_t)(32 * kk))));
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        sacc[q][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[q][kk], sacc[q][b], 0, 0, 0);
    }
  }
  bf16x8_t pf[NQ][2 * KB];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    dense_softmax<KB, MASK>(sacc[q], st.oacc[q], st.m_run[q], st.l_run[q], st.thr[q], st.neg_m[q], pf[q], c, k_valid,
                            bad, hl);
  if constexpr (UNTRACKED_V) {
    static_assert(KB == 1, "one 32-key block per call");
    u32x2_t r[16];
    v_operands_untracked(Vs, ad, r);
#pragma unroll
    for (int cch = 0; cch < 2; ++cch)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const u32x2_t lo = r[(4 * cch + db) * 2], hi = r[(4 * cch + db) * 2 + 1];
        const bf16x8_t af = as_bf16x8(u32x4_t{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          st.oacc[q][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, pf[q][cch], st.oacc[q][db], 0, 0, 0);
      }
    return;
  }
  // key chunk outer, d block inner: 4*NQ independent accumulator chains.
#pragma unroll
  for (int cch = 0; cch < 2 * KB; ++cch) {
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
template <int NW, int NQ, int ST, int TK, int OCC>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void attn_dense_kernel(AttnArgs a) {
  constexpr int BM = 32 * NW * NQ;
  constexpr int STAGE = 2 * TK * 256;                      // K + V tile bytes
  constexpr int NDMA = TK * 256 / 1024;                    // 1 KiB DMA instructions per matrix per tile
  constexpr int DMA_PER_WAVE = (NDMA + NW - 1) / NW;       // per wave (waves >= NDMA issue none when NW > NDMA)
  constexpr int DMA_TILE = 2 * DMA_PER_WAVE;               // this wave's DMA instructions per tile, K and V
  static_assert(TK % 32 == 0, "tile shape");
  static_assert(NDMA % NW == 0 || (NW > NDMA && ST == 2), "an uneven DMA split needs the full wait of two stages");
  constexpr bool QDMA = NQ == 1 && NW == 4 * OCC;  // one workgroup per CU
  // The 12-wavefront launch runs one workgroup per (segment, KV head) pair,
  // so its K/V bytes, like every launch's Q rows, are read once: streaming
  // loads for them (C2 step 27.7 -> 27.2 us).  The other launches share a
  // pair's K/V between the workgroups of its m-tiles and keep the default.
  constexpr int KV_AUX = NW == 12 ? kStreamAux : 0;
  constexpr int QOFF = ST * STAGE;                 // Q rows after the K/V stages (NW * 8 KiB)
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int L = xcd_remap(blockIdx.x, a.xcd_chunk);
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
  const uint16_t* kseg = a.k + (int64_t)krow0 * a.k_stride + hkv * HD;
  const uint16_t* vseg = a.v + (int64_t)krow0 * a.v_stride + hkv * HD;
  DenseAddr ad;
  dense_addr(ad, lane, kS, vS);

  // DMA instruction j (global index q = DMA_PER_WAVE*wave + j, or q = wave
  // when there are more wavefronts than instructions) covers tile rows 4q..4q+3.
  // Each tile gets buffer resources based at its first row (scalar work), so
  // the per-lane offsets are the same for every tile and no VALU work is
  // spent per tile; rows past the segment's last still read as zero.
  auto issue = [&](uint8_t* stage, int k0) {
    const uint32_t rows_left = (uint32_t)(Lk - 1 - k0);  // k0 < Lk: only tiles that exist are issued
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kseg + (int64_t)k0 * a.k_stride, rows_left * kS + HD * 2);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vseg + (int64_t)k0 * a.v_stride, rows_left * vS + HD * 2);
#pragma unroll
    for (int j = 0; j < DMA_PER_WAVE; ++j) {
      const int q = NW > NDMA ? wave : DMA_PER_WAVE * wave + j;
      if (q >= NDMA) break;  // wave-uniform
      const uint32_t row = (uint32_t)(4 * q);
      // the swizzle XOR applies to the chunk only: with a token stride that
      // is not a multiple of 256 bytes, XOR-ing rl * kS + chunk would carry
      // into the row offset
      dma16<KV_AUX>(krs, stage + q * 1024, row * kS + ad.kdma_row + (ad.kdma_chunk ^ (uint32_t)(64 * (q & 3))));
      dma16<KV_AUX>(vrs, stage + TK * 256 + q * 1024, row * vS + ad.vdma);
    }
  };

  const int ntiles = (Lk + TK - 1) / TK;
#pragma unroll
  for (int j = 0; j < ST - 1; ++j)
    if (j < ntiles) issue(lds + j * STAGE, j * TK);

  // Q^T fragments; rows past the segment read as zero through the buffer bound.
  // A workgroup that owns its CU (NW == 4 * OCC) has LDS to spare: its Q rows
  // are DMA'd in whole 256-byte rows (4 rows per instruction, the K tile's
  // swizzle) and the fragments read back like K operands.  Otherwise every
  // load instruction carries 32-byte pieces of 32 rows straight to VGPRs.
  bf16x8_t qf[NQ][8];
  int tokq[NQ], headq[NQ];
  bool okq[NQ];
  {
    const uint32_t qS = (uint32_t)(a.q_stride * 2);
    const uint32_t qbytes = Lq > 0 ? (uint32_t)Lq * qS : 0u;
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(a.q + (int64_t)qrow0 * a.q_stride, qbytes);
    if constexpr (QDMA) {
      // instruction j, lane L: row R = 4j + L/16 of this wave's 32, physical
      // chunk L%16 = logical chunk (L%16) ^ (R & 15)
      const int rl = lane >> 4, P = lane & 15;
      const int m0 = m_base + wave * 32 + rl;
      int tok = m0 / g, rem = m0 - tok * g;
      const int q4 = 4 / g, r4 = 4 - q4 * g;  // m advances by 4 per instruction
      uint8_t* qdst = lds + QOFF + wave * 8192;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int R = 4 * j + rl;
        const uint32_t off = m0 + 4 * j < M
                                 ? (uint32_t)tok * qS + (uint32_t)((hkv * g + rem) * HD * 2) +
                                       (uint32_t)((P ^ (R & 15)) * 16)
                                 : qbytes;
        dma16<kStreamAux>(qrs, qdst + j * 1024, off);
        tok += q4;
        rem += r4;
        if (rem >= g) {
          rem -= g;
          ++tok;
        }
      }
      okq[0] = m_base + wave * 32 + lrow < M;
      tokq[0] = 0;
      headq[0] = 0;
    } else {
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
  }
  if constexpr (QDMA) {
    vm_wait<0>();  // this wave's Q rows and its share of tile 0
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[0][kk] = as_bf16x8(
          *reinterpret_cast<const u32x4_t*>(lds + QOFF + wave * 8192 + (ad.kbase ^ (uint32_t)(32 * kk))));
  }

  DenseState<NQ> st;
  dense_state_init(st);
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
    uint8_t* cur = lds + (t % ST) * STAGE;
    if (t + ST - 1 < ntiles) issue(lds + ((t + ST - 1) % ST) * STAGE, (t + ST - 1) * TK);
    dense_tile<NQ, TK, false>(cur, cur + TK * 256, ad, qf, st, c, TK);
  }
  if (ntiles > 0) {
    const int t = ntiles - 1;
    vm_wait<0>();
    __syncthreads();
    uint8_t* cur = lds + (t % ST) * STAGE;
    dense_tile<NQ, TK, true>(cur, cur + TK * 256, ad, qf, st, c, Lk - t * TK);
  }

  if constexpr (NQ == 1) {
    // O goes through LDS so that every global store writes whole 256-byte
    // rows: lane (lrow, hl) holds, per d block db and quad rq, d = 32 db +
    // 8 rq + 4 hl + 0..3, i.e. half hl of 16-byte chunk 4 db + rq of its row.
    // The wave's 32 rows x 256 bytes land in its own 8 KiB of the (now free)
    // K/V stages, chunks XOR-swizzled by row; read back, instruction j
    // carries rows 4j .. 4j+3, one 16-byte chunk per lane.
    // O staging needs NW * 8 KiB (the Q rows, or the front of LDS); the launch gives at least that
    const float l_tot = pair_sum32(st.l_run[0]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    // With Q by DMA a wavefront stages O in its own Q rows, which no other
    // wavefront reads, so it stores as soon as it is done; otherwise in the
    // K/V stages once every wavefront is done reading them.
    uint8_t* ot;
    if constexpr (QDMA) {
      ot = lds + QOFF + wave * 8192;
    } else {
      __syncthreads();
      ot = lds + wave * 8192;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        u32x2_t w;
        w[0] = cvt_pk_bf16(st.oacc[0][db][4 * rq + 0] * inv, st.oacc[0][db][4 * rq + 1] * inv);
        w[1] = cvt_pk_bf16(st.oacc[0][db][4 * rq + 2] * inv, st.oacc[0][db][4 * rq + 3] * inv);
        const int chunk = 4 * db + rq;
        *reinterpret_cast<u32x2_t*>(ot + lrow * 256 + ((chunk ^ (lrow & 15)) * 16) + 8 * hl) = w;
      }
    const int rsub = lane >> 4, ch = lane & 15;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * j + rsub;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ot + r * 256 + ((ch ^ (r & 15)) * 16));
      const int m = m_base + wave * 32 + r;
      if (m < M) {
        const int tok = m / g;
        const int head = hkv * g + (m - tok * g);
        st128(a.o + (int64_t)(qrow0 + tok) * a.o_stride + head * HD + ch * 8, v);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const float l_tot = pair_sum32(st.l_run[q]);
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
}

// ---------------------------------------------------------------------------
// K3b: block rows vs [cached rows (by slot) ; block rows], with the swizzled
// LDS tile layout of K3a.  Tile = 128 keys; wavefront w DMAs tile rows
// 32w..32w+31 (8 K + 8 V instructions, per-lane 64-bit addresses so caches
// above 4 GiB work) and computes exactly those 32 keys for the workgroup's 32
// M rows; the four wavefronts' softmax states are merged in LDS at the end.
// A cached row whose slot is outside the cache is excluded (masked) from the
// softmax.
constexpr int CK_TILE = 128;
constexpr int CK_STAGE = 2 * CK_TILE * 256;
// LDS of the kernel with RB row blocks: two stages and the slot ring
// ([4 tiles][4 RB wavefronts][64] words); the final merge reuses both
constexpr int ck_lds_bytes(int rb) { return 2 * CK_STAGE + 4 * 4 * rb * 64 * 4; }

// Cache and block rows of a segment are read by exactly one workgroup, each
// 16-byte piece by one lane of one DMA instruction: streaming loads (the q
// loads keep the default policy: a lane reads each q line in four 32-byte
// steps and relies on the cache between them).
__device__ __forceinline__ void gdma16(const void* g, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_dst, 16, 0, kStreamAux);
}

// The four wavefronts' softmax states of one row block (each holds the same
// 32 M rows over its own keys) merged, normalised and written to o -- or,
// when the keys are split across workgroups, written as a partial record
// for attn_combine_kernel.  Every thread of the workgroup calls it once (it
// holds workgroup barriers).  The four wavefronts of a row block park their
// unscaled O^T partials as [row][d] f32 in 32 rows x 2 x 256 bytes of a
// stage (d 0..63 in the K rows, 64..127 in the V rows of their key block;
// 16-byte chunk c of a row at c ^ (row & 15),
// so that 16 lanes on 16 rows hit 16 different chunks), and their row maxima
// and sums in the idle slot ring.  Row block 0 uses the stage the last tile
// did not use, free once every wavefront has passed the last tile's first
// barrier (with RB = 1 a wavefront only ever reads its own rows, so at once);
// row block 1 uses the last tile's stage after one more barrier.  Then thread
// (row q, d0 .. d0 + 15) of each row block merges its four partials,
// wavefronts in order, each scaled term (and each term of the row sum)
// rounded before it is added.
template <int RB>
__device__ __forceinline__ void cached_merge_store(const AttnArgs& a, uint8_t* lds, int last_stage, float* ring,
                                                        const DenseState<1>& st, int s, int hkv, int mt, int split,
                                                        int qrow0, int M, int m_base, int g, int tid, int rblk) {
  const int wave = (tid >> 6) & 3;
  const int lane = tid & 63;
  const int lrow = lane & 31;
  const int hl = lane >> 5;
  // piece p of wave w: part + p * CK_TILE * 256 + w * 8 KiB
  uint8_t* part = lds + (rblk == 0 ? last_stage ^ 1 : last_stage) * CK_STAGE;
  float* ml = ring + rblk * 4 * 2 * 32;
  const float l_tot = pair_sum32(st.l_run[0]);
  if (hl == 0) {
    ml[(wave * 2 + 0) * 32 + lrow] = st.m_run[0];
    ml[(wave * 2 + 1) * 32 + lrow] = l_tot;
  }
  auto park = [&]() {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + 8 * rq + 4 * hl;
        uint8_t* row = part + (d >> 6) * CK_TILE * 256 + (wave * 32 + lrow) * 256;
        const f32x4_t v = {st.oacc[0][db][4 * rq], st.oacc[0][db][4 * rq + 1], st.oacc[0][db][4 * rq + 2],
                           st.oacc[0][db][4 * rq + 3]};
        *reinterpret_cast<f32x4_t*>(row + ((((d & 63) >> 2) ^ (lrow & 15)) << 4)) = v;
      }
  };
  if (rblk == 0) park();
  if constexpr (RB > 1) {
    lds_barrier();  // every wavefront is done with the last tile's stage
    if (rblk == 1) park();
  }
  lds_barrier();
  tid &= 255;
  const int q = tid & 31;
  const int d0 = (tid >> 5) * 16;
  float mw[4], mq = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = ml[(w * 2) * 32 + q];
    mq = fmaxf(mq, mw[w]);
  }
  const float mq_use = (mq == -INFINITY) ? 0.f : mq;
  float lq = 0.f;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float f = (mw[w] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw[w] - mq_use);
    lq = __fadd_rn(lq, __fmul_rn(ml[(w * 2 + 1) * 32 + q], f));  // f = 0 for a wavefront without keys
    const uint8_t* row = part + (d0 >> 6) * CK_TILE * 256 + (w * 32 + q) * 256;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(row + (((((d0 & 63) >> 2) + c4) ^ (q & 15)) << 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[4 * c4 + e] = __fadd_rn(acc[4 * c4 + e], __fmul_rn(v[e], f));
    }
  }
  const int mrow = m_base + q;
  if (mrow < M) {
    const int tq = mrow / g;
    const int hq = hkv * g + (mrow - tq * g);
    if (a.n_split == 1) {
      const float inv = lq > 0.f ? 1.f / lq : 0.f;
      uint16_t* op = a.o + (int64_t)(qrow0 + tq) * a.o_stride + hq * HD + d0;
      u32x4_t w0, w1;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        w0[w] = cvt_pk_bf16(acc[2 * w] * inv, acc[2 * w + 1] * inv);
        w1[w] = cvt_pk_bf16(acc[8 + 2 * w] * inv, acc[8 + 2 * w + 1] * inv);
      }
      st128(op, w0);
      st128(op + 8, w1);
    } else {
      const int64_t Prec = (((int64_t)s * a.Hkv + hkv) * a.mtiles + mt) * a.n_split + split;
      float* po = a.ws + (Prec * 32 + q) * HD + d0;
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        f32x4_t v4 = {acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
        *reinterpret_cast<f32x4_t*>(po + i) = v4;
      }
      if (d0 == 0) {  // one writer per row
        const int64_t nrec = (int64_t)a.n_seg * a.Hkv * a.mtiles * a.n_split;
        float* pml = a.ws + nrec * 32 * HD + (Prec * 32 + q) * 2;
        pml[0] = mq;
        pml[1] = lq;
      }
    }
  }
}

// One 32-key block of the four-wavefront K3b: K operands from LDS, keys set in
// `bad` left out of the softmax by a small conditional block (a single
// softmax code path keeps the accumulators in place).
__device__ __forceinline__ void cached_tile(const uint8_t* Ks, const uint8_t* Vs, const DenseAddr& ad,
                                            const bf16x8_t (&qf)[1][8], DenseState<1>& st, float c, uint64_t bad) {
  const int hl = (threadIdx.x & 63) >> 5;
  f32x16_t sacc[1];
#pragma unroll
  for (int i = 0; i < 16; ++i) sacc[0][i] = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        as_bf16x8(*reinterpret_cast<const u32x4_t*>(Ks + (ad.kbase ^ (uint32_t)(32 * kk)))), qf[0][kk], sacc[0], 0, 0, 0);
  if (bad) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = 8 * (i >> 2) + 4 * hl + (i & 3);
      if ((bad >> key) & 1ull) sacc[0][i] = -INFINITY;
    }
  }
  bf16x8_t pf[2];
  dense_softmax<1, false>(sacc, st.oacc[0], st.m_run[0], st.l_run[0], st.thr[0], st.neg_m[0], pf, c, 32, 0, hl);
  // all 16 V^T operands are read (one asm block) before the first product:
  // the MFMAs read their source registers after issue, so no register they
  // use may be rewritten by a later LDS read while they run
  u32x2_t vr[16];
  v_operands_untracked(Vs, ad, vr);
#pragma unroll
  for (int cch = 0; cch < 2; ++cch)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const u32x2_t lo = vr[(4 * cch + db) * 2], hi = vr[(4 * cch + db) * 2 + 1];
      st.oacc[0][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(u32x4_t{lo[0], lo[1], hi[0], hi[1]}), pf[cch],
                                                               st.oacc[0][db], 0, 0, 0);
    }
}

// RB row blocks of 32 M rows of one (segment, KV head) per workgroup, four
// wavefronts each: wavefront w + 4 r computes keys 32 w .. 32 w + 31 of every
// tile for row block r.  With RB = 1 a wavefront DMAs exactly the 32 rows it
// computes and never waits for another one until the merge.  With RB = 2 the
// two row blocks share every tile -- each K/V row is fetched once for 64 M
// rows -- and wavefront w + 4 r DMAs half of those 32 rows (instructions
// 4 r .. 4 r + 3); a workgroup barrier after the wait makes a tile visible
// to both, and one before a stage is refilled retires its last readers.
// Two wavefronts per SIMD as the register budget: the whole state then stays
// in VGPRs (with a budget of 512 the compiler moves the O^T accumulators
// between AGPRs and VGPRs around every softmax rescale).
// PAGED: the cached rows of segment s are given by a page table instead of a
// slot list -- `slot_off` holds cached_len (int32 per segment) and `slots`
// the page table ([n_seg][max_pages] int32 page ids, 256-row pages): cached
// row r sits in cache row page_table[s][r / 256] * 256 + r % 256.  A 128-key
// tile starts at a multiple of 128, so its cached rows lie in one page.  Each
// wavefront DMAs its own copy of the page ids of its key range (up to 64) as
// its first memory operation -- no wavefront waits for another -- so its first
// K/V tiles wait on one round of loads (page ids, offsets and Q together)
// instead of two (slot offsets, then the slot list).
template <int RB, bool PAGED>
// The launch geometry and the tables the first, dependent loads read come as
// leading scalar arguments (14 dwords): the library is built with kernel
// argument preloading, so they are in SGPRs when a wave starts instead of one
// scalar load away (the rest of AttnArgs is loaded as usual).  `slots` is
// null when there is no cache.  `chunk_pages` = XCD chunk (1..16) + 32 x the
// page table's row length (0 in the slot-list form), so that everything the
// page-id fetch needs is preloaded.
__global__ __launch_bounds__(256 * RB) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_cached_kernel(
    const int32_t* __restrict__ slot_off, const int32_t* __restrict__ seg_ids, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ slots, int chunk_pages, int logical_blocks, int mtiles, int n_split, int Hkv,
    int keys_per_split, AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int NJ = 8 / RB;  // K (and V) DMA instructions per wavefront per tile
  const int xcd_chunk = chunk_pages & 31;
  const int max_pages = chunk_pages >> 5;
  const int L = xcd_remap(blockIdx.x, xcd_chunk);
  if (L >= logical_blocks) return;
  const int mblocks = (mtiles + RB - 1) / RB;
  int r = L;
  const int split = r % n_split;
  r /= n_split;
  const int mb = r % mblocks;
  r /= mblocks;
  const int hkv = r % Hkv;
  const int s = r / Hkv;
  const int kbeg0 = split * keys_per_split;  // this split's first key (past Lk: no tiles)
  const int tid = threadIdx.x;
  const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  uint32_t* slot_ring = reinterpret_cast<uint32_t*>(lds + 2 * CK_STAGE);  // [4 tiles][4 RB waves][64]
  // Page-table form: each wavefront's page ids (pg0 .. pg0 + 63 of the
  // segment's row, one per lane; lanes past the row's end read its first id) sit in
  // the upper half of the ring -- the merge at the end parks every row
  // block's m / l in its first 256 RB words while other wavefronts may still
  // read page ids for their last tiles.  Their address needs no load, so the
  // fetch is the kernel's first memory operation and the segment's offsets
  // are loaded behind it.
  const int pg0 = kbeg0 >> 8;
  uint32_t* const page_ring = slot_ring + 512 * RB + wave_id * 64;
  if constexpr (PAGED) {
    if (slots != nullptr && max_pages > 0) {  // else no row has a page: nothing to fetch
      const int32_t* row = slots + (int64_t)s * max_pages;
      const int idx = pg0 + lane;
      __builtin_amdgcn_global_load_lds(idx < max_pages ? row + idx : row,
                                       (__attribute__((address_space(3))) void*)page_ring, 4, 0, 0);
    }
  }
  // The slot list of segment s needs slot_off only: its first fetches are
  // issued before the segment's rows (cu_q, possibly behind seg_ids) are
  // known, so that those two dependent loads overlap.
  // (A load of memory that an earlier DMA into LDS also reads -- the slot
  // fetches read slot_off as their dummy -- can no longer be a scalar load,
  // so in the slot-list form the offsets are loaded first.)
  const int slot_base = PAGED ? 0 : slot_off[s];
  const int n_c = PAGED ? max(slot_off[s], 0) : slot_off[s + 1] - slot_base;
  const int sid = seg_ids ? seg_ids[s] : s;
  const int qrow0 = cu_q[sid];
  const int Lq = cu_q[sid + 1] - qrow0;

  const int wave = wave_id & 3;     // key block of the tile
  const int rblk = wave_id >> 2;    // row block
  const int mt = mb * RB + rblk;
  const int m_base = mt * 32;
  const int jb = rblk * NJ;         // first DMA instruction of this wavefront
  const int lrow = lane & 31;
  const int hl = lane >> 5;
  const int rl = lane >> 4, P = lane & 15;

  // ---- per-lane DMA geometry: instruction j of key block w covers tile rows
  // 32 w + 4j + rl; K chunk (P ^ rl) ^ 4(j & 3), V chunk P ^ 4 rl.
  const uint32_t kchunk = (uint32_t)((P ^ rl) * 16);
  const uint32_t vchunk = (uint32_t)((P ^ (4 * rl)) * 16);
  const int64_t row_elems = (int64_t)Hkv * HD;
  // without a cache (cache_slots = 0, slots may be null) every cached row is
  // outside it: the fetches then read slot_off[0], a valid dummy
  const bool have_slots = n_c > 0 && slots != nullptr && (!PAGED || max_pages > 0);
  const int32_t* sp = have_slots && !PAGED ? slots + slot_base : slot_off;
  // Per-wave pipeline: the slots of tile t+2 are fetched before tile t+1's
  // DMA is issued, so that after computing tile t the wave can issue tile
  // t+2 into the stage it just freed while tile t+1 is still in flight --
  // two tiles in flight.  Vector memory operations complete in issue order,
  // so each wait is "at most N newer operations outstanding": a tile is
  // 2 NJ DMA instructions, a slot fetch one.
  // The slots arrive by DMA too (lane l: the slot of key 32 w + l of the
  // tile) into a ring of four per-wave entries behind the stages, and lanes
  // read them from LDS after the wait that retires the fetch: no register is
  // ever written by a load the compiler does not know about.
  auto fetch_slots = [&](int t) {
    const int kidx = kbeg0 + t * CK_TILE + 32 * wave + lrow;
    const int32_t* src = have_slots ? sp + min(max(kidx, 0), n_c - 1) : sp;
    __builtin_amdgcn_global_load_lds(
        src, (__attribute__((address_space(3))) void*)(slot_ring + ((t & 3) * 4 * RB + wave_id) * 64), 4, 0, 0);
  };
  // After the prologue's wait lane l holds page id pg0 + l in a register, and
  // the page of a tile (the same for the whole wavefront) is one lane read.
  int page_reg = 0;
  const uint32_t n_pages = (uint32_t)min(a.cache_slots >> 8, (int64_t)1 << 23);
  // the first cache row of tile t's page, or -1 past the page table or for a
  // page id outside the cache (whose rows are then masked)
  auto page_of = [&](int t) -> int {
    const int pg = (kbeg0 + t * CK_TILE) >> 8;
    const int pid = __builtin_amdgcn_readlane(page_reg, (pg - pg0) & 63);
    return have_slots && pg < max_pages && (uint32_t)pid < n_pages ? pid * 256 : -1;
  };
  // this lane's slots of tile t (rows 4 (jb + j) + rl of the wave's 32); call after the wait
  auto read_slots = [&](int t, int (&dst)[NJ]) {
    if constexpr (PAGED) {
      const int row0 = page_of(t);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int kidx = kbeg0 + t * CK_TILE + 32 * wave + 4 * (jb + j) + rl;
        // a page outside the cache leaves the slot outside too (masked below)
        dst[j] = row0 >= 0 ? row0 + (kidx & 255) : -1;
      }
    } else {
      const uint32_t* e = slot_ring + ((t & 3) * 4 * RB + wave_id) * 64;
#pragma unroll
      for (int j = 0; j < NJ; ++j) dst[j] = (int)e[4 * (jb + j) + rl];
    }
  };
  // ---- prologue: the slots of the first three tiles (the page ids went
  // out at the start), then the Q^T fragments (their address needs the
  // segment's rows); D(0) and D(1) are issued as soon as the slots have
  // landed, with q still in flight, and a wait that retires q follows them
  // (so the compiler's own wait tracking has no q load left to wait for
  // inside the tile loop).  Slot fetches past the key range read a clamped,
  // valid index and go unused.
  if constexpr (!PAGED) {
    fetch_slots(0);
    fetch_slots(1);
    fetch_slots(2);
  }
  asm volatile("" ::: "memory");  // the slot / page fetches stay the oldest operations
  const int g = a.g;
  const int M = Lq * g;
  if (mb * RB * 32 >= M) {  // the whole workgroup: no live row block
    vm_wait<0>();            // no DMA into LDS may outlive the workgroup
    return;
  }
  const int Lk = n_c + Lq;
  const int kbeg = min(kbeg0, Lk);
  const int kend = min(Lk, kbeg + keys_per_split);
  // Rows past kend read the last valid row; a cached row with an invalid
  // slot reads block row 0 (never the cache, which may be absent).  Both are
  // masked out of the softmax, so only the address needs to be valid.
  // Row addresses, branch-free: a row comes from the cache (base + slot *
  // cache row bytes) or from the block (base + block row * token stride);
  // each is one 32 x 32 -> 64-bit multiply-add.  Slots are int32, so one
  // unsigned compare against the slot count also rejects negative slots.
  const uint32_t cache_row_b = (uint32_t)(row_elems * 2);
  const uint32_t n_slots = (uint32_t)min(a.cache_slots, (int64_t)1 << 31);
  const uint32_t kS_b = (uint32_t)(a.k_stride * 2), vS_b = (uint32_t)(a.v_stride * 2);
  const uint64_t kc0 = (uint64_t)(uintptr_t)(a.k_cache + hkv * HD);
  const uint64_t vc0 = (uint64_t)(uintptr_t)(a.v_cache + hkv * HD);
  const uint64_t kb0 = (uint64_t)(uintptr_t)(a.k + (int64_t)qrow0 * a.k_stride + hkv * HD);
  const uint64_t vb0 = (uint64_t)(uintptr_t)(a.v + (int64_t)qrow0 * a.v_stride + hkv * HD);
  auto issue = [&](uint8_t* stage, int k0, const int (&slot)[NJ]) {
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const int j = jb + jj;
      const int kidx = min(k0 + 32 * wave + 4 * j + rl, max(kend - 1, 0));
      const uint32_t sl = (uint32_t)slot[jj];
      const bool cached = kidx < n_c;
      const bool use_cache = cached && sl < n_slots;
      // a cached row with an invalid slot reads block row 0 (masked later)
      const uint32_t idx = use_cache ? sl : (cached ? 0u : (uint32_t)(kidx - n_c));
      const uint64_t kaddr = (use_cache ? kc0 : kb0) + (uint64_t)idx * (use_cache ? cache_row_b : kS_b);
      const uint64_t vaddr = (use_cache ? vc0 : vb0) + (uint64_t)idx * (use_cache ? cache_row_b : vS_b);
      const int q = 8 * wave + j;
      gdma16(reinterpret_cast<const uint8_t*>(kaddr) + (kchunk ^ (uint32_t)(64 * (jj & 3))), stage + q * 1024);
      gdma16(reinterpret_cast<const uint8_t*>(vaddr) + vchunk, stage + CK_TILE * 256 + q * 1024);
    }
  };
  // keys of this wave's block of tile t whose slot is invalid, as a 32-bit
  // mask (bit = key within the block), from the slot ring after the wait
  auto invalid_keys = [&](int t) -> uint32_t {
    const int kidx = kbeg + t * CK_TILE + 32 * wave + lrow;
    uint32_t sl;
    if constexpr (PAGED) {
      sl = (uint32_t)page_of(t);
    } else {
      sl = slot_ring[((t & 3) * 4 * RB + wave_id) * 64 + lrow];
    }
    const bool bad = kidx < n_c && kidx < kend && sl >= n_slots;
    return (uint32_t)__builtin_amdgcn_ballot_w64(bad);
  };

  const int m = m_base + lrow;
  const bool m_ok = m < M;
  const int tok = m_ok ? m / g : 0;
  const int head = hkv * g + (m_ok ? m - tok * g : 0);
  bf16x8_t qf[1][8];
  {
    const uint32_t qS = (uint32_t)(a.q_stride * 2);
    const uint32_t qbytes = Lq > 0 ? (uint32_t)Lq * qS : 0u;
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(a.q + (int64_t)qrow0 * a.q_stride, qbytes);
    const uint32_t qoff = m_ok ? (uint32_t)tok * qS + (uint32_t)(head * HD + hl * 8) * 2u : qbytes;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[0][kk] = as_bf16x8(bload(qrs, qoff + (uint32_t)kk * 32u, 0u));
  }
  const int ntiles = (kend - kbeg + CK_TILE - 1) / CK_TILE;
  uint32_t bad_t0 = 0, bad_t1 = 0;  // invalid-key masks of tiles t and t+1
  vm_wait<8>();  // S(0..2) or the page ids; the eight q loads may be outstanding
  if constexpr (PAGED) page_reg = (int)page_ring[lane];

  int s0[NJ], s1[NJ];
  read_slots(0, s0);
  read_slots(1, s1);
  if (ntiles > 0) {
    bad_t0 = invalid_keys(0);
    issue(lds, kbeg, s0);                                    // D(0)
  }
  if (ntiles > 1) {
    bad_t1 = invalid_keys(1);
    issue(lds + CK_STAGE, kbeg + CK_TILE, s1);               // D(1)
  }
  if (ntiles > 1)  // q has landed; D(0) and D(1) may be in flight
    vm_wait<4 * NJ>();
  else if (ntiles == 1)
    vm_wait<2 * NJ>();
  else
    vm_wait<0>();

  DenseAddr ad;
  dense_addr(ad, lane, 0u, 0u);
  DenseState<1> st;
  dense_state_init(st);
  const float c = a.scale_log2;

  for (int t = 0; t < ntiles; ++t) {
    const int k0 = kbeg + t * CK_TILE;
    // D(t) has landed once at most the operations issued after it -- S(t+2)
    // and D(t+1), when they exist -- are outstanding.  At t = 0 only D(1)
    // follows D(0) (the prologue retired S(2) before issuing both).
    if (t + 1 >= ntiles)
      vm_wait<0>();
    else if (PAGED || t == 0 || t + 2 >= ntiles)
      vm_wait<2 * NJ>();
    else
      vm_wait<2 * NJ + 1>();
    if constexpr (RB > 1) lds_barrier();  // every wavefront's part of D(t) has landed
    uint8_t* cur = lds + (t & 1) * CK_STAGE + wave * 32 * 256;  // this key block's 32 rows
    const int k_valid = kend - (k0 + 32 * wave);
    uint64_t badk = bad_t0;
    if (k_valid < 32) badk |= k_valid <= 0 ? 0xffffffffull : (0xffffffffull << k_valid) & 0xffffffffull;
    cached_tile(cur, cur + CK_TILE * 256, ad, qf, st, c, badk);
    uint32_t bad_t2 = 0;
    if (t + 2 < ntiles) {
      // stage t&1 is free again (with RB > 1 once both row blocks are done
      // with it): issue D(t+2) there, after S(t+3) (S(t+2) landed behind D(t+1))
      if constexpr (RB > 1) lds_barrier();
      if constexpr (!PAGED) vm_wait<2 * NJ>();  // S(t+2); D(t+1) may stay in flight
      int cur_slots[NJ];
      read_slots(t + 2, cur_slots);
      bad_t2 = invalid_keys(t + 2);
      if (!PAGED && t + 3 < ntiles) fetch_slots(t + 3);
      issue(lds + (t & 1) * CK_STAGE, k0 + 2 * CK_TILE, cur_slots);
    }
    bad_t0 = bad_t1;
    bad_t1 = bad_t2;
  }
  cached_merge_store<RB>(a, lds, (ntiles - 1) & 1, reinterpret_cast<float*>(slot_ring), st, s, hkv, mt, split,
                              qrow0, M, m_base, g, tid, rblk);
}

// Merge the n_split partial records of every (segment, head, M row).
// grid: (n_seg*Hkv*mtiles*32) rows / 8 per block; block 256 = 8 rows x 32
// threads, 4 d each (16-byte partial reads, 8-byte bf16 writes).  The split
// loops are unrolled so that their loads are in flight together: one round
// trip for the row maxima, one for the sums and accumulators.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int row_rec = blockIdx.x * 8 + (threadIdx.x >> 5);  // (s, hkv, mt, q) flattened
  const int d0 = (threadIdx.x & 31) * 4;
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
#pragma unroll 8
  for (int sp = 0; sp < a.n_split; ++sp) mx = fmaxf(mx, ml[((P0 + sp) * 32 + q) * 2]);
  const float mu = (mx == -INFINITY) ? 0.f : mx;
  float l = 0.f, acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
#pragma unroll 8
  for (int sp = 0; sp < a.n_split; ++sp) {
    const float* rec = ml + ((P0 + sp) * 32 + q) * 2;
    const f32x4_t x = *reinterpret_cast<const f32x4_t*>(a.ws + ((P0 + sp) * 32 + q) * HD + d0);
    const float w = (rec[0] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(rec[0] - mu);
    l += rec[1] * w;
    acc0 += x[0] * w;
    acc1 += x[1] * w;
    acc2 += x[2] * w;
    acc3 += x[3] * w;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int tq = mrow / g;
  const int hq = hkv * g + (mrow - tq * g);
  uint32_t* op = reinterpret_cast<uint32_t*>(a.o + (int64_t)(qrow0 + tq) * a.o_stride + hq * HD + d0);
  op[0] = cvt_pk_bf16(acc0 * inv, acc1 * inv);
  op[1] = cvt_pk_bf16(acc2 * inv, acc3 * inv);
}

static const float kLog2e = 1.4426950408889634f;

// K3a launch shapes (one query block of 32 rows per wavefront, two LDS
// stages): 4 wavefronts (128 M rows) with 32-key tiles, or 8 wavefronts
// (256 M rows sharing each K/V tile) with 64-key tiles once the key stream
// is long enough (max_seqlen_k >= 2048) to amortise the larger tiles.
constexpr int DENSE_ST = 2;
constexpr int DENSE_LONG_K = 2048;
constexpr int kOneWgMinPairs = 160;  // (segment, KV head) pairs for the 12-wavefront launch

static int common_checks(const char* name, const void* q, const void* k, const void* v, const void* o, int Hq,
                         int Hkv, int D, int64_t qs, int64_t ks, int64_t vs, int64_t os) {
  if (D != HD) return fail(DLLM_ERR_UNSUPPORTED, "%s: head_dim %d not supported (the kernels handle 128)", name, D);
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

// K3a launch shape: wavefronts per workgroup (4, 12 or 8), keys per tile,
// M tiles per (segment, KV head), XCD chunk and grid.  One function for the
// launch and for dllm_attn_varlen_launch_shape, so that the two cannot drift.
struct DensePlan {
  int nw, tk, mtiles, xcd_chunk, grid;
  int64_t logical;
};
static DensePlan dense_plan(int n_seg, int max_seqlen_q, int max_seqlen_k, int Hq, int Hkv) {
  DensePlan p = {};
  const int g = Hq / Hkv;
  const bool wide = max_seqlen_k >= DENSE_LONG_K;
  // (segment, KV head) pairs of 257..384 M rows: one 12-wavefront workgroup
  // each, so the pair's K/V tiles are read into LDS once instead of by three
  // workgroups (3 % faster for 8 x 384 tokens, 32 heads) -- when there are
  // enough pairs to occupy most of the 256 CUs.  Fewer pairs run faster as
  // three 4-wavefront workgroups each (32 heads x 384 tokens: 1 sequence
  // 12.6 vs 19.8 us, 4 sequences 20.2 vs 23.3 us; 6 sequences 27.4 vs 25.1).
  const int64_t m_rows = (int64_t)max_seqlen_q * g;
  const bool one_wg = !wide && m_rows > 256 && m_rows <= 384 && (int64_t)n_seg * Hkv >= kOneWgMinPairs;
  p.nw = wide ? 8 : (one_wg ? 12 : 4);
  p.tk = wide ? 64 : 32;
  const int bm = 32 * p.nw;
  p.mtiles = (int)((m_rows + bm - 1) / bm);
  p.logical = (int64_t)p.mtiles * Hkv * n_seg;
  // chunks of up to 16 m-tiles of one (segment, KV head): 4..16 measured
  // within 2 % of one contiguous range per XCD on uniform batches
  p.xcd_chunk = p.mtiles < 16 ? p.mtiles : 16;
  const int64_t grain = 8 * (int64_t)p.xcd_chunk;
  p.grid = (int)((p.logical + grain - 1) / grain * grain);
  return p;
}

extern "C" int dllm_attn_varlen_launch_shape(int n_seg, int max_seqlen_q, int max_seqlen_k, int Hq, int Hkv, int D,
                                             int* wavefronts, int* tile_keys, int* grid) {
  if (D != HD || Hq <= 0 || Hkv <= 0 || Hq % Hkv || n_seg < 0 || max_seqlen_q < 0 || max_seqlen_k < 0)
    return fail(DLLM_ERR_INVALID_ARG, "dllm_attn_varlen_launch_shape: unsupported sizes");
  const DensePlan p = dense_plan(n_seg, max_seqlen_q, max_seqlen_k, Hq, Hkv);
  if (wavefronts) *wavefronts = p.nw;
  if (tile_keys) *tile_keys = p.tk;
  if (grid) *grid = (n_seg == 0 || max_seqlen_q == 0) ? 0 : p.grid;
  return DLLM_OK;
}

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
  const DensePlan plan = dense_plan(n_seg, max_seqlen_q, max_seqlen_k, Hq, Hkv);
  const bool wide = plan.nw == 8, one_wg = plan.nw == 12;
  const int nw = plan.nw;
  a.mtiles = plan.mtiles;
  a.n_split = 1;
  if (plan.logical > (int64_t)1 << 30) return fail(DLLM_ERR_INVALID_ARG, "%s: problem too large", name);
  a.logical_blocks = (int)plan.logical;
  a.scale_log2 = softmax_scale * kLog2e;
  // Long key streams: 8 wavefronts (256 M rows) per workgroup, 64-key tiles,
  // one workgroup per CU.  Shorter ones: 4 wavefronts, 32-key tiles, three
  // workgroups per CU (independent workgroups overlap the softmax of one with
  // the MFMAs of another), or 12 wavefronts for pairs of 257..384 M rows.
  // Measured: the 4-wavefront shape is 5-12 % faster up to 1280 keys
  // (4 x 1280, Dream GQA varlen with up to 1245 keys), the 8-wavefront one
  // 6 % faster at 4096 keys.
  auto kern = wide ? attn_dense_kernel<8, 1, DENSE_ST, 64, 2>
                   : (one_wg ? attn_dense_kernel<12, 1, DENSE_ST, 32, 3> : attn_dense_kernel<4, 1, DENSE_ST, 32, 3>);
  int lds_bytes = DENSE_ST * 2 * (wide ? 64 : 32) * 256;
  if (wide || one_wg)
    lds_bytes += nw * 8192;  // Q rows after the stages (one workgroup per CU), later each wavefront's O staging
  else if (nw * 8192 > lds_bytes)
    lds_bytes = nw * 8192;  // O staging
  if ((rc = set_lds(kern, lds_bytes, name))) return rc;
  a.xcd_chunk = plan.xcd_chunk;
  kern<<<dim3(plan.grid), dim3(64 * nw), lds_bytes, reinterpret_cast<hipStream_t>(stream)>>>(a);
  return check_launch(name);
}

// One workgroup per CU fits (the kernel's LDS allows only one), so the plan
// counts generations of 256 workgroups.  Row blocks per workgroup: 2 when a
// (segment, KV head) has at least two 32-row M tiles and pairing them saves
// a whole generation (16 segments x 4 KV heads x 7 M tiles, 28 query heads,
// against 732 keys: 448 -> 256 workgroups, 28 -> 19.5 us); otherwise 1,
// which streams the same bytes with twice the workgroups (4 x 32 heads x 2 M
// tiles against 672 keys: 16.5 us, against 19.3 us paired on 128 CUs).
// Then the keys are split, only while the splits still fit in one
// generation (each split adds a partial record and the combine launch), with
// at least two 128-key tiles per split.
static int block_cached_plan(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int& mtiles, int& rb,
                             int& n_split, int& keys_per_split) {
  const int g = Hq / Hkv;
  mtiles = (max_q * g + 31) / 32;
  const int64_t pairs1 = (int64_t)n_seg * Hkv * mtiles;
  const int64_t pairs2 = (int64_t)n_seg * Hkv * ((mtiles + 1) / 2);
  rb = (mtiles >= 2 && (pairs1 + 255) / 256 > (pairs2 + 255) / 256) ? 2 : 1;
  const int64_t pairs = rb == 2 ? pairs2 : pairs1;
  int64_t want = pairs > 0 ? 256 / pairs : 1;
  const int max_split = max_keys > 0 ? (max_keys + 255) / 256 : 1;
  if (want > max_split) want = max_split;
  if (want < 1) want = 1;
  n_split = (int)want;
  const int tiles = (max_keys + CK_TILE - 1) / CK_TILE;
  const int tiles_per_split = (tiles + n_split - 1) / n_split;
  keys_per_split = tiles_per_split * CK_TILE;
  if (keys_per_split <= 0) keys_per_split = CK_TILE;
  // a split's keys span at most 64 pages of 256 rows: the page-table form
  // keeps that many page ids per wavefront in LDS (both forms plan alike, so
  // one workspace size serves both)
  if (keys_per_split > 64 * 256 - 256) keys_per_split = 64 * 256 - 256;
  n_split = max_keys > 0 ? (max_keys + keys_per_split - 1) / keys_per_split : 1;
  return 0;
}

extern "C" size_t dllm_attn_block_cached_workspace_size(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int D) {
  (void)D;
  if (n_seg <= 0 || max_q <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv) return 0;
  int mtiles, rb, n_split, kps;
  block_cached_plan(n_seg, max_q, max_keys, Hq, Hkv, mtiles, rb, n_split, kps);
  if (n_split <= 1) return 0;
  const size_t nrec = (size_t)n_seg * Hkv * mtiles * n_split;
  return nrec * 32 * (HD + 2) * sizeof(float);
}

extern "C" int dllm_attn_block_cached_launch_shape(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int D,
                                                   int* row_blocks, int* n_split, int* grid) {
  if (D != HD || Hq <= 0 || Hkv <= 0 || Hq % Hkv || n_seg < 0 || max_q < 0 || max_keys < 0)
    return fail(DLLM_ERR_INVALID_ARG, "dllm_attn_block_cached_launch_shape: unsupported sizes");
  int mtiles = 0, rb = 1, ns = 1, kps = 0;
  block_cached_plan(n_seg, max_q, max_keys, Hq, Hkv, mtiles, rb, ns, kps);
  const int mblocks = (mtiles + rb - 1) / rb;
  const int64_t logical = (int64_t)ns * mblocks * Hkv * n_seg;
  const int64_t per_pair = (int64_t)ns * mblocks;
  const int64_t grain = 8 * (per_pair < 16 ? per_pair : 16);
  if (row_blocks) *row_blocks = rb;
  if (n_split) *n_split = ns;
  if (grid) *grid = (n_seg == 0 || max_q == 0) ? 0 : (int)((logical + grain - 1) / grain * grain);
  return DLLM_OK;
}

// Slot-list form (paged = false): slots / slot_off as documented for
// dllm_attn_block_cached_fwd.  Page-table form (paged = true): `slots` is the
// [n_seg][max_pages] page table, `slot_off` the per-segment cached lengths.
static int block_cached_impl(const char* name, const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v,
                             dllm_bf16* o, const int32_t* cu, const int32_t* seg_ids, int n_seg, int max_q,
                             int max_keys, const dllm_bf16* k_cache, const dllm_bf16* v_cache, int64_t cache_slots,
                             const int32_t* slots, const int32_t* slot_off, int Hq, int Hkv, int D,
                             int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok, int64_t o_stride_tok,
                             float softmax_scale, void* workspace, size_t workspace_bytes, void* stream,
                             bool paged = false, int max_pages = 0) {
  int rc = common_checks(name, q, k, v, o, Hq, Hkv, D, q_stride_tok, k_stride_tok, v_stride_tok, o_stride_tok);
  if (rc) return rc;
  if (n_seg < 0 || max_q < 0 || max_keys < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative size", name);
  if (n_seg == 0 || max_q == 0) return DLLM_OK;
  if (!cu || !slot_off) return fail(DLLM_ERR_INVALID_ARG, "%s: null cu / slot_off", name);
  if ((int64_t)max_q * q_stride_tok * 2 + 4096 >= ((int64_t)1 << 32))
    return fail(DLLM_ERR_UNSUPPORTED, "%s: a block spans more than 4 GiB of q", name);
  if (k_stride_tok * 2 >= ((int64_t)1 << 32) || v_stride_tok * 2 >= ((int64_t)1 << 32))
    return fail(DLLM_ERR_UNSUPPORTED, "%s: k / v token strides must be below 4 GiB", name);
  if (cache_slots > 0 && (!k_cache || !v_cache || !slots))
    return fail(DLLM_ERR_INVALID_ARG, "%s: null cache / %s", name, paged ? "page table" : "slots");
  if (paged && (max_pages < 0 || (cache_slots > 0 && max_pages == 0)))
    return fail(DLLM_ERR_INVALID_ARG, "%s: max_pages %d: a page table with a cache needs at least one page per row",
                name, max_pages);
  if (paged && cache_slots % 256)
    return fail(DLLM_ERR_INVALID_ARG, "%s: cache rows %lld: the cache must be whole 256-row pages", name,
                (long long)cache_slots);
  if (paged && ((int64_t)n_seg * max_pages >= ((int64_t)1 << 31) || max_pages >= (1 << 26)))
    return fail(DLLM_ERR_INVALID_ARG, "%s: page table too large", name);
  if (cache_slots > 0 && (!aligned16(k_cache) || !aligned16(v_cache)))
    return fail(DLLM_ERR_INVALID_ARG, "%s: caches must be 16-byte aligned", name);
  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slots = cache_slots;
  a.cu_q = cu; a.cu_k = cu; a.seg_ids = seg_ids; a.slots = slots; a.slot_off = slot_off;
  a.q_stride = q_stride_tok; a.k_stride = k_stride_tok; a.v_stride = v_stride_tok; a.o_stride = o_stride_tok;
  a.n_seg = n_seg; a.Hkv = Hkv; a.g = Hq / Hkv;
  int mtiles, rb, n_split, kps;
  block_cached_plan(n_seg, max_q, max_keys, Hq, Hkv, mtiles, rb, n_split, kps);
  a.mtiles = mtiles; a.n_split = n_split; a.keys_per_split = kps;
  if (n_split > 1) {
    const size_t need = dllm_attn_block_cached_workspace_size(n_seg, max_q, max_keys, Hq, Hkv, D);
    if (!workspace || workspace_bytes < need)
      return fail(DLLM_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", name, need,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(DLLM_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", name);
    a.ws = reinterpret_cast<float*>(workspace);
  }
  const int mblocks = (mtiles + rb - 1) / rb;
  const int64_t logical = (int64_t)n_split * mblocks * Hkv * n_seg;
  if (logical > (int64_t)1 << 30) return fail(DLLM_ERR_INVALID_ARG, "%s: problem too large", name);
  a.logical_blocks = (int)logical;
  a.scale_log2 = softmax_scale * kLog2e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // one chunk per (segment, KV head): its row blocks and splits read the same
  // cached rows; the pairs of one segment go to all eight XCDs
  const int64_t per_pair = (int64_t)n_split * mblocks;
  a.xcd_chunk = (int)(per_pair < 16 ? per_pair : 16);
  const int64_t grain = 8 * (int64_t)a.xcd_chunk;
  const int nb = (int)((logical + grain - 1) / grain * grain);
  auto launch = [&](auto kern, int threads, int lds_bytes) -> int {
    int r = set_lds(kern, lds_bytes, name);
    if (r) return r;
    // no cache: no slot list or page table to read (the kernels test for null)
    const int32_t* table = cache_slots > 0 ? a.slots : nullptr;
    const int chunk_pages = a.xcd_chunk + 32 * (paged ? max_pages : 0);
    kern<<<dim3(nb), dim3(threads), lds_bytes, st>>>(a.slot_off, a.seg_ids, a.cu_q, table, chunk_pages,
                                                      a.logical_blocks, a.mtiles, a.n_split, a.Hkv, a.keys_per_split,
                                                      a);
    return DLLM_OK;
  };
  if (rb == 2)
    rc = paged ? launch(attn_cached_kernel<2, true>, 512, ck_lds_bytes(2))
               : launch(attn_cached_kernel<2, false>, 512, ck_lds_bytes(2));
  else
    rc = paged ? launch(attn_cached_kernel<1, true>, 256, ck_lds_bytes(1))
               : launch(attn_cached_kernel<1, false>, 256, ck_lds_bytes(1));
  if (rc) return rc;
  if ((rc = check_launch(name))) return rc;
  if (n_split > 1) {
    const int64_t rows = (int64_t)n_seg * Hkv * a.mtiles * 32;
    attn_combine_kernel<<<dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, st>>>(a);
    if ((rc = check_launch(name))) return rc;
  }
  return DLLM_OK;
}

extern "C" int dllm_attn_block_cached_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                                          const int32_t* cu, const int32_t* seg_ids, int n_seg, int max_q,
                                          int max_keys, const dllm_bf16* k_cache, const dllm_bf16* v_cache,
                                          int64_t cache_slots, const int32_t* slots, const int32_t* slot_off,
                                          int Hq, int Hkv, int D, int64_t q_stride_tok, int64_t k_stride_tok,
                                          int64_t v_stride_tok, int64_t o_stride_tok, float softmax_scale,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  return block_cached_impl("dllm_attn_block_cached_fwd", q, k, v, o, cu, seg_ids, n_seg, max_q, max_keys, k_cache,
                           v_cache, cache_slots, slots, slot_off, Hq, Hkv, D, q_stride_tok, k_stride_tok,
                           v_stride_tok, o_stride_tok, softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int dllm_attn_block_cached_paged_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v,
                                                dllm_bf16* o, const int32_t* cu, const int32_t* seg_ids, int n_seg,
                                                int max_q, int max_keys, const dllm_bf16* k_cache,
                                                const dllm_bf16* v_cache, int num_pages, const int32_t* page_table,
                                                int max_pages, const int32_t* cached_len, int Hq, int Hkv, int D,
                                                int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                                                int64_t o_stride_tok, float softmax_scale, void* workspace,
                                                size_t workspace_bytes, void* stream) {
  const char* name = "dllm_attn_block_cached_paged_fwd";
  if (num_pages < 0) return fail(DLLM_ERR_INVALID_ARG, "%s: negative num_pages", name);
  if (!cached_len && n_seg > 0) return fail(DLLM_ERR_INVALID_ARG, "%s: null cached_len", name);
  return block_cached_impl(name, q, k, v, o, cu, seg_ids, n_seg, max_q, max_keys, k_cache, v_cache,
                           (int64_t)num_pages * 256, page_table, cached_len, Hq, Hkv, D, q_stride_tok, k_stride_tok,
                           v_stride_tok, o_stride_tok, softmax_scale, workspace, workspace_bytes, stream, true,
                           max_pages);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the split partials go to `scratch`, a file-scope
// device array (one copy per GPU, held until the process ends), instead of
// a caller workspace.  In host code `scratch` names a host-side stand-in, not
// device memory: its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is
// ever handed to kernels.  The partial records are written in full by the
// splits before the combine kernel reads them, so nothing needs clearing
// between calls; calls that overlap on one GPU share the array and race.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (looked up on first use).
static int scratch_ptr(const char* name, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DLLM_ERR_HIP, "%s: hipGetDevice: %s", name, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(DLLM_ERR_UNSUPPORTED, "%s: device %d beyond %d", name, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DLLM_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", name, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DLLM_OK;
}

extern "C" size_t dllm_attn_block_cached_noalloc_max_workspace(void) { return kScratchBytes; }

extern "C" int dllm_attn_block_cached_fwd_noalloc(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v,
                                                  dllm_bf16* o, const int32_t* cu, const int32_t* seg_ids,
                                                  int n_seg, int max_q, int max_keys, const dllm_bf16* k_cache,
                                                  const dllm_bf16* v_cache, int64_t cache_slots, const int32_t* slots,
                                                  const int32_t* slot_off, int Hq, int Hkv, int D,
                                                  int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                                                  int64_t o_stride_tok, float softmax_scale, void* stream) {
  const char* name = "dllm_attn_block_cached_fwd_noalloc";
  const size_t need = dllm_attn_block_cached_workspace_size(n_seg, max_q, max_keys, Hq, Hkv, D);
  if (need > kScratchBytes)
    return fail(DLLM_ERR_UNSUPPORTED, "%s: this launch needs %zu bytes of split partials, beyond the %zu-byte static scratch",
                name, need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    int rc = scratch_ptr(name, &ws);
    if (rc) return rc;
  }
  return block_cached_impl(name, q, k, v, o, cu, seg_ids, n_seg, max_q, max_keys, k_cache, v_cache, cache_slots,
                           slots, slot_off, Hq, Hkv, D, q_stride_tok, k_stride_tok, v_stride_tok, o_stride_tok,
                           softmax_scale, ws, need > 0 ? kScratchBytes : 0, stream);
}

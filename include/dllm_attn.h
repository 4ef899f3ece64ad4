/*
 * dllm_attn.h -- C ABI of the MI355X (gfx950) diffusion-LLM attention path.
 *
 * Every entry point is asynchronous on the HIP stream it is given (pass the
 * caller's current stream, e.g. torch.cuda.current_stream().cuda_stream),
 * takes raw device pointers, element strides and sizes, never allocates
 * device memory and never throws.  Return value 0 means the work was
 * enqueued; a negative DLLM_ERR_* code means nothing was launched and
 * dllm_last_error() describes why (thread-local, valid until the next call
 * on the same thread).
 *
 * Tensors are bfloat16 (raw 16-bit patterns, type dllm_bf16), row-major,
 * innermost dimension contiguous.  "Rows" are tokens: q is [rows, Hq, D],
 * k / v are [rows, Hkv, D]; *_stride_tok is the element distance between
 * consecutive tokens (>= H*D).  Heads are contiguous inside a token row.
 *
 * Each declaration names the reference interface (chosen-ox/dLLM-Serve,
 * file:line) whose behaviour it reproduces.
 */
#ifndef DLLM_ATTN_H
#define DLLM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t dllm_bf16; /* bfloat16 bit pattern */

#define DLLM_OK 0
#define DLLM_ERR_INVALID_ARG (-1) /* shape / stride / alignment / size mismatch */
#define DLLM_ERR_UNSUPPORTED (-2) /* valid request the library does not implement (e.g. head_dim != 128) */
#define DLLM_ERR_WORKSPACE (-3)   /* workspace pointer missing or too small */
#define DLLM_ERR_HIP (-4)         /* a HIP runtime call or kernel launch failed */

/* Message for the last failing call on this thread ("" if none). */
const char* dllm_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int dllm_abi_version(void);

/*
 * K1 -- KV-cache scatter.  Replaces store_kvcache / store_kvcache_kernel
 * (dllmserve/layers/attention.py:11-50).
 *
 * For i in [0, n_tok): k_cache[slot_mapping[i] * row_elems + e] = key[i * key_stride_tok + e]
 * and the same for value / v_cache, e in [0, row_elems), row_elems = Hkv * D.
 * The cache is viewed as flat rows of row_elems elements (its slot stride is
 * row_elems), as the reference asserts at attention.py:44.  cache_slots is
 * the number of rows the cache holds; a slot outside [0, cache_slots) is
 * skipped instead of written out of bounds (the reference does not check).
 * Bit-exact copy.
 */
int dllm_store_kvcache(const dllm_bf16* key, int64_t key_stride_tok,
                       const dllm_bf16* value, int64_t value_stride_tok,
                       dllm_bf16* k_cache, dllm_bf16* v_cache, int64_t cache_slots,
                       const int32_t* slot_mapping, int n_tok, int row_elems,
                       void* stream);

/*
 * K2 -- KV-cache gather.  Replaces load_kvcache / load_kvcache_kernel
 * (dllmserve/layers/attention.py:53-92):  key[i] = k_cache[slot_mapping[i]],
 * value[i] = v_cache[slot_mapping[i]].  Rows whose slot is outside
 * [0, cache_slots) are left untouched.  Bit-exact copy.
 */
int dllm_load_kvcache(dllm_bf16* key, int64_t key_stride_tok,
                      dllm_bf16* value, int64_t value_stride_tok,
                      const dllm_bf16* k_cache, const dllm_bf16* v_cache, int64_t cache_slots,
                      const int32_t* slot_mapping, int n_tok, int row_elems,
                      void* stream);

/*
 * K3a -- non-causal (bidirectional) varlen attention over packed segments.
 * Replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k,
 * max_seqlen_q, max_seqlen_k, softmax_scale, causal=False)
 * (dllmserve/layers/attention.py:289-299, the mode-0/1 rows of
 * _mixed_sparse_dense_attention, attention.py:168-187).
 *
 * Segment s covers q rows [cu_q[id], cu_q[id+1]) and k/v rows
 * [cu_k[id], cu_k[id+1]) where id = seg_ids ? seg_ids[s] : s, s in [0, n_seg).
 * seg_ids lets a caller run a subset of the sequences of one packed batch in
 * place, without packing copies.  For every q row t of segment s and head h:
 *   o[t, h] = sum_u softmax_u(scale * q[t, h] . k[u, h / (Hq/Hkv)]) v[u, h / (Hq/Hkv)]
 * bf16 inputs, fp32 accumulation, bf16 output.  max_seqlen_q / max_seqlen_k
 * must bound every segment's q / k length (as in flash-attn; max_seqlen_q
 * sizes the grid).  A segment may span at most 4 GiB of q, k or v.  D must be 128;
 * Hq must be a multiple of Hkv.  Pointers must be 16-byte aligned and the
 * token strides multiples of 8 elements.  Rows of o outside the segments are
 * not written; the rows of a segment with no keys are written as zeros.
 */
int dllm_attn_varlen_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                         const int32_t* cu_q, const int32_t* cu_k, const int32_t* seg_ids,
                         int n_seg, int max_seqlen_q, int max_seqlen_k, int Hq, int Hkv, int D,
                         int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                         int64_t o_stride_tok, float softmax_scale, void* stream);

/*
 * Launch shape dllm_attn_varlen_fwd picks for these sizes, without launching:
 * wavefronts per workgroup (4, 12 or 8), keys per LDS tile and the grid (0
 * when there is nothing to do).  No counterpart in the reference (flash-attn
 * chooses its tiling internally); it lets tests and profiles name the kernel
 * a given call runs.  Any output pointer may be null.
 */
int dllm_attn_varlen_launch_shape(int n_seg, int max_seqlen_q, int max_seqlen_k, int Hq, int Hkv, int D,
                                  int* wavefronts, int* tile_keys, int* grid);

/*
 * K3b -- attention of the current generation block against cached KV plus
 * the block itself (mode 2 / "reuse cache").  Replaces the load_kvcache +
 * torch.cat + flash_attn_varlen_func sequence of
 * dllmserve/layers/attention.py:235-265,289-299.
 *
 * Segment s (id = seg_ids ? seg_ids[s] : s) has q rows and block k/v rows
 * [cu[id], cu[id+1]) (the block tokens only) and n_c = slot_off[s+1] -
 * slot_off[s] cached rows whose cache slots are slots[slot_off[s] + r].
 * Keys/values of segment s are [cache rows r = 0..n_c-1 ; block rows].
 * The cache is [cache_slots, Hkv, D] with slot stride Hkv*D (flat rows, as
 * store_kvcache writes it).  A cached row whose slot is outside
 * [0, cache_slots) is left out of the softmax (the reference would read out
 * of bounds); with cache_slots = 0, k_cache, v_cache and slots may be null
 * and every cached row is left out.  max_q bounds the block length of every
 * segment.
 * The work is split over the keys when there are few segments; the partial
 * results go to `workspace`, whose size must be at least
 * dllm_attn_block_cached_workspace_size(...) bytes (0 is valid when that
 * function returns 0).
 */
size_t dllm_attn_block_cached_workspace_size(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int D);
/* Launch shape of dllm_attn_block_cached_fwd for these sizes, without
 * launching: 32-row blocks per workgroup (1 or 2), key splits (> 1 adds the
 * combine launch) and the grid.  No counterpart in the reference; for tests
 * and profiles.  Any output pointer may be null. */
int dllm_attn_block_cached_launch_shape(int n_seg, int max_q, int max_keys, int Hq, int Hkv, int D,
                                        int* row_blocks, int* n_split, int* grid);
int dllm_attn_block_cached_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                               const int32_t* cu, const int32_t* seg_ids, int n_seg, int max_q, int max_keys,
                               const dllm_bf16* k_cache, const dllm_bf16* v_cache, int64_t cache_slots,
                               const int32_t* slots, const int32_t* slot_off,
                               int Hq, int Hkv, int D,
                               int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                               int64_t o_stride_tok, float softmax_scale,
                               void* workspace, size_t workspace_bytes, void* stream);

/*
 * K3b, page-table form: the cached rows of each segment are given the way
 * the runner holds them, as a page table and a length, instead of a slot
 * list.  The signature the boundary of the hot path names for this kernel
 * (page_table, max_pages, cached_len); the rows are those the reference's
 * state-2 slot list addresses (dllmserve/engine/model_runner.py:257-273:
 * concatenation over pages j of page_j * 256 + 0..255, the last page
 * partly), read by load_kvcache and concatenated with the block
 * (dllmserve/layers/attention.py:235-265).
 *
 * Segment s (the s-th of the launch, as for slot_off) has cached_len[s]
 * cached rows; cached row r is cache row page_table[s * max_pages + r / 256]
 * * 256 + r % 256, in a cache of num_pages pages of 256 rows ([num_pages *
 * 256, Hkv, D], the reference's [num_blocks, 256, Hkv, D]).  A row whose page
 * id is outside [0, num_pages), or whose page index is >= max_pages, is left
 * out of the softmax.  Same workspace (dllm_attn_block_cached_workspace_size)
 * and results as dllm_attn_block_cached_fwd over the equivalent slot lists;
 * the kernel needs one dependent load (the page ids) before its first K/V
 * tile instead of two (slot offsets, then the slot list).
 */
int dllm_attn_block_cached_paged_fwd(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                                     const int32_t* cu, const int32_t* seg_ids, int n_seg, int max_q, int max_keys,
                                     const dllm_bf16* k_cache, const dllm_bf16* v_cache, int num_pages,
                                     const int32_t* page_table, int max_pages, const int32_t* cached_len,
                                     int Hq, int Hkv, int D,
                                     int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                                     int64_t o_stride_tok, float softmax_scale,
                                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * K3b without a caller workspace.  No counterpart in the reference: this is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  Same
 * arguments, kernels and results as dllm_attn_block_cached_fwd, but the split
 * partials go to a static device array of the library (one per GPU, held
 * until the process ends) of dllm_attn_block_cached_noalloc_max_workspace()
 * bytes (16 MiB); a launch whose dllm_attn_block_cached_workspace_size(...)
 * exceeds it fails with DLLM_ERR_UNSUPPORTED and launches nothing.  The call
 * allocates nothing.  Every call on one GPU shares that array: calls that
 * overlap on one GPU (different streams, or host threads) race and must be
 * serialised by the caller.
 */
size_t dllm_attn_block_cached_noalloc_max_workspace(void);
int dllm_attn_block_cached_fwd_noalloc(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, dllm_bf16* o,
                                       const int32_t* cu, const int32_t* seg_ids, int n_seg, int max_q,
                                       int max_keys, const dllm_bf16* k_cache, const dllm_bf16* v_cache,
                                       int64_t cache_slots, const int32_t* slots, const int32_t* slot_off,
                                       int Hq, int Hkv, int D,
                                       int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                                       int64_t o_stride_tok, float softmax_scale, void* stream);

/*
 * K5 / K6 -- sparse KV selection fused with the KV-cache scatter (mode 1 /
 * "compute cache").  Replaces _select_important_head_kv (head_select != 0,
 * dllmserve/layers/attention.py:344-413), _select_important_kv (head_select
 * == 0, attention.py:308-342) and the store_kvcache call that follows them
 * (attention.py:189-233).  Each job carries its own head_select and
 * pool_kernel (the reference reads both per sequence, attention.py:211,329,
 * 387), so one call serves a step mixing SparseConfigs.
 *
 * jobs is an int32 array [n_job][8]: {row0, n_tok, blk_start, blk_len, n_keep,
 * slot_off, head_select, pool_k}.  For job j the sequence occupies q/k/v rows
 * [row0, row0+n_tok) (within [0, n_rows)); the current block is rows
 * [blk_start, blk_start+blk_len) of the sequence; the candidates are the
 * other Kc = n_tok - blk_len rows in order (prefix, then suffix).  Per
 * selection head (each KV head when head_select != 0, one shared head
 * otherwise) the n_keep candidates with the highest pooled score are written,
 * best first, to cache slots slots[slot_off + r], r in [0, n_keep)
 * (slot_off + n_keep <= n_slots).  Scoring rule (deterministic; bit-exact
 * against the oracle), with g = Hq / Hkv and dot(h, j) = f64 sum over d
 * ascending of qbar[h, d] * k[cand j, h / g, d]:
 *   qbar[h, d]  = bf16(f32(f64 sum_t q[blk_start+t, h, d], t ascending) / blk_len))
 *   raw[kv, j]  = max over the g query heads h of KV head kv of bf16(f32(dot(h, j)))
 *                 (head_select == 0: one raw[j] = bf16(f32(sum over kv ascending of
 *                  (sum over h of kv's group ascending of dot(h, j)))), f64 sums)
 *   score[j]    = bf16(f32(raw[j]) / f32(sqrt(D)))   (IEEE division)
 *   pooled[j]   = max of score over [j - pool_k/2, j - pool_k/2 + pool_k - 1]
 *                 clipped to the candidates (no pooling when pool_k <= 1)
 *   order: pooled descending, then candidate index ascending.
 * There is no limit on Kc.  idx_out (nullable) receives the selected
 * candidate indices as int64 [n_job][Hkv][max_keep] (a head_select == 0 job
 * writes row 0 of its entry only; entries r >= n_keep are not written).
 * Jobs are clamped to the launch sizes: Kc to max_kc, n_keep to
 * min(max_keep, Kc); a job whose rows, block or slots fall outside the given
 * sizes selects and writes nothing.  workspace must hold
 * dllm_select_kv_workspace_size(...) bytes, 16-byte aligned.
 */
size_t dllm_select_kv_workspace_size(int n_job, int max_kc, int Hq, int Hkv, int D);
int dllm_select_kv_store(const dllm_bf16* q, const dllm_bf16* k, const dllm_bf16* v, int64_t n_rows,
                         int64_t q_stride_tok, int64_t k_stride_tok, int64_t v_stride_tok,
                         const int32_t* jobs, int n_job, int max_kc, int max_keep,
                         int Hq, int Hkv, int D, float sqrt_d,
                         dllm_bf16* k_cache, dllm_bf16* v_cache, int64_t cache_slots,
                         const int32_t* slots, int64_t n_slots, int64_t* idx_out,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * K7 -- NeoX rotary embedding of q and k in one launch.  Replaces
 * RotaryEmbedding.forward / apply_rotary_emb
 * (dllmserve/layers/rotary_embedding.py:6-17,41-57), applied to q and k
 * before attention at dllmserve/models/llada.py:81 and dream.py:90.
 *
 * cos_sin_cache is the reference's f32 table [max_position, D] (cos of the
 * D/2 frequencies, then their sin; rotary_embedding.py:30-38).  For token i
 * with p = positions[i] (int64), head h, j in [0, D/2):
 *   x1 = x[i,h,j], x2 = x[i,h,j+D/2] as f32, c = table[p][j], s = table[p][D/2+j]
 *   out[i,h,j]     = bf16(x1*c - x2*s)
 *   out[i,h,j+D/2] = bf16(x2*c + x1*s)
 * each product and sum rounded to f32 (no fused multiply-add), bf16 by
 * round-to-nearest-even: bit-exact against that f32 expression evaluated op
 * by op.  q is [n_tok, Hq, D] and k [n_tok, Hkv, D] with the given token
 * strides; out may equal in (in place) but must not otherwise overlap it.
 * A token whose position is outside [0, max_position) is not written (the
 * reference's table lookup would fail).  D must be a multiple of 16.
 */
int dllm_rope_neox(const dllm_bf16* q_in, int64_t q_in_stride, dllm_bf16* q_out, int64_t q_out_stride,
                   const dllm_bf16* k_in, int64_t k_in_stride, dllm_bf16* k_out, int64_t k_out_stride,
                   const int64_t* positions, const float* cos_sin_cache, int64_t max_position,
                   int n_tok, int Hq, int Hkv, int D, void* stream);

/*
 * K8 -- softmax-max of logit rows.  Replaces
 *   probs = F.softmax(logits, dim=-1); x0_p, x0 = torch.max(probs, dim=-1)
 * on bf16 logits (dllmserve/engine/model_runner.py:862-863,886-887, the
 * low-confidence branch of _reconstruct_and_sample_optimized_v2; also :697-701).
 *
 * logits is [M, V] bf16 with row stride ld elements.  Per row, in f32:
 *   m = max_j l_j,  s = sum_j exp(l_j - m),  P_j = bf16(exp(l_j - m) / s)
 *   x0_p[r] = max_j P_j = bf16(1 / s),  x0[r] = min { j : P_j == x0_p[r] }
 * (torch.max returns the first maximal index).  Rows holding NaN or only
 * -inf give unspecified results (torch's are NaN).  V must be a multiple of
 * 8; logits 16-byte aligned, ld a multiple of 8 and >= V.  One workgroup
 * reduces each row, so dllm_softmax_max_workspace_size returns 0 and
 * workspace may be null (the arguments keep the signature stable).
 */
size_t dllm_softmax_max_workspace_size(int M, int V);
int dllm_softmax_max(const dllm_bf16* logits, int64_t ld, int M, int V, int64_t* x0, dllm_bf16* x0_p,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * K8 with sampling noise.  Replaces add_gumbel_noise + softmax + max for
 * sequences sampled at temperature > 0 (dllmserve/engine/model_runner.py:
 * 592-600,826-836,859-866).  Row r with row_temperature[r] = T > 0 is first
 * transformed as the reference does:
 *   v_j = bf16(f32(exp(f64 l_j) / (-log u_j)^T)),  u_j uniform in [0, 1) (f64)
 * and x0 / x0_p are then taken over v as in dllm_softmax_max; rows with
 * T <= 0 are plain.  u_j = 2^-53 * (SplitMix64(seed + (c + 1) *
 * 0x9E3779B97F4A7C15) >> 11) with c = (row_base + r) * V + j: counter-based,
 * so the draws of a row depend on (seed, row_base + r, j) only, not on how
 * rows are split into calls.  (torch's generator stream is not reproduced;
 * the noise follows the same distribution.)  row_temperature may be null
 * (then this is dllm_softmax_max).
 */
int dllm_softmax_max_sample(const dllm_bf16* logits, int64_t ld, int M, int V, const double* row_temperature,
                            uint64_t seed, int64_t row_base, int64_t* x0, dllm_bf16* x0_p,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * K9 -- low-confidence unmasking of one denoising step.  Replaces the
 * per-sequence loop of _reconstruct_and_sample_optimized_v2
 * (dllmserve/engine/model_runner.py:895-949: mask test, steps_remain,
 * num_to_unmask, the is_full_attention first-token rule, torch.topk and the
 * token write-back).
 *
 * seq_params is int32 [n_seq][5]: {tok_off, win_len, row_off, steps_remain,
 * first_rule}.  Sequence b's window is tokens[tok_off + j], j in [0, win_len)
 * (the positions the reference's `indices` name); its predictions and
 * confidences are x0[row_off + j] and conf[row_off + j] (conf: x0_p from
 * dllm_softmax_max for "low_confidence", or the caller's uniform draws for
 * "random", :903-907).  With nmask = #{j : tokens[tok_off + j] == mask_id}:
 *   k = min(ceil(nmask / steps_remain), nmask)     (0 when steps_remain <= 0)
 *   if first_rule and k > 0 and position 0 is masked: it takes x0[row_off]
 *     and k -= 1 (:917-935)
 *   the k masked positions with the highest conf (ties: lower j first, the
 *   set torch.topk returns) take their x0.
 * n_unmasked (nullable) receives the k of each sequence before the
 * first-token rule.  A sequence whose window or rows fall outside
 * [0, n_tokens) / [0, n_rows) is left unchanged (n_unmasked 0).  max_win must
 * bound every win_len and be at most 8192 (the reference's gen_length cap).
 */
int dllm_lowconf_unmask(int64_t* tokens, int64_t n_tokens, const int32_t* seq_params, int n_seq, int max_win,
                        const int64_t* x0, const dllm_bf16* conf, int64_t n_rows, int64_t mask_id,
                        int32_t* n_unmasked, void* stream);

/*
 * S1 -- device-side step metadata.  Replaces the host loops that build one
 * diffusion step's inputs and launch tables: ModelRunner._run_diffusion's
 * row / position / slot-list construction (dllmserve/engine/model_runner.py:
 * 231-321, slot lists :257-273,287-302), the per-sequence mode and
 * selection sizes of _mixed_sparse_dense_attention (dllmserve/layers/
 * attention.py:168-265, sequence.py:99-152) and the sampler's windows
 * (model_runner.py:791-818,911-920).
 *
 * seq_state is int32 [n_seq][12] per sequence: {P (prompt tokens), N (all
 * tokens), sparse (0: no SparseConfig), block_len, current_block_idx,
 * step_in_block, cache_state, delay_step, steps, current_step, head_select,
 * pool_kernel}; ratio is the
 * f64 retention ratio per sequence.  Sequence b's cache pages are
 * pages[page_off[b] .. page_off[b+1]).  Outputs, for the step the state
 * describes (n = n_seq):
 *   cu [n+1]            packed row offsets of the fed rows (all N rows; only
 *                       the block's rows in cache state 2)
 *   dense_ids [max(1,n)]  sequences of full attention (state 0/1 or none), most rows
 *                        first (ties by index)
 *   cached_ids [max(1,n)] sequences in state 2, in order
 *   slot_off [n+1]      their slot ranges in `slots`
 *   jobs [max(1,n)][8]  state-1 selection jobs {row0, n_tok, blk_start,
 *                       blk_len, n_keep, slot_off, head_select, pool_k} (as
 *                       dllm_select_kv_store)
 *   slots [slots_cap]   n_keep slots per state-2 sequence, then per state-1
 *                       sequence: page[r / 256] * 256 + r % 256 (-1 past its pages)
 *   positions, token_index [rows_cap] (int64) position of each fed row and
 *                       its index b * tok_stride + position in the token table
 *   smp_params [n][5], smp_rows [win_cap]  the dllm_lowconf_unmask parameters
 *                       and the fed row of each window position
 *   counts [8]          {rows, n_dense, n_cached, n_job, slots, window
 *                       positions, capacity exceeded (0/1), sequences in an
 *                       invalid state}
 * n_keep = min(max(1, int(Kc * ratio)), Kc).  When a capacity is exceeded only
 * the per-sequence tables are written.  n_seq must be at most 1024.
 */
int dllm_step_build(const int32_t* seq_state, const double* ratio, const int32_t* pages, const int32_t* page_off,
                    int n_seq, int64_t tok_stride, int32_t* cu, int32_t* dense_ids, int32_t* cached_ids,
                    int32_t* slot_off, int32_t* jobs, int32_t* slots, int slots_cap, int64_t* positions,
                    int64_t* token_index, int rows_cap, int32_t* smp_params, int64_t* smp_rows, int win_cap,
                    int32_t* counts, void* stream);

/*
 * S2 -- advance every sequence's state by one denoising step on the device:
 * current_step += 1 (Scheduler.postprocess, scheduler.py:117-120) and, for
 * sparse sequences, PerRequestSparseState.advance_step (state.py:77-104).
 * block_len must be >= 1.
 */
int dllm_step_advance(int32_t* seq_state, int n_seq, void* stream);

/*
 * Same-run clock control for benchmarks.  No counterpart in the reference:
 * a register-only MFMA loop (n_cu workgroups of 8 wavefronts, one per CU,
 * each wavefront 4 independent v_mfma_f32_32x32x16_bf16 chains of `iters`
 * steps) whose throughput depends only on the matrix pipe and the shader
 * clock; a benchmark reports its TFLOP/s beside the kernels it times.
 * sink: n_cu * 512 floats.  dllm_mfma_probe_flops gives the FLOPs of one call.
 */
int64_t dllm_mfma_probe_flops(int n_cu, int iters);
int dllm_mfma_probe(float* sink, int n_cu, int iters, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DLLM_ATTN_H */

/*
 * sglang_neuron_amd — C ABI of the MI355X (gfx950) paged decode-attention path.
 *
 * The library is libsglang_neuron_amd.so, built with hipcc for gfx950 from sglang_neuron_amd/csrc/. Every
 * function takes raw device pointers, int32/int64 sizes, and a hipStream_t passed as `void *`. Each returns an int
 * status: SNA_OK (0), or a negative code with a message that sna_last_error() gives back on the calling thread.
 * Nothing throws across the ABI, and no function allocates device memory. Kernels are enqueued on the caller's
 * stream in call order, so a store followed by a decode on one stream sees the store. The library's only state is the
 * thread-local error string and, for sna_paged_decode_gqa_noalloc, each device's scratch array and its address.
 *
 * Conventions (sglang-neuron, reference paths under /root/reference/sglang_neuron):
 *   - A token slot is page * page_size + offset; page = slot / page_size (attention/backend.py:6-7).
 *   - Page 0 is reserved: a pool of `size` slots has size / page_size + 1 pages (mem_cache/memory_pool.py:20-21,
 *     106-107).
 *   - Block tables are int32 [B, width] with -1 past a row's pages (attention/backend.py:114-130).
 *   - seq_lens count the prefix plus the new token (attention/backend.py:36). The new token sits at position
 *     seq_len - 1 and is attended in-band, as the reference appends it (attention_decode_paged.py:167-169,
 *     attention_decode.py:262-269).
 *   - MHA caches are head-major, [num_blocks, kv_heads, page_size, head_dim] (memory_pool.py:186-191). FP8 K is
 *     stored unpacked (fp8_packed_k = False; the reference's packed [.., page/2, d, 2] K is a Trainium-kernel
 *     layout, attention_decode.py:207-223).
 *   - FP8 is OCP e4m3fn. A stored value is e4m3fn_RNE(clamp(float(x) / s, -448, 448)), where s is the
 *     dequantization scale (swa_fused.py:73-75, qkv.py:69-70, mla_decode_attention_torch.py:216-220), or, for an MHA
 *     cache of dtype SNA_DTYPE_FP8_E4M3FN_MUL, e4m3fn_RNE(clamp(bf16_RNE(x * m), -448, 448)) with the GPT-OSS
 *     quantization multiplier m (attention_decode.py:259-260).
 */
#ifndef SGLANG_NEURON_AMD_H_
#define SGLANG_NEURON_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define SNA_OK 0
#define SNA_ERR_INVALID_ARGUMENT (-1) /* a null pointer, a bad shape or size, an unsupported combination */
#define SNA_ERR_WORKSPACE (-2)        /* the workspace is smaller than the plan needs */
#define SNA_ERR_LAUNCH (-3)           /* the HIP runtime refused a launch */
#define SNA_ERR_UNSUPPORTED (-4)      /* a dtype or head layout this build has no kernel for */

/* ---- dtypes of cache storage ----
 * SNA_DTYPE_FP8_E4M3FN and SNA_DTYPE_FP8_E4M3FN_MUL caches hold the same e4m3fn bytes; they differ in what the scale
 * arrays hold and so in how a store rounds:
 *   FP8_E4M3FN      scale = s, the dequantization scale: byte = e4m3fn_RNE(clamp(float(x) / s, +-448)) (the divide of
 *                   qkv.py:69-70 and swa_fused.py:73-75); value = float(byte) * s.
 *   FP8_E4M3FN_MUL  scale = m, the reference's GPT-OSS k_scale / v_scale: the inverted checkpoint scale as a bf16 value
 *                   (gpt_oss/mxfp4/common.py:481-485, 1 / bf16(s) rounded to bf16): byte =
 *                   e4m3fn_RNE(clamp(bf16_RNE(x * m), +-448)) (the decode write of attention_decode.py:259-260, a
 *                   product of two bf16 tensors); value = float(byte) / m (the dequantization the model folds into the
 *                   softmax scale and the output projection, gpt_oss/mxfp4/model_decode.py:62-70).
 * The two give different bytes unless m and 1 / s are powers of two. */
#define SNA_DTYPE_BF16 0
#define SNA_DTYPE_FP8_E4M3FN 1
#define SNA_DTYPE_FP8_E4M3FN_MUL 2

/* Library ABI version (major * 100 + minor). */
int sna_version(void);

/* The message of the calling thread's last failing call ("" if none). The pointer is valid until the thread's
 * next call into the library. */
const char *sna_last_error(void);

/* =====================================================================================================
 * KV-pool stores
 * ===================================================================================================== */

/* Store one token per entry of `slots` into an MHA pool layer.
 *   k, v        [n_tokens, num_kv_heads, head_dim] bf16, contiguous.
 *   slots       [n_tokens] int64 token slots. A slot < 0 or >= num_blocks * page_size is written to slot 0, the
 *               reserved padding page (attention_decode.py:288-291; transformer/model.py:99-102).
 *   k_scale, v_scale
 *               [num_kv_heads] fp32: the dequantization scales s (SNA_DTYPE_FP8_E4M3FN) or the quantization
 *               multipliers m (SNA_DTYPE_FP8_E4M3FN_MUL). Required for an FP8 cache and ignored for bf16.
 *   k_cache, v_cache
 *               [num_blocks, num_kv_heads, page_size, head_dim], of dtype cache_dtype.
 * FP8_E4M3FN: byte = e4m3fn_RNE(clamp(float(x) / s[h], +-448)), bit-exact with the reference's divide-and-clamp
 * (qkv.py:69-79, swa_fused.py:73-75). FP8_E4M3FN_MUL: byte = e4m3fn_RNE(clamp(bf16_RNE(x * m[h]), +-448)), bit-exact
 * with the GPT-OSS decode write (attention_decode.py:259-260, 288-300). bf16 cache: a copy
 * (attention_decode_paged.py:174-176).
 * Replaces: the pool write that the reference's compiled graphs do. The reference pool's own set_kv_buffer refuses
 * (mem_cache/memory_pool.py:178-179); this is upstream SGLang's
 * MHATokenToKVPool.set_kv_buffer(layer, loc, cache_k, cache_v, k_scale, v_scale) for this pool layout. */
int sna_kv_store_mha(const void *k, const void *v, const int64_t *slots, int64_t n_tokens, const float *k_scale,
                     const float *v_scale, void *k_cache, void *v_cache, int64_t num_blocks, int32_t num_kv_heads,
                     int32_t page_size, int32_t head_dim, int32_t cache_dtype, void *stream);

/* The QKV writer after the projection: optional per-head RMSNorm of Q and K, rotate-half RoPE of Q and K, Q written
 * out, K and V stored into the MHA pool layer as sna_kv_store_mha stores them.
 *   qkv          [n_tokens, qkv_stride] bf16: the projection's output (bias included), heads [Q Hq | K Hkv | V Hkv]
 *                of head_dim each (64 or 128). Tensors and row strides 16-byte aligned.
 *   q_norm, k_norm
 *                [head_dim] bf16 RMSNorm gammas, both or neither (NULL: no QK norm); eps as the model's.
 *   cos, sin     [n_tokens, rope_stride] bf16, head_dim columns each (qkv_paged.py's [1, T, d] over contiguous
 *                halves; qkv.py's caches repeat the first half, and the two forms then agree).
 *   slots        [n_tokens] int64; out-of-pool or negative slots go to slot 0, as for sna_kv_store_mha.
 *   q_out        [n_tokens, num_q_heads, head_dim] bf16.
 *   k_cache, v_cache, k_scale, v_scale, num_blocks, page_size, cache_dtype
 *                as for sna_kv_store_mha (per-KV-head scales; one per-tensor scale is all heads alike), cache_dtype
 *                SNA_DTYPE_BF16 or SNA_DTYPE_FP8_E4M3FN. The writer divides, as the reference's prefill writers do
 *                (qkv.py:69-70); a GPT-OSS pool of multipliers m is written by passing SNA_DTYPE_FP8_E4M3FN with the
 *                scales bf16(1 / m), as its prefill does (gpt_oss/mxfp4/model_prefill.py:41-43).
 * Every rounding of the reference's torch path is kept (bf16 norm output, bf16 gamma product, bf16 RoPE products and
 * sum). The norm's fp32 sum of squares (the reference leaves its order to the backend) runs in a stated order: each
 * square rounded, a lane's 8 in sequence, then the head's lane sums folded in halves; 1 / sqrt is correctly rounded.
 * Replaces: the torch writer of _torch_qkv_paged after its projection (ops/attention/qkv_paged.py:45-68: _rms, rope,
 * the cache writes) and of _torch_qkv (ops/attention/qkv.py:57-85: rope, the FP8 divide-and-clamp, the writes); the
 * projection itself (`hidden @ weights + bias`) is a plain GEMM left to the caller. */
int sna_qkv_norm_rope_store(const void *qkv, int64_t qkv_stride, int64_t n_tokens, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t head_dim, const void *q_norm, const void *k_norm, float eps,
                            const void *cos, const void *sin, int64_t rope_stride, const int64_t *slots, void *q_out,
                            void *k_cache, void *v_cache, const float *k_scale, const float *v_scale,
                            int64_t num_blocks, int32_t page_size, int32_t cache_dtype, void *stream);

/* Per-head absmax scales, s[h] = max |x[:, h, :]| / 448, or 1 for an all-zero head.
 *   x         [n_tokens, num_heads, head_dim] bf16.
 *   scale_out [num_heads] fp32.
 *   workspace at least sna_absmax_workspace_bytes(n_tokens, num_heads) bytes of device memory.
 * This has no reference counterpart. The reference's FP8 KV scale is one per-tensor value from the checkpoint
 * (gpt_oss/mxfp4/common.py:475-487), while the per-KV-head calibration is this path's extension. */
int64_t sna_absmax_workspace_bytes(int64_t n_tokens, int32_t num_heads);
int sna_kv_absmax_scale(const void *x, int64_t n_tokens, int32_t num_heads, int32_t head_dim, float *scale_out,
                        void *workspace, int64_t workspace_bytes, void *stream);

/* Store absorbed-MLA compact rows [latent(512) | k_pe(64)] into an MLA pool layer with one scale per token.
 *   rows      [n_tokens, row_dim] bf16, with row_dim = 576 (deepseek_v2/model.py:101-111 builds them).
 *   slots     [n_tokens] int64. Out-of-pool or negative slots go to slot 0 (deepseek_v2/model.py:64-70).
 *   cache     [num_slots, row_dim] of cache_dtype (FP8: uint8 storage, memory_pool.py:313-315).
 *   row_scale [num_slots] fp32. FP8: written with s_t = max|row_t| / 448 (or 1 for a zero row), and each byte is
 *             e4m3fn_RNE(clamp(x / s_t)). Ignored for bf16.
 * Replaces: _write_rows (deepseek_v2/model.py:64-70); the pool's set_mla_kv_buffer refuses in the reference
 * (memory_pool.py:417-418). Per-token scales are this path's extension (the reference has none). */
int sna_kv_store_mla(const void *rows, const int64_t *slots, int64_t n_tokens, int32_t row_dim, void *cache,
                     float *row_scale, int64_t num_slots, int32_t cache_dtype, void *stream);

/* Quantize, pack and scatter DSA cache rows in the reference's 640-byte layout:
 *   bytes [0, 128)   k_pe: 64 bf16 = bf16_RNE(x / kv_scale)
 *   bytes [128, 640) latent: 512 e4m3fn = e4m3fn_RNE(clamp(x / kv_scale)); latent dim c = 256a + 128b + p is at byte
 *                    128 + 256a + 2p + b (kv_row_layout.py:62-84).
 *   rows   [n_tokens, 576] bf16 in [k_pe(64) | latent(512)] order (mla_decode_attention_torch.py:42).
 *   slots  [n_tokens] int64 flat row ids. A slot < 0 or >= num_rows is skipped (_scatter,
 *          mla_decode_attention_torch.py:193-201).
 *   cache  [num_rows, 640] uint8.
 * Replaces: pack_kv_rows + _scatter (mla_decode_attention_torch.py:193-221). */
int sna_kv_store_dsa(const void *rows, const int64_t *slots, int64_t n_tokens, float kv_scale, void *cache,
                     int64_t num_rows, void *stream);

/* =====================================================================================================
 * Split-K planning (host side; no device access)
 * ===================================================================================================== */

/* The split plan of a decode launch.
 *
 * GQA (kind 0): `split_tiles` is how many key tiles each split covers and `n_work` is the number of (sequence, split)
 * items the split-K kernel runs. Partials are kept per (row, split): the workspace holds batch * max_splits of them.
 * A plan whose rows all fit one split (max_splits <= 1) needs no workspace: its split-K kernel writes the final output
 * and no combine pass runs.
 *
 * MLA and DSA (kinds 1, 2): a stream split. Row b's keys (paged: the seq_len - 1 prior positions; sparse: the index
 * list) form ceil(keys / 16) tiles (at least 1), the rows' tiles are laid end to end, and workgroup w takes tiles
 * [cta_start[w], cta_start[w + 1]) of that sequence: n_ctas workgroups (one per CU) of equal tile counts, each
 * starting in row cta_row[w] at tile cta_off[w] of that row. A workgroup whose range holds a whole row writes its
 * output; a row split over several workgroups is merged inside the same launch (its workgroups publish partials and
 * the last to arrive, with those still waiting for it, merges them), so one launch is the whole decode. row_keys[b] is
 * row b's key count: an MLA or DSA launch uses these host lengths, not the device's seq_lens, unless the MLA plan is a
 * device split (device_split = 1: planned from a bound, its launch cuts the split from the device's seq_lens). */
#define SNA_MAX_WORK_MAP 512
#define SNA_MAX_CTAS 256      /* workgroups of an MLA / DSA stream split */
#define SNA_MAX_PLAN_ROWS 256 /* rows of an MLA / DSA plan */

typedef struct {
  int32_t split_tiles;
  int32_t n_work;
  int32_t tile;         /* keys per tile of the kernel family: 32 (GQA) or 16 (MLA, DSA) */
  int32_t target_ctas;  /* the workgroup count the plan aimed for */
  int32_t max_splits;   /* GQA: the most splits any row has; MLA / DSA: the most workgroups any row spans */
  int32_t batch;        /* rows the plan was made for */
  int32_t empty_rows;   /* rows with no prior key (seq_len 1), or -1 when planned from a bound (0 for a GQA device
                           split, which gives every row a split) */
  int32_t depth;        /* GQA: the plan's shape (3: one round of two 4-wave workgroups per CU, for launches with
                           enough work to fill the chip with long splits; 2: small launches of several rounds). The
                           kernels keep two tiles per wave in their register rings either way. The planner picks it;
                           splits were sized for it. */
  int32_t work_n;       /* GQA: entries in work[] (0: the kernels locate their items from the device's seq_lens) */
  uint32_t work[SNA_MAX_WORK_MAP]; /* GQA, a plan from host seq_lens with n_work and B <= SNA_MAX_WORK_MAP: item i
                           is row (work[i] & 0x7fffffff) >> 6, split work[i] & 63, bit 31 set on a row's last item, in
                           launch order (a row's items consecutive, splits 0, 1, ...). The decode kernels read it from their arguments and skip the device-side search
                           over seq_lens; a row's last item attends its own token, and its combine merges exactly the
                           row's items, even where the device's length needs fewer splits. */
  int32_t n_ctas;       /* MLA / DSA: workgroups of the stream split (per 16-head group) */
  int32_t total_tiles;  /* MLA / DSA: tiles of all rows */
  int32_t wait_polls;   /* MLA / DSA: how many times a workgroup that owns merge blocks of a split row polls for the
                           row's last partial before it hands its blocks to the last to arrive (0: the last to
                           arrive merges alone); a workgroup whose range continues into another row never polls */
  uint32_t cta_start[SNA_MAX_CTAS + 1];
  uint16_t cta_row[SNA_MAX_CTAS];
  uint16_t cta_off[SNA_MAX_CTAS];
  int32_t row_keys[SNA_MAX_PLAN_ROWS];
  int32_t device_split; /* 1 for a plan from a bound whose launch splits from the device's seq_lens, so one captured
                           launch serves every length up to the bound (0: the plan's own split). MLA: the stream split
                           (the same apportionment, by bisection of the longest piece); n_ctas is the launch's
                           workgroups per head group (the bound the workspace is sized for), row_keys the bound's key
                           count, and cta_* are unused. GQA (B <= 512 rows of at most 2^17 - 1 tiles): the split size,
                           by the planner's one-round rule on the device's lengths, to fit n_work items (the bound's
                           own item count, at least B); every row gets at least one split (a row with no prior key
                           attends and stores its own token in a split of no tile), max_splits bounds any row's, and
                           split_tiles is unused. */
} sna_split_plan;

/* Plan a decode from host copies of seq_lens (exact) or, with host_seq_lens == NULL, from an upper bound
 * max_seq_len for every row (a device-split plan, whose launch reads the device's seq_lens: GQA up to 512 rows of at
 * most 2^17 - 1 tiles of 32 keys, else the bound's own split with n_work bounding the device's count; MLA, each length held to
 * the block table's width).
 * `kind`: 0 GQA, 1 MLA, 2 DSA. For DSA, seq_lens are ignored: `n_keys_per_row` (the index-list length) is the
 * row's key count. `window` is the sliding window (0 = full). `ctas_per_item` is the number of workgroups that
 * one (sequence, split) item launches: num_kv_heads for GQA, and 1 for MLA and DSA. `num_cus` is the device's CU
 * count (0 = 256). Returns SNA_OK and fills *plan. MLA and DSA plans hold at most SNA_MAX_PLAN_ROWS rows of at most
 * 65535 tiles each. GQA: a device length needing more splits than the plan holds leaves those keys unread (all
 * reads stay inside the workspace; the row's own token is still attended and stored); a shorter one only leaves
 * splits empty. */
int sna_plan_decode(int32_t kind, const int32_t *host_seq_lens, int32_t B, int32_t max_seq_len, int32_t window,
                    int32_t n_keys_per_row, int32_t ctas_per_item, int32_t num_cus, sna_split_plan *plan);

/* Workspace bytes a decode with this plan needs. GQA: batch * max_splits * heads * (head_dim_v + 2) * 4 (+ 256 for
 * a device split: the launch's split size, for its combine pass), or 0 when max_splits <= 1. MLA / DSA: a 256 KiB block of counters, then 2 * n_ctas partials of heads * (head_dim_v + 2) fp32.
 * The counters must be zero before the first call on a workspace (allocate it zeroed); every completed call leaves
 * them zero. Calls that share a workspace must be ordered (one stream). */
int64_t sna_decode_workspace_bytes(const sna_split_plan *plan, int32_t num_q_heads, int32_t head_dim_v);

/* The MLA / DSA workspace's counter block, checked and repaired. It has no counterpart in the reference (its NKI
 * kernels keep no state across launches); it is for callers that want to know a merge could not be trusted. A launch
 * that finds a counter past what a zeroed block allows sets a sticky status bit: SNA_WS_DIRTY_ARRIVAL (a row's
 * arrival count past its workgroups: the block was not zero on entry, or two launches overlapped on it; that row's
 * output is unreliable) or SNA_WS_DIRTY_DONE (the finished-workgroups count past the grid: the counters may no longer
 * return to zero by themselves).
 * sna_stream_workspace_status waits for `stream`, returns the status word in *status (0: every launch since the last
 * call found the block clean) and clears it. sna_stream_workspace_reset zeroes the counter block on `stream` (a fill
 * kernel, no memset, so it may be captured); launches ordered after it find it clean. workspace_bytes is the
 * workspace's size (at least the counter block). */
#define SNA_WS_DIRTY_ARRIVAL 1
#define SNA_WS_DIRTY_DONE 2
int sna_stream_workspace_status(void *workspace, int64_t workspace_bytes, int32_t *status, void *stream);
int sna_stream_workspace_reset(void *workspace, int64_t workspace_bytes, void *stream);

/* Host check of one decode batch's operands, before any launch (host copies of every array):
 *   seq_lens     [B] int64, prefix plus the new token: each in [1, INT32_MAX] (positions are int32 in the kernels).
 *   block_table  [B, table_stride] int32, table_width valid columns: a row's ceil(seq_len / page_size) pages must fit
 *                the table and name pages inside the pool [0, num_blocks) (a -1 inside a row would drop its keys).
 *   new_slots    [B] int64 or NULL: a live row's slot lies inside the pool off the reserved page 0, at the row's
 *                position in its page, slot % page == (seq_len - 1) % page, on the row's last page, and no two live
 *                rows share one. A row that is not live is a padding row: its write is redirected to slot 0 and not
 *                checked.
 *   active       [B] int32 or NULL: 1 for a live row (the reference's active flags). NULL: a row is live unless it is
 *                a padding row by its operands, its own token only (seq_len 1) written to page 0 or outside the pool.
 * Returns SNA_ERR_INVALID_ARGUMENT naming the first offending row. The decode entry points themselves check shapes
 * only (their operands are device memory).
 * Replaces: the refusals of decode_operands (attention/mla_operands.py:54-97: an int32 position bound, a live row's
 * slot that disagrees with its position, a table too narrow for the row, two live rows sharing a write slot). */
int sna_check_decode_operands(const int64_t *seq_lens, const int32_t *block_table, int64_t table_stride,
                              int32_t table_width, const int64_t *new_slots, const int32_t *active, int32_t B,
                              int32_t page_size, int64_t num_blocks);

/* =====================================================================================================
 * Decode attention
 * ===================================================================================================== */

/* GQA paged decode over an MHA pool layer, with the step's own token attended in-band and optionally stored.
 *   q            [B, num_q_heads, head_dim] bf16 (after projection, QK norm and RoPE).
 *   k_cache, v_cache
 *                [num_blocks, num_kv_heads, page_size, head_dim] of cache_dtype.
 *   k_scale, v_scale
 *                [num_kv_heads] fp32, FP8 only (NULL for bf16): dequantization scales s (SNA_DTYPE_FP8_E4M3FN), or the
 *                GPT-OSS quantization multipliers m (SNA_DTYPE_FP8_E4M3FN_MUL: a cached byte is worth byte / m, and the
 *                step's token is stored and attended as the decode write of attention_decode.py:259-260 rounds it).
 *   block_table  [B, table_stride] int32, of which `table_width` columns are valid; -1 marks no page.
 *   seq_lens     [B] int32, prefix plus the new token (>= 1).
 *   k_new, v_new [B, num_kv_heads, head_dim] bf16: the step's token. With an FP8 cache it is attended as
 *                dequant(quant(x)), the value the store writes (attention_decode.py:259-269).
 *   new_slots    [B] int64 or NULL. If not NULL, the decode also stores k_new / v_new at these slots, bit-exact
 *                with sna_kv_store_mha of the same cache_dtype. Positions < seq_len - 1 are read, so the store never
 *                races the reads.
 *   sinks        [num_q_heads] fp32 or NULL. exp(sink_h - max) joins the softmax denominator
 *                (attention_decode.py:274-275).
 *   window       0 for full attention, or W > 0: keys at positions [seq_len - W, seq_len - 1], the new one
 *                included (gpt_oss/attention_masks.py:47-52; swa_fused.py:115).
 *   sm_scale     softmax scale applied to q.k (dequantized k).
 *   out          [B, num_q_heads, head_dim] bf16.
 *   plan, workspace
 *                from sna_plan_decode(kind 0) and at least sna_decode_workspace_bytes(plan, num_q_heads, head_dim).
 * A key at position p < seq_len - 1 is visible iff its table entry is >= 0, lies in [0, num_blocks), and p is in
 * the window. This is the reference's mask (attention_decode_paged.py:165-166, attention_decode_mask.py:64-81).
 * Scores, softmax and accumulation are fp32. The group num_q_heads / num_kv_heads must be <= 16.
 * Replaces: the attention core of _torch_attention_decode_paged (attention_decode_paged.py:159-177) and of
 * _torch_attention_decode (attention_decode.py:259-300), which nkilib's attention_block_tkg runs on Trainium
 * (attention_decode_paged.py:63-126). */
int sna_paged_decode_gqa(const void *q, const void *k_cache, const void *v_cache, const float *k_scale,
                         const float *v_scale, const int32_t *block_table, int64_t table_stride, int32_t table_width,
                         const int32_t *seq_lens, const void *k_new, const void *v_new, const int64_t *new_slots,
                         const float *sinks, int32_t window, float sm_scale, void *out, int32_t B,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                         int64_t num_blocks, int32_t cache_dtype, const sna_split_plan *plan, void *workspace,
                         int64_t workspace_bytes, void *stream);

/* sna_paged_decode_gqa for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). It has no counterpart in the reference. Same arguments and results as
 * sna_paged_decode_gqa without the workspace: the split partials go to a scratch array of
 * SNA_NOALLOC_SCRATCH_BYTES (16 MiB) that the library holds on each GPU it runs on until the process ends (its device
 * address is looked up on the first call on a device). A plan whose partials need more is refused with
 * SNA_ERR_WORKSPACE. Nothing is allocated, freed or cleared per call: every partial a combine pass reads was written
 * by the same call. Calls that overlap on one GPU (other streams, other threads) share the array and race; serialize
 * them. */
#define SNA_NOALLOC_SCRATCH_BYTES (16ll << 20)
int sna_paged_decode_gqa_noalloc(const void *q, const void *k_cache, const void *v_cache, const float *k_scale,
                                 const float *v_scale, const int32_t *block_table, int64_t table_stride,
                                 int32_t table_width, const int32_t *seq_lens, const void *k_new, const void *v_new,
                                 const int64_t *new_slots, const float *sinks, int32_t window, float sm_scale,
                                 void *out, int32_t B, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t page_size, int64_t num_blocks, int32_t cache_dtype,
                                 const sna_split_plan *plan, void *stream);

/* Absorbed-MLA paged decode over an MLA pool layer of compact rows [latent(512) | k_pe(64)].
 *   ql_nope      [B, num_heads, 512] bf16 (W_UK folded in); q_pe [B, num_heads, 64] bf16 (RoPE'd).
 *   cache        [num_blocks * page_size, 576] of cache_dtype; row_scale [num_blocks * page_size] fp32 (FP8).
 *   block_table, seq_lens
 *                as for GQA. History keys are positions < seq_len - 1 (mla.py:48-50).
 *   compact_new  [B, 576] bf16: the step's own row, attended in-band as dequant(quant(row)) with its own
 *                per-token scale.
 *   new_slots    [B] int64 or NULL: also store compact_new there, bit-exact with sna_kv_store_mla.
 *   out          [B, num_heads, 512] bf16. Scores are fp32 sm_scale * (ql_nope . latent + q_pe . k_pe), softmax is
 *                fp32, out = probs . latent.
 * Replaces: mla_decode (ops/attention/mla.py:32-53). On Trainium that is paged_absorbed_mla
 * (nki/deepseek_mla_decode.py:510-557). */
int sna_mla_decode(const void *ql_nope, const void *q_pe, const void *cache, const float *row_scale,
                   const int32_t *block_table, int64_t table_stride, int32_t table_width, const int32_t *seq_lens,
                   const void *compact_new, const int64_t *new_slots, float sm_scale, void *out, int32_t B,
                   int32_t num_heads, int32_t page_size, int64_t num_blocks, int32_t cache_dtype,
                   const sna_split_plan *plan, void *workspace, int64_t workspace_bytes, void *stream);

/* DSA sparse absorbed-MLA decode over 640-byte packed rows (spec query tokens per sequence, one CP rank).
 *   B            query tokens: B / spec sequences of spec tokens each (spec 1: one per sequence; GLM's MTP verify
 *                runs spec 8), sequence s owning rows s * spec .. s * spec + spec - 1.
 *   q_absorbed   [B, num_heads, 512] bf16; q_pe [B, num_heads, 64] bf16.
 *   cache        [num_blocks * page_size, 640] uint8 (sna_kv_store_dsa's layout); kv_scale is per tensor.
 *   indices      [B, n_indices] int32 global token positions, per query token; < 0 entries are empty.
 *   block_table  [B / spec, table_stride] int32 per sequence (logical block -> physical block); `table_width` valid
 *                columns.
 *   positions    [B] int32, each query token's absolute position.
 *   own_rows     [B, 576] bf16 in [k_pe | latent] order: the step's rows. Each token attends its own row and its
 *                sequence's other spec - 1 rows from their packed bytes, at their positions (kept iff <= its own),
 *                whatever their slots or table entries (mla_decode_attention_torch.py:89-103, 181-190).
 *   new_slots    [B] int64 or NULL: the cache rows the own rows are stored to in this launch, bit-exact with
 *                sna_kv_store_dsa (a slot < 0 or past the cache is skipped; of rows sharing a slot the last one's
 *                bytes land). As in the reference, where steps 0-1 store every own row before any gather, an index
 *                resolving to such a row attends the stored bytes. NULL: the caller has stored them
 *                (sna_kv_store_dsa) before the launch.
 *   ctx_out      [B, num_heads, 512] bf16; lse_out [B, num_heads] fp32 (natural log), or NULL.
 * Position pos resolves to row table[pos / page_size] * page_size + pos % page_size. It is dropped when pos < 0,
 * its block is outside the table or unallocated, or the row is outside the cache. A resolved key is kept iff
 * pos <= position, and the own row always is.
 * plan: from sna_plan_decode(kind 2) with n_keys_per_row = n_indices + spec - 1 (a row's keys: its index list, then
 * its siblings' rows).
 * Replaces: mla_decode_attention_torch_ref with cp_degree = 1 (mla_decode_attention_torch.py:38-130).
 * On Trainium that is mla_decode_attention (models/glm52/kernels/decode/attention/mla/mla_decode_attention.py:207). */
int sna_mla_decode_sparse(const void *q_absorbed, const void *q_pe, const void *cache, float kv_scale,
                          const int32_t *indices, int32_t n_indices, const int32_t *block_table, int64_t table_stride,
                          int32_t table_width, const int32_t *positions, const void *own_rows,
                          const int64_t *new_slots, float sm_scale, void *ctx_out, float *lse_out, int32_t B,
                          int32_t spec, int32_t num_heads, int32_t page_size,
                          int64_t num_blocks, const sna_split_plan *plan, void *workspace, int64_t workspace_bytes,
                          void *stream);

/* Log-sum-exp merge of partial attention results, e.g. one per decode-context-parallel rank:
 *   o_parts   [n_parts, n_rows, dim] fp32, each normalized by its own softmax sum.
 *   lse_parts [n_parts, n_rows] fp32 natural-log LSE (-inf for an empty part).
 *   out       [n_rows, dim] bf16 = sum_i exp(lse_i - LSE) o_i, LSE = logsumexp_i lse_i. lse_out [n_rows] or NULL.
 * Replaces: the DCP merge (attention_decode.py:277-285) and the CP softmax combine of
 * models/glm52/kernels/decode/attention_layer.py:653. */
int sna_lse_combine(const float *o_parts, const float *lse_parts, int32_t n_parts, int64_t n_rows, int32_t dim,
                    void *out, float *lse_out, void *stream);

/* =====================================================================================================
 * Prefill attention over the pool
 * ===================================================================================================== */

/* Segmented prefill attention: a chunk's queries attend to their request's prior and, causally, to the chunk
 * itself, every key read from the pool (store the chunk's K/V first, e.g. with sna_kv_store_mha).
 *   q            [T, num_q_heads, head_dim] bf16, contiguous, 16-byte aligned; request r owns rows
 *                q_start[r] .. q_start[r + 1] - 1, its query i at position prior_lens[r] + i.
 *   k_cache, v_cache  one layer's pool [num_blocks, num_kv_heads, page_size, head_dim]: FP8 e4m3fn
 *                (kv_dtype SNA_DTYPE_FP8_E4M3FN) with per-KV-head dequantization scales k_scale / v_scale
 *                [num_kv_heads], FP8 e4m3fn with GPT-OSS multipliers (SNA_DTYPE_FP8_E4M3FN_MUL: a byte is worth
 *                byte / m, the dequantization model_prefill.py:103-108 folds into the softmax scale and the output),
 *                or bf16 (SNA_DTYPE_BF16; the scales are not read and may be NULL).
 *   block_table  [R, table_width] int32 (row stride table_stride), -1 past a row's pages; keys on a -1 page are not
 *                attended.
 *   q_start      [R + 1] int32, prior_lens [R] int32 (device); max_q_len >= every request's chunk length.
 *   sinks        [num_q_heads] fp32 logits joining the softmax denominator, or NULL. window > 0: the query at
 *                position p sees keys (p - window, p].
 *   out          [T, num_q_heads, head_dim] bf16.
 * head_dim 64 or 128, page_size a multiple of 16, num_q_heads / num_kv_heads <= 128.
 * Replaces: segmented_attention (ops/attention/attention_segmented_cte.py:21-47, its torch path :50-75) and the
 * attention of the fused sliding-window prefill (ops/attention/swa_fused.py:78-120), which reads the chunk's own
 * K/V unquantized where this reads them back from the pool. */
int sna_prefill_attention(const void *q, const void *k_cache, const void *v_cache, const float *k_scale,
                          const float *v_scale, const int32_t *block_table, int64_t table_stride, int32_t table_width,
                          const int32_t *q_start, const int32_t *prior_lens, int32_t R, int32_t max_q_len,
                          const float *sinks, float sm_scale, int32_t window, void *out, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_blocks,
                          int32_t kv_dtype, void *stream);

/* =====================================================================================================
 * DSA indexer (the step that picks the sparse decode's positions)
 * ===================================================================================================== */

/* Store index-key rows keys [n_tokens, head_dim] bf16 (16-byte aligned) into an index-key cache [n_slots, head_dim]
 * of e4m3fn bytes as e4m3fn(clamp(key, +-448)) (no scale); slots < 0 or >= n_slots are skipped.
 * Replaces: pack_indexer_keys_fp8 and the cache append of indexer_kv_score_torch_ref
 * (models/glm52/kernels/decode/attention/indexer/indexer_torch.py:44-53, :228-234). */
int sna_index_key_store(const void *keys, const int64_t *slots, int64_t n_tokens, int32_t head_dim, uint8_t *cache,
                        int64_t n_slots, void *stream);

/* Index scores of every cached key: out[b, e] (bf16, row stride out_stride, e < width) =
 *   bf16(min(sum_h w[b, h] * relu(q[b, h, :] . key_e * head_dim^-0.5), live ? 1e30 : -1e30)),
 * key e of row b read at page block_table[b, e / page_size], offset e % page_size of keys [num_blocks, page_size,
 * head_dim] (e4m3fn bytes); live: e < limits[b] (positions before the query's own) and the page valid.
 *   q [B, num_heads, 128] bf16 (the rotated index queries, 16-byte aligned), w [B, num_heads] fp32 (the head weights,
 *   already scaled by num_heads^-0.5); num_heads 16, 32, 64 or 128; head_dim 128.
 * Replaces: the score of indexer_kv_score_torch_ref (indexer_torch.py:254-268), after the model's projections. */
int sna_indexer_scores(const void *q, const float *w, const uint8_t *keys, const int32_t *block_table,
                       int64_t table_stride, int32_t table_width, const int32_t *limits, int32_t B, int32_t num_heads,
                       int32_t head_dim, int32_t page_size, int64_t num_blocks, int32_t width, void *out,
                       int64_t out_stride, void *stream);

/* The k largest of each row of bf16 scores [B, width] (row stride score_stride): out[b, 0 .. k) int32 (row stride
 * out_stride) = their positions e, those above the k-th largest value first, then its ties (the lowest positions),
 * each group in position order; a selected score <= -1e30 / 2 (a dead key) is written as -1. Exact: the selected
 * values are the k largest. B <= 65535. workspace: device memory of at least sna_topk_workspace_bytes(B, width)
 * bytes, 4-byte aligned, any contents (every word is written before it is read); calls that share a workspace on
 * different streams race.
 * Replaces: indexer_topk_local_torch_ref's selection (indexer_torch.py:296-309); its slot order is a Trainium
 * layout, the set is the same. */
int64_t sna_topk_workspace_bytes(int32_t B, int32_t width);
int sna_topk_positions(const void *scores, int64_t score_stride, int32_t B, int32_t width, int32_t k, int32_t *out,
                       int64_t out_stride, void *workspace, int64_t workspace_bytes, void *stream);

/* =====================================================================================================
 * Decode metadata on the device
 * ===================================================================================================== */

/* The decode block table from SGLang's req_to_token map, built on the device (no host view, no upload):
 *   req_to_token      [r2t_rows, r2t_width] int32 token slots, row stride r2t_stride elements.
 *   req_pool_indices  [B] int64 rows of req_to_token; seq_lens [B] int64 (prefix + new token).
 *   table             [B, width] int32 out, contiguous: table[b, j] = floor(req_to_token[row_b, j * page_size] /
 *                     page_size) while j * page_size < seq_len_b, else -1. A row index outside [0, r2t_rows), or a
 *                     column whose first token lies past req_to_token's width, gives -1.
 *   seq_lens_i32      [B] int32 out (seq_lens narrowed for the decode entry points), or NULL.
 * With width = ceil(max seq_len / page_size) the table is the reference's, entry for entry.
 * Replaces: NeuronAttnBackend._block_table (attention/backend.py:114-130), which builds it on the host from a numpy
 * view of req_to_token every step. */
int sna_block_table(const int32_t *req_to_token, int64_t r2t_rows, int64_t r2t_width, int64_t r2t_stride,
                    const int64_t *req_pool_indices, const int64_t *seq_lens, int32_t B, int32_t page_size,
                    int32_t width, int32_t *table, int32_t *seq_lens_i32, void *stream);

/* A sliding-window layer's trimmed block table, built on the device:
 *   table      [B, table_width] int32, row stride table_stride elements; seq_lens [B] int64.
 *   trimmed    [B, n_blocks] int32 out, contiguous: trimmed[b, i] = table[b, start_b + i], -1 past table_width, with
 *              start_b = max(floor((seq_len_b - 1) / page_size) - n_blocks + 1, 0).
 *   pos_offset [B] int32 out: start_b * page_size, the position of the trimmed table's first key.
 * Replaces: the decode window trim of model_executor/graph_runner.py:1121-1133 (host torch ops, then an upload). */
int sna_window_table(const int32_t *table, int64_t table_stride, int32_t table_width, const int64_t *seq_lens,
                     int32_t B, int32_t page_size, int32_t n_blocks, int32_t *trimmed, int32_t *pos_offset,
                     void *stream);

/* =====================================================================================================
 * Page items: what a prefill-decode transfer moves
 * ===================================================================================================== */

/* A pool's regions as its get_contiguous_buf_infos gives them (host arrays of n_regions): region r is region_lens[r]
 * bytes at device address region_ptrs[r], page p its item_lens[r] bytes at region_ptrs[r] + p * item_lens[r]
 * (addresses and item sizes multiples of 16, items under 2 GiB, under 2^31 items a region). pages: device int32
 * [n_pages]. Every call moves whole items, one workgroup per (page, region), in launches of up to 96 regions on
 * `stream`.
 * Replaces: the page-item addressing of NeuronMHATokenToKVPool.get_contiguous_buf_infos (mem_cache/memory_pool.py:
 * 193-202) and the transfer's per-item WRITE (disaggregation/state_transfer.py:9-10), on one GPU. */

/* The wire bytes of n_pages pages over the regions: n_pages * sum(item_lens); -1 for bad arguments. */
int64_t sna_page_items_wire_bytes(const int64_t *item_lens, int32_t n_regions, int64_t n_pages);

/* Gathers the items (r, pages[i]) into `wire`, region-major: region r's items start at n_pages * (sum of item_lens
 * before r), item i at + i * item_lens[r]. A page outside region r (negative or >= region_lens[r] / item_lens[r])
 * writes zeros in its place. wire: device, 16-B aligned, at least sna_page_items_wire_bytes bytes. */
int sna_page_items_pack(const uint64_t *region_ptrs, const int64_t *region_lens, const int64_t *item_lens,
                        int32_t n_regions, const int32_t *pages, int64_t n_pages, void *wire, int64_t wire_bytes,
                        void *stream);

/* Scatters a wire buffer of sna_page_items_pack's layout into the items (r, pages[i]); a page outside region r is
 * skipped. pages must be distinct (two writes of one item race). */
int sna_page_items_unpack(const void *wire, int64_t wire_bytes, const uint64_t *region_ptrs,
                          const int64_t *region_lens, const int64_t *item_lens, int32_t n_regions,
                          const int32_t *pages, int64_t n_pages, void *stream);

/* Copies item (r, src_pages[i]) of the source regions to item (r, dst_pages[i]) of the destination regions, both
 * with items of item_lens[r] bytes (a destination block of a larger page is addressed in units of the source item,
 * as a stripe into a replicated page is); an item whose source or destination page is outside its region is skipped.
 * dst_pages must be distinct. */
int sna_page_items_copy(const uint64_t *src_ptrs, const int64_t *src_lens, const uint64_t *dst_ptrs,
                        const int64_t *dst_lens, const int64_t *item_lens, int32_t n_regions,
                        const int32_t *src_pages, const int32_t *dst_pages, int64_t n_pages, void *stream);

/* ---- diagnostics ---- */

/* Decode n e4m3fn bytes to bf16 bits with the conversion instruction the decode kernels use for gathered pages. It
 * lets a test compare that instruction with the exact decoding on all 256 byte values. */
int sna_diag_fp8_to_bf16(const uint8_t *in, uint16_t *out, int64_t n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SGLANG_NEURON_AMD_H_ */

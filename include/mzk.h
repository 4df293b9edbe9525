/* mzk.h -- C ABI of the mzoo_amd HIP library (MI355X / gfx950).
 *
 * Drop-in boundary for the DeepSeek-V4.1-style sparse-attention inference path of
 * pmonad/mzoo.  Every entry point:
 *   - takes raw device pointers, explicit sizes and a hipStream_t (passed as void*);
 *   - never allocates, frees or synchronises (callers own every buffer, so the calls
 *     can be recorded into a HIP graph);
 *   - returns MZK_OK (0) or a negative status; mzk_last_error() then describes it.
 * Citations name the reference interface each entry point replaces
 * (paths relative to the reference repository root).
 */
#ifndef MZK_H
#define MZK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MZK_OK 0
#define MZK_EINVAL (-1)       /* bad argument (shape, dtype, null pointer) */
#define MZK_EUNSUPPORTED (-2) /* valid request this build does not implement */
#define MZK_ELAUNCH (-3)      /* the HIP launch itself failed */

/* element dtypes of floating-point tensors */
#define MZK_F32 0
#define MZK_BF16 1
#define MZK_F16 2

/* Library version (major*10000 + minor*100 + patch). */
int mzk_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char* mzk_last_error(void);

/* ---------------------------------------------------------------------------------
 * Piece 1: block quantizers (src/mzoo/archs/owlet1/quant.py)
 * --------------------------------------------------------------------------------- */

/* _fake_quant_fp8_block(x, block_size)  -- owlet1/quant.py:72-86.
 * x, y: [rows, n] of `dtype`, row-major.  y may alias x.  n % block_size must be 0
 * (the reference's pass-through for other n is the caller's job). */
int mzk_fake_quant_fp8_block(const void* x, void* y, int dtype, int64_t rows, int64_t n,
                             int block_size, void* stream);

/* _fake_quant_fp4_block(x, block_size, e4m3_scales)  -- owlet1/quant.py:49-66. */
int mzk_fake_quant_fp4_block(const void* x, void* y, int dtype, int64_t rows, int64_t n,
                             int block_size, int e4m3_scales, void* stream);

/* Packed form of _fake_quant_fp8_block (owlet1/quant.py:81-85): codes [rows, n] e4m3
 * bytes and scales [rows, n/block_size] fp32 (powers of two).  Used for the FP8
 * indexer queries/keys (SGLang/DeepSeek V3.2 layout: 128 codes + 1 fp32 per row). */
int mzk_quant_fp8_block(const void* x, int dtype, int64_t rows, int64_t n, int block_size,
                        uint8_t* codes, float* scales, void* stream);

/* Packed MXFP4 of _fake_quant_fp4_block(x, 32) (owlet1/quant.py:49-66, the indexer's
 * quantizer at owlet1/indexer.py:106,129): packed [rows, n/2] (element 2i in the low
 * nibble), e8m0 [rows, n/32] (scale = 2^(byte-127)). */
int mzk_quant_mxfp4(const void* x, int dtype, int64_t rows, int64_t n, uint8_t* packed,
                    uint8_t* e8m0, void* stream);

/* Dequantizers of the two packed forms above, to `dtype`. */
int mzk_dequant_fp8_block(const uint8_t* codes, const float* scales, int64_t rows, int64_t n,
                          int block_size, void* y, int dtype, void* stream);
int mzk_dequant_mxfp4(const uint8_t* packed, const uint8_t* e8m0, int64_t rows, int64_t n,
                      void* y, int dtype, void* stream);

/* FP8-b128 latent cache entry (FlashMLA V3.2 / SGLang DSA layout,
 * layers/attn/fp_attn_notes.md:1085-1131): [nope e4m3 | nope/128 fp32 scales | rope bf16].
 * 656 bytes at nope=512, rope=64.  The nope slice is _fake_quant_fp8_block(., 128)
 * (owlet1/quant.py:72-86); the rope slice is stored as bf16.
 * x: [rows, nope+rope] of `dtype`.  Row i is written to entry dst_index[i] of `cache`
 * (dst_index may be NULL: entry i).  This is the cache write of
 * DeepseekV41CSACache.update / update_compressor_states (owlet1/cache.py:84-124). */
int mzk_pack_latent_fp8_b128(const void* x, int dtype, int64_t rows, int nope, int rope,
                             const int64_t* dst_index, uint8_t* cache, void* stream);
int mzk_unpack_latent_fp8_b128(const uint8_t* cache, int64_t rows, int nope, int rope, void* y,
                               int dtype, void* stream);

/* DeepSeek-V4.1 cache entries, FlashMLA's kv_cache_format ("V4.1" and "V4.1 fp4" rows):
 *   fmt 0: [D e4m3 codes][D/32 e8m0 scale bytes] -- _fake_quant_fp8_block(x, 32)
 *          (owlet1/quant.py:72-86; the window cache of owlet1/attention.py:154); D=512: 528 B
 *   fmt 1: [D/2 e2m1 bytes, element 2i in the low nibble][D/16 e4m3 scale bytes]
 *          -- _fake_quant_fp4_block(x, 16, e4m3_scales=True) (quant.py:49-66; the
 *          compressed cache of attention.py:183); D=512: 288 B
 * x [rows, D] (D a multiple of 32, dtype 0/1/2, 16-byte aligned); entry r goes to cache row
 * dst_index[r] (or r when dst_index is NULL).  Unpacking gives exactly the fake-quantized
 * values. */
int mzk_pack_cache_v41(const void* x, int dtype, int64_t rows, int D, int fmt, uint8_t* out,
                       const int64_t* dst_index, void* stream);
int mzk_unpack_cache_v41(const uint8_t* cache, int64_t rows, int D, int fmt, void* y, int dtype,
                         void* stream);

/* Decode-step prologue in one launch, for one new token per batch row:
 *  (1) the token's latent kv [B, nope+rope] (kv_dtype) into its window-ring slot, entry
 *      b*win_batch_entries + positions[b] % win_cap of win_cache (FP8-b128 entries as
 *      mzk_pack_latent_fp8_b128) -- the window write of DeepseekV41CSACache.update
 *      (owlet1/cache.py:84-94), with the ring slot derived on the device;
 *  (2) the indexer query quantization (owlet1/indexer.py:129): q_idx [q_rows, q_dim]
 *      (q_dtype) to FP8 b128 (q_format 0: q_codes [q_rows, q_dim] e4m3 + q_scales
 *      [q_rows, q_dim/128] fp32, as mzk_quant_fp8_block) or MXFP4 (q_format 1: q_codes =
 *      packed [q_rows, q_dim/2] + q_e8m0 [q_rows, q_dim/32], as mzk_quant_mxfp4). */
int mzk_decode_prologue(const void* kv, int kv_dtype, int64_t B, int nope, int rope,
                        const int64_t* positions, uint8_t* win_cache, int64_t win_batch_entries,
                        int win_cap, const void* q_idx, int q_dtype, int64_t q_rows, int q_dim,
                        int q_format, uint8_t* q_codes, float* q_scales, uint8_t* q_e8m0,
                        void* stream);

/* Group emission inside a decode step, for one new token per batch row (positions [B]):
 * the per-token work of DeepseekV41Compressor.forward with its cache layer
 * (owlet1/cache.py:96-124, :159-172), the compressed-cache append (owlet1/attention.py:173-192)
 * and the indexer's key publication (owlet1/indexer.py:96-117), with all state on the device.
 *   kv, gate    fp32 [B, 576]: the token's compressor projections (gate unused at ratio 1)
 *   carry_kv/_gate  fp32 [B, ratio, 576]: the partial group; the token goes to slot pos % ratio
 * When (pos + 1) % ratio == 0 the row's group g = (pos+1)/ratio - 1 (if g < cache_cap):
 *   latent = RMSNorm(bf16(sum_r kv_r * softmax_r(gate_r)))  (norm_weight bf16 [576], eps;
 *            the pinned order of mzk_compress), bf16;
 *   cache entry b*cache_batch_entries + g = FP8-b128 of the latent with its trailing 64
 *            channels rotated at position g*ratio (row g*ratio of rope_table);
 *   with wk (bf16 [128, 576]): key = RoPE(k_norm(bf16(latent . wk^T))) -- 8 partials per output
 *            (partial j: 16-byte chunks j, j+8, ... in order) meet in an xor butterfly --, quantized as key
 *            b*key_batch_entries + g: key_format 0 FP8 b128 (k_codes [.., 128] e4m3 +
 *            k_scales fp32), 1 MXFP4 (k_codes [.., 64] e2m1 + k_scales e8m0 [.., 4]).
 * rope_table: bf16 [table_rows, 64], row p = cos (32) | sin (32) of position p (the compress
 * RoPE).  step_cos / step_sin (bf16 [B, 32], or NULL): receive row pos of the table -- the
 * token's RoPE for the step's later launches.  Rows with pos < 0 do nothing.  Limit: every
 * position must be below table_rows -- a row at pos >= table_rows gets no step tables and no
 * prologue (its step_cos / step_sin, window slot and quantized query keep their previous
 * contents, with no error); SparseDecodeLayer refuses such positions on the host.
 * The step's prologue (kv_proj non-NULL), at the token's RoPE (row pos of the table):
 *   kv_proj bf16 [B, 576] (the wkv projection) -> RoPE(kv_norm(kv_proj)) (kv_weight bf16 [576],
 *            kv_eps; the pinned order of mzk_rms_norm) packed FP8-b128 into window-ring slot
 *            b*win_batch_entries + pos % win_cap (owlet1/attention.py:149-154), as
 *            mzk_decode_prologue;
 *   q_idx bf16 [B, 64, 128] (or NULL) -> RoPE of channels 64..127 (owlet1/indexer.py:126-128),
 *            quantized per head: q_format 0 FP8 b128 (q_codes [B, 64, 128] e4m3 + q_scales
 *            fp32 [B, 64]), 1 MXFP4 (q_codes [B, 64, 64] e2m1 + q_scales e8m0 [B, 64, 4]) --
 *            the query operands of mzk_indexer_scores_fp8 / _mxfp4. */
int mzk_decode_emit(const int64_t* positions, int64_t B, const float* kv, const float* gate, float* carry_kv,
                    float* carry_gate, int ratio, const void* norm_weight, float eps, uint8_t* cache,
                    int64_t cache_batch_entries, int64_t cache_cap, const void* wk, const void* k_norm_weight,
                    float k_eps, int key_format, uint8_t* k_codes, void* k_scales, int64_t key_batch_entries,
                    const void* rope_table, int64_t table_rows, void* step_cos, void* step_sin,
                    const void* kv_proj, const void* kv_weight, float kv_eps, uint8_t* win_cache,
                    int64_t win_batch_entries, int win_cap, const void* q_idx, int q_format, uint8_t* q_codes,
                    void* q_scales, void* stream);

/* The two compressors of a hierarchical decode step (owlet1/cache.py:96-124, :159-172 with the
 * 4x fine compressor and the dense coarse one, owlet1/attention.py:173-192) in one launch: the
 * fine branch exactly as mzk_decode_emit with the arguments up to q_scales, and a coarse
 * branch without index key, prologue or step tables -- as mzk_decode_emit(positions, B,
 * c_kv, c_gate, c_carry_kv, c_carry_gate, c_ratio, c_norm_weight, c_eps, c_cache,
 * c_cache_batch_entries, c_cache_cap, NULL, ..., rope_table, table_rows, NULL, ...) -- the
 * same results as those two calls.  One kernel when the fine ratio is 4 and the coarse
 * ratio 2..128 with B <= 1024 rows (else the two launches).  Both branches share positions
 * and the RoPE table. */
int mzk_decode_emit_pair(const int64_t* positions, int64_t B, const float* kv, const float* gate, float* carry_kv,
                         float* carry_gate, int ratio, const void* norm_weight, float eps, uint8_t* cache,
                         int64_t cache_batch_entries, int64_t cache_cap, const void* wk, const void* k_norm_weight,
                         float k_eps, int key_format, uint8_t* k_codes, void* k_scales, int64_t key_batch_entries,
                         const void* rope_table, int64_t table_rows, void* step_cos, void* step_sin,
                         const void* kv_proj, const void* kv_weight, float kv_eps, uint8_t* win_cache,
                         int64_t win_batch_entries, int win_cap, const void* q_idx, int q_format, uint8_t* q_codes,
                         void* q_scales, const float* c_kv, const float* c_gate, float* c_carry_kv,
                         float* c_carry_gate, int c_ratio, const void* c_norm_weight, float c_eps, uint8_t* c_cache,
                         int64_t c_cache_batch_entries, int64_t c_cache_cap, void* stream);

/* The decode step's group emission and indexer scores in one launch (owlet1/cache.py:96-124,
 * :159-172 and owlet1/indexer.py:96-143 for one token per row): the same results as
 * mzk_decode_emit (ratio 4, with the index key wk and the kv prologue; q_idx NULL) followed
 * by mzk_indexer_decode_fused over the emitted keys with the query's RoPE from row `pos` of
 * rope_table -- the carry, caches, keys, window entry, step tables and scores bit for bit.
 * The emission arguments are mzk_decode_emit's up to win_cap; then q_idx bf16 [B, Hi, 128]
 * (unrotated; its trailing 64 channels rotated with the table row), w fp32 [B, Hi] (already
 * x Hi^-0.5), Hi <= 64 index heads, G keys per row (key batch stride key_batch_entries,
 * format key_format), scores fp32 [B, score_stride] (-inf at and beyond the visible count).
 * With c_kv non-NULL a keyless coarse branch joins the launch, as mzk_decode_emit_pair's
 * (c_* arguments; c_ratio 2 .. 128, B <= 1024).  Per row one workgroup emits the fine group
 * (and scores the new key itself), one writes the window entry, 9 pool the coarse group, and
 * ceil(G / K) score, K = 512, 1024 or 2048 keys: the least that leaves at most one scoring
 * workgroup per compute unit.  On a group step the window workgroup computes half of the
 * key projection and hands it to the emission workgroup through key_half, int64 [B, 40]
 * (16-byte aligned, zero before the first call; the launch keeps a per-row count of group
 * steps there, and word 33 of a row turns nonzero, and stays, if the emission workgroup gave
 * up waiting).  Calls that overlap on one key_half race.  ratio must be 4 (MZK_EINVAL
 * otherwise). */
int mzk_decode_emit_scores(const int64_t* positions, int64_t B, const float* kv, const float* gate, float* carry_kv,
                           float* carry_gate, int ratio, const void* norm_weight, float eps, uint8_t* cache,
                           int64_t cache_batch_entries, int64_t cache_cap, const void* wk, const void* k_norm_weight,
                           float k_eps, int key_format, uint8_t* k_codes, void* k_scales, int64_t key_batch_entries,
                           const void* rope_table, int64_t table_rows, void* step_cos, void* step_sin,
                           const void* kv_proj, const void* kv_weight, float kv_eps, uint8_t* win_cache,
                           int64_t win_batch_entries, int win_cap, const void* q_idx, const float* w, int Hi,
                           int64_t G, float* scores, int64_t score_stride, const float* c_kv, const float* c_gate,
                           float* c_carry_kv, float* c_carry_gate, int c_ratio, const void* c_norm_weight, float c_eps,
                           uint8_t* c_cache, int64_t c_cache_batch_entries, int64_t c_cache_cap, void* key_half,
                           void* stream);

/* ---------------------------------------------------------------------------------
 * Piece 2: KV compressor and RoPE
 * --------------------------------------------------------------------------------- */

/* DeepseekV41Compressor.forward after its two fp32 projections (owlet1/cache.py:157-172)
 * plus its RMSNorm (owlet1/norm_rope.py:25-30):
 *   out[b, g] = w * dtype( h * rsqrt(mean(h^2) + eps) ),
 *   h = dtype( sum_r kv[b, g*ratio + r] * softmax_r(gate[b, g*ratio + r]) )   (ratio > 1)
 *   h = dtype( kv[b, g] )                                                      (ratio == 1)
 * kv, gate: fp32 [B, tokens_per_batch, D] (gate unused at ratio 1); norm_weight [D] of
 * weight_dtype; out [B, n_groups, D] of out_dtype.  D <= 1024.  Evaluation order is fixed
 * (see compressor.hip), so results are reproducible bit for bit. */
int mzk_compress(const float* kv, const float* gate, int64_t B, int64_t n_groups, int ratio,
                 int D, int64_t tokens_per_batch, const void* norm_weight, int weight_dtype,
                 float eps, void* out, int out_dtype, void* stream);

/* apply_rotary_pos_emb (owlet1/norm_rope.py:126-145): x [rows, D] of `dtype`; the trailing
 * rope_dim channels are rotated as (even, odd) pairs with cos/sin [rows/heads, rope_dim/2]
 * fp32 (one table row per `heads` consecutive x rows); inverse != 0 conjugates. */
int mzk_rope(const void* x, int dtype, const float* cos_t, const float* sin_t, int64_t rows,
             int D, int rope_dim, int heads, int inverse, void* y, void* stream);

/* DeepseekV41RMSNorm.forward (owlet1/norm_rope.py:25-30) of any width:
 *   out[r] = out_dtype( weight * x_dtype( h * (1 / sqrt(sum(h^2) / D + eps)) ) ),  h = fp32(x[r])
 * the sum of squares in a fixed order (lane l of a wave sums channels l, l+64, ... from 0,
 * then an xor butterfly), so results are reproducible bit for bit.  x [rows, D] with row
 * stride x_row_stride elements; out [rows, D] contiguous.  out_dtype is the promotion of
 * weight_dtype and x_dtype (the reference's `self.weight * hidden_states`). */
int mzk_rms_norm(const void* x, int x_dtype, int64_t rows, int D, int64_t x_row_stride, const void* weight,
                 int weight_dtype, float eps, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------------
 * Piece 3: lightning-indexer scores (MFMA)
 *   score[row, g] = Di^-0.5 * sum_h w[row,h] * relu(q[row,h] . k[b,g])  for g < vis,
 *   -inf otherwise, vis = min(G, (positions[row] + 1) / ratio)
 * -- owlet1/indexer.py:124-143, layers/attn/golden_ref.py:213-227,
 *    layers/attn/indexer/fwd.py:112-132.  rows = B*S, row = b*S + s; `w` [rows, Hi] is
 * already multiplied by Hi^-0.5; positions [rows] int64 may be NULL (position = s).
 * Keys: batch b starts at key b*k_batch_stride.  scores: [rows, score_stride] fp32.
 * Hi <= 64. Di: multiple of 64 (fp8 / mxfp4), 32/64/96/128/256 (bf16).
 * --------------------------------------------------------------------------------- */

/* FP8 (SGLang/DeepSeek V3.2 indexer layout): q_codes [rows, Hi, Di] e4m3 + q_scales
 * [rows, Hi] fp32; k_codes [B, G, Di] e4m3 + k_scales [B, G] fp32 (one pow2 scale per row,
 * i.e. mzk_quant_fp8_block with block_size = Di). */
int mzk_indexer_scores_fp8(const uint8_t* q_codes, const float* q_scales, const float* w,
                           const uint8_t* k_codes, const float* k_scales, int64_t B, int64_t S,
                           int Hi, int Di, int64_t G, int64_t k_batch_stride,
                           const int64_t* positions, int ratio, float* scores,
                           int64_t score_stride, void* stream);

/* MXFP4 (the model's own indexer quantizer, owlet1/indexer.py:106,129): packed e2m1
 * [rows, Hi, Di/2] / [B, G, Di/2] + e8m0 [rows, Hi, Di/32] / [B, G, Di/32]
 * (mzk_quant_mxfp4 output). */
int mzk_indexer_scores_mxfp4(const uint8_t* q_packed, const uint8_t* q_e8m0, const float* w,
                             const uint8_t* k_packed, const uint8_t* k_e8m0, int64_t B, int64_t S,
                             int Hi, int Di, int64_t G, int64_t k_batch_stride,
                             const int64_t* positions, int ratio, float* scores,
                             int64_t score_stride, void* stream);

/* Decode form of the FP8 indexer with the step's prologue fused in, one new token per
 * batch row (S = 1): the bf16 indexer query q_idx [B, Hi, 128] is quantized in the kernel
 * (FP8 b128, identical to mzk_quant_fp8_block with block_size 128 -- owlet1/indexer.py:129
 * with owlet1/quant.py:72-86) and scored against k_codes / k_scales exactly as
 * mzk_indexer_scores_fp8 would score the quantized query.  Optional extras, each written
 * once per row:
 *   q_codes [B, Hi, 128] e4m3 + q_scales [B, Hi] fp32 -- the quantized query (both or
 *     neither);
 *   kv [B, nope + rope] bf16 -- the new token's latent, appended to the window ring as
 *     mzk_decode_prologue does (entry b*win_batch_entries + positions[b] % win_cap of
 *     win_cache; owlet1/cache.py:84-94); NULL skips the append.
 * Replaces mzk_decode_prologue + mzk_indexer_scores_fp8 in the decode step (one launch
 * instead of two).  Di must be 128; nope a multiple of 128 up to 1024, rope even up to
 * 256; positions required. */
int mzk_indexer_decode_fp8(const void* q_idx, const float* w, const uint8_t* k_codes,
                           const float* k_scales, int64_t B, int Hi, int Di, int64_t G,
                           int64_t k_batch_stride, const int64_t* positions, int ratio,
                           float* scores, int64_t score_stride, uint8_t* q_codes,
                           float* q_scales, const void* kv, int nope, int rope,
                           uint8_t* win_cache, int64_t win_batch_entries, int win_cap,
                           void* stream);

/* The same for the MXFP4 indexer: q_idx [B, Hi, 128] bf16 is quantized in the kernel to
 * MXFP4 (identical to mzk_quant_mxfp4: block 32, ue8m0 scales -- owlet1/indexer.py:129
 * with owlet1/quant.py:49-66) and scored against k_packed / k_e8m0 exactly as
 * mzk_indexer_scores_mxfp4 would score the quantized query.  Optional extras: q_packed
 * [B, Hi, 64] + q_e8m0 [B, Hi, 4] (both or neither), and the window append of kv as in
 * mzk_indexer_decode_fp8.  Replaces mzk_decode_prologue + mzk_indexer_scores_mxfp4 in the
 * decode step. */
int mzk_indexer_decode_mxfp4(const void* q_idx, const float* w, const uint8_t* k_packed, const uint8_t* k_e8m0,
                             int64_t B, int Hi, int Di, int64_t G, int64_t k_batch_stride, const int64_t* positions,
                             int ratio, float* scores, int64_t score_stride, uint8_t* q_packed, uint8_t* q_e8m0,
                             const void* kv, int nope, int rope, uint8_t* win_cache, int64_t win_batch_entries,
                             int win_cap, void* stream);

/* bf16 q [rows, Hi, Di] and k [B, G, Di] -- the contract of layers/attn/indexer/fwd.py:112. */
/* The decode step's whole per-token prologue and its indexer in one launch
 * (q_format 0: FP8 as mzk_indexer_decode_fp8, k_scales fp32 [B, kbs], q_scales fp32 [B, Hi];
 * 1: MXFP4 as mzk_indexer_decode_mxfp4, k_scales = e8m0 [B, kbs, 4], q_scales = e8m0
 * [B, Hi, 4]).  Replaces, for one new token per row (owlet1/attention.py:150-155 and
 * owlet1/indexer.py:126-133):
 *   q_idx bf16 [B, Hi, 128] unrotated -> apply_rotary_pos_emb on its trailing q_rope_dim
 *     channels (32, 64, 96 or 128) with q_cos / q_sin bf16 [B, q_rope_dim/2] (the compress
 *     RoPE) -> quantized and scored as the two entries above;
 *   kv bf16 [B, 576] (the wkv projection) -> DeepseekV41RMSNorm (kv_weight bf16 [576],
 *     kv_eps; sum of squares in 64 lane partials combined by an xor butterfly) -> RoPE of
 *     channels 512..575 with kv_cos / kv_sin bf16 [B, 32] -> FP8-b128 entry (as
 *     mzk_pack_latent_fp8_b128) at ring slot b*win_batch_entries + positions[b] % win_cap.
 * nope / rope must be 512 / 64.  q_idx, k_codes, q_codes, q_cos, q_sin 16-byte aligned. */
int mzk_indexer_decode_fused(int q_format, const void* q_idx, const float* w, const uint8_t* k_codes,
                             const void* k_scales, int64_t B, int Hi, int Di, int64_t G,
                             int64_t k_batch_stride, const int64_t* positions, int ratio,
                             float* scores, int64_t score_stride, uint8_t* q_codes, void* q_scales,
                             const void* q_cos, const void* q_sin, int q_rope_dim, const void* kv,
                             const void* kv_weight, float kv_eps, const void* kv_cos,
                             const void* kv_sin, int nope, int rope, uint8_t* win_cache,
                             int64_t win_batch_entries, int win_cap, void* stream);

int mzk_indexer_scores_bf16(const void* q, const float* w, const void* k, int64_t B, int64_t S,
                            int Hi, int Di, int64_t G, int64_t k_batch_stride,
                            const int64_t* positions, int ratio, float* scores,
                            int64_t score_stride, void* stream);

/* ---------------------------------------------------------------------------------
 * Piece 4: top-k selection
 * --------------------------------------------------------------------------------- */

/* Per-row top-k of fp32 scores -- replaces `index_scores.topk(min(k, G), sorted=False)`
 * and the -inf -> dummy-slot mapping of owlet1/indexer.py:158-165,
 * layers/attn/golden_ref.py:230-243 and layers/attn/indexer/attn.py:67-81.
 * scores [rows, cols] (row stride `row_stride` floats) -> out [rows, topk] int32
 * (row stride `out_stride`): the selected column indices in ascending order, then -1.
 * -inf entries are never selected; among equal scores the lower index wins. */
int mzk_topk_rows(const float* scores, int64_t rows, int64_t cols, int64_t row_stride, int topk,
                  int32_t* out, int64_t out_stride, void* stream);

/* mzk_topk_rows with a caller-owned workspace, for long rows: rows of 32769 .. 524288
 * columns are split over 8192-column chunk workgroups (histogram -> per-row selection ->
 * index-ordered write, three launches), so a few long rows still fill the GPU; other sizes
 * run mzk_topk_rows.  Same contract and results.  `workspace` (16-byte aligned) holds
 * *bytes from mzk_topk_workspace_bytes(rows, cols, &bytes) (0: none needed). */
int mzk_topk_workspace_bytes(int64_t rows, int64_t cols, int64_t* bytes);
int mzk_topk_rows_ws(const float* scores, int64_t rows, int64_t cols, int64_t row_stride, int topk,
                     int32_t* out, int64_t out_stride, void* workspace, int64_t workspace_bytes, void* stream);

/* The indexer's published block bias from a top-k index list -- owlet1/indexer.py:158-165
 * (`block_bias.scatter_(-1, safe, 0.0)` over a -inf row, the -inf picks and -1 slots
 * dropped): bias [rows, G] fp32 (row stride bias_row_stride) is 0 at the columns
 * idx[r, :topk] names (entries outside [0, G) are empty) and -inf elsewhere. */
int mzk_topk_bias(const int32_t* idx, int64_t rows, int topk, int64_t idx_row_stride, int64_t G, float* bias,
                  int64_t bias_row_stride, void* stream);

/* The inverse: the visible columns of an additive attention mask as index lists, for the
 * attention interface that receives the reference's dense mask (eager_attention_forward,
 * owlet1/attention.py:42-71, with the mask of :202-214).  mask [rows, cols] of mask_dtype
 * (row stride row_stride); a column is visible where the mask is 0 and masked where it is
 * -inf or the dtype's lowest finite value (transformers' eager fill).  idx [rows, cap] int32:
 * the visible columns ascending, then -1; counts [rows].  flags (one int, zeroed by the
 * caller) gets bit 0 if any other value occurs (not representable as a selection) and bit 1
 * if a row has more than cap visible columns (its list is then truncated). */
int mzk_mask_to_indices(const void* mask, int mask_dtype, int64_t rows, int64_t cols, int64_t row_stride, int cap,
                        int32_t* idx, int32_t* counts, int* flags, void* stream);

/* Level one of the two-level candidate selection -- replaces select_candidate_blocks
 * (owlet1/indexer.py:14-40; tickets/0009-indexer-hierarchical.md).  logits [rows, width]
 * fp32 (row stride row_stride; unreachable positions already -inf), compress_lens [rows]
 * int64 (the query's visible group count): block maxima over blocks of block_size
 * positions (the tail block padded with -inf), the block holding position
 * compress_lens-1 pinned to +inf, the top topk_blocks blocks whose score is above -inf
 * (lowest block index first among equal scores; the reference leaves ties unspecified).
 * Outputs (either may be NULL, not both): mask [rows, width] uint8 0/1 (row stride
 * mask_stride) -- the reference's bool mask -- and block_idx_out [rows, topk_blocks] int32,
 * the selected blocks ascending then -1 (the compact candidate list).  workspace:
 * mzk_candidate_blocks_workspace_bytes, 16-byte aligned. */
int mzk_candidate_blocks_workspace_bytes(int64_t rows, int64_t width, int block_size, int topk_blocks, int64_t* bytes);
int mzk_candidate_blocks(const float* logits, int64_t rows, int64_t width, int64_t row_stride,
                         const int64_t* compress_lens, int topk_blocks, int block_size, uint8_t* mask,
                         int64_t mask_stride, int32_t* block_idx_out, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* Level two: score only the candidates -- replaces a candidate-using layer's dense scoring
 * plus `index_scores.masked_fill(~shared["candidates"], -inf)` (owlet1/indexer.py:150-151;
 * the gather form of tickets/0009-indexer-hierarchical.md:29-32; the score itself as
 * mzk_indexer_scores_fp8 / _mxfp4, owlet1/indexer.py:129-143).  cand_blocks [B*S, cand_stride]
 * int32 is the compact list of mzk_candidate_blocks (blocks ascending, then -1; n_blocks
 * entries used).  scores [B*S, n_blocks*block_size] fp32 (row stride score_stride) on the
 * candidate axis: slot j holds key cand_blocks[row][j / block_size] * block_size +
 * j % block_size, with the same bits as the dense kernel's score of that key, or -inf if the
 * block entry is -1, the key is >= G or not visible at the row's position.  Di = 128,
 * B*S <= 65535. */
int mzk_indexer_candidate_scores_fp8(const uint8_t* q_codes, const float* q_scales, const float* w,
                                     const uint8_t* k_codes, const float* k_scales, int64_t B, int64_t S, int Hi,
                                     int Di, int64_t G, int64_t k_batch_stride, const int64_t* positions, int ratio,
                                     const int32_t* cand_blocks, int64_t cand_stride, int n_blocks, int block_size,
                                     float* scores, int64_t score_stride, void* stream);
int mzk_indexer_candidate_scores_mxfp4(const uint8_t* q_packed, const uint8_t* q_e8m0, const float* w,
                                       const uint8_t* k_packed, const uint8_t* k_e8m0, int64_t B, int64_t S, int Hi,
                                       int Di, int64_t G, int64_t k_batch_stride, const int64_t* positions, int ratio,
                                       const int32_t* cand_blocks, int64_t cand_stride, int n_blocks, int block_size,
                                       float* scores, int64_t score_stride, void* stream);
/* The top-k over the candidate axis back to key positions, i.e. the top-k of the masked
 * dense row (owlet1/indexer.py:158-161): slot_idx [rows, k] (row stride idx_stride, -1 =
 * empty) -> pos_out [rows, k] (out_stride; may be slot_idx itself with equal strides).
 * Ascending slots map to ascending positions; -1 and empty slots stay -1. */
int mzk_candidate_positions(const int32_t* slot_idx, int64_t rows, int k, int64_t idx_stride,
                            const int32_t* cand_blocks, int64_t cand_stride, int n_blocks, int block_size,
                            int32_t* pos_out, int64_t out_stride, void* stream);
/* The two in one launch (block_size 8, the model's candidate_block_size; other sizes run
 * the two): the top-k of candidate-axis scores [rows, slots] (row stride row_stride; slots =
 * n_blocks * block_size <= 32768) written as key positions into out [rows, topk] --
 * ascending, lowest position first among equal scores, then -1; the list mzk_topk_rows +
 * mzk_candidate_positions give. */
int mzk_candidate_topk(const float* scores, int64_t rows, int64_t slots, int64_t row_stride, int topk,
                       const int32_t* cand_blocks, int64_t cand_stride, int n_blocks, int block_size, int32_t* out,
                       int64_t out_stride, void* stream);

/* ---------------------------------------------------------------------------------
 * Piece 5: sparse shared-latent MQA attention
 * --------------------------------------------------------------------------------- */

/* One softmax per (row, head) over [window ; dense ; gathered top-k] entries + sink,
 * K == V, scale D^-0.5 -- replaces eager_attention_forward over the concatenated KV
 * (owlet1/attention.py:42-71, :199-229), golden(level="sparse"/"compressed")
 * (layers/attn/golden_ref.py:103-168) and csa2_attn.fwd (layers/attn/csa2_attn/fwd.py:238-286).
 *   q          [B*S rows, H, D] bf16; row = b*S + s; positions [rows] int64 (absolute)
 *   fmt        0: entries are bf16 [D]; 1: FP8-b128 latent entries (nope = 512 or 128)
 *   window src win: row sees tokens max(0, pos-window+1)..pos of batch b at entry
 *              b*win_batch_entries + (win_cap ? tok % win_cap : tok)  (window 0 and
 *              win NULL: no window source; at least one source must be given)
 *   dense src  entries 0..min(dense_cap, (pos+1)/dense_ratio)-1 at b*dense_batch_entries
 *              (dense may be NULL)
 *   sparse src main_kv entries idx[row*idx_row_stride + j], j < topk; idx < 0 or >= G is
 *              empty (main_kv may be NULL)
 *   sinks      [H] fp32 natural-log logit or NULL
 *   nsplit     splits of the entry axis per row; > 1 needs a workspace of
 *              rows*nsplit*H*(2*D+8) bytes: each split's output O/l in bf16 by
 *              16-channel group, [rows, nsplit, D/16, H, 16] (a workgroup's stores are then
 *              contiguous), then its (m, l) in fp32 [rows, nsplit, H, 2] (m in log2 units);
 *              merged by a second kernel -- or, with mzk_sparse_mqa_set_merge(1), inside
 *              the attention launch when the workspace has mzk_sparse_mqa_workspace_bytes bytes (zero-filled before its
 *              first use; every complete call leaves its merge records zero again), D > 256,
 *              nsplit divides 64, rows or rows * ceil(H/64) is a multiple of 8, and
 *              rows * nsplit * ceil(H/64)
 *              workgroups fit the device's CUs (each split then waits for its siblings on
 *              the XCD that ran them and merges 64/nsplit of their heads; the result is
 *              bit-identical to the merge kernel's)
 *   out        [rows, H, D] bf16;  lse [B, H, S] fp32 (natural log, sink included).
 *              With nsplit > 1, out == lse == NULL writes only the partials (the merge is
 *              then mzk_sparse_mqa_combine). */
int mzk_sparse_mqa(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                   const int64_t* positions, const void* win, int64_t win_batch_entries,
                   int win_cap, int window, const void* dense, int64_t dense_batch_entries,
                   int dense_cap, int dense_ratio, const void* main_kv,
                   int64_t main_batch_entries, int64_t G, const int32_t* idx,
                   int64_t idx_row_stride, int topk, const float* sinks, int nsplit,
                   float* workspace, int64_t workspace_bytes, void* out, float* lse,
                   void* stream);

/* The workspace mzk_sparse_mqa / _rope take for nsplit splits of `rows` rows: the split
 * partials (rows*nsplit*H*(2*D+8) bytes, 16-byte aligned) then the in-launch merge's records
 * (16 bytes per row and 64-head group, then 16 bytes of status: word 0 is set to 1 by a split
 * that gave up waiting for its siblings, word 1 counts the groups merged inside attention
 * launches, word 2 the workgroups that took the cross-XCD cache path); 0 when nsplit is 1.  No counterpart in the
 * reference (its split-free kernel needs no workspace). */
int mzk_sparse_mqa_workspace_bytes(int64_t rows, int H, int D, int nsplit, int64_t* bytes);

/* Where the split merge runs: 0: the merge kernel after the attention launch (the
 * default); 1: inside the attention launch where it applies; 2: inside, with every workgroup
 * taking the cache write-back / invalidate path of a group spread over several XCDs (a test
 * mode).  Process-wide.  The in-launch merge is bit-identical to the merge kernel and, on
 * MI355X, not faster (config 2 equal within noise, configs 4 and 5 slower).  No
 * counterpart in the reference: a switch of this build's own launch structure, for tests
 * and A/B timing. */
int mzk_sparse_mqa_set_merge(int mode);

/* Merge the nsplit partials a previous mzk_sparse_mqa call left in `workspace` with the
 * sink: the log-sum-exp combination of the split softmaxes (equal to the one softmax of
 * owlet1/attention.py:64-70 over all entries). */
int mzk_sparse_mqa_combine(const float* workspace, int64_t B, int64_t S, int H, int D,
                           int nsplit, const float* sinks, void* out, float* lse, void* stream);

/* mzk_sparse_mqa with the query's RoPE and the output's inverse RoPE fused in
 * (owlet1/attention.py:147 and :226 around the attention of :217-229): q arrives unrotated
 * and its channels nope..D-1 are rotated with rope_cos / rope_sin bf16 [rows, rope_dim/2]
 * (the row's position_embeddings, apply_rotary_pos_emb) as the kernel loads it; the bf16
 * output gets the inverse rotation (sin negated) -- in the split merge when nsplit > 1.
 * FP8 latent rows only (fmt 1, D 576, nope 512, rope_dim 64); cos / sin 16-byte aligned. */
int mzk_sparse_mqa_rope(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                        const int64_t* positions, const void* win, int64_t win_batch_entries,
                        int win_cap, int window, const void* dense, int64_t dense_batch_entries,
                        int dense_cap, int dense_ratio, const void* main_kv,
                        int64_t main_batch_entries, int64_t G, const int32_t* idx,
                        int64_t idx_row_stride, int topk, const float* sinks, int nsplit,
                        float* workspace, int64_t workspace_bytes, void* out, float* lse,
                        const void* rope_cos, const void* rope_sin, int rope_dim, void* stream);

/* mzk_sparse_mqa_rope (rope_cos / rope_sin may be NULL: then mzk_sparse_mqa) for one decode
 * step (S = 1, out and lse given) that also advances the positions it reads: positions[b] +=
 * 1 for every row once the call's launches have read them -- in the split merge's launch,
 * which reads no position (nsplit > 1 with the merge kernel), else in a launch of its own
 * after the attention.  Saves a decode step its separate `positions += 1` launch (1.5-2.5 us
 * inside a HIP graph on MI355X).  A caller whose later launches of the same step read the
 * same positions advances them once, on the last call.  No counterpart in the reference:
 * its decoder derives each step's position_ids on the host from the tokens the cache has
 * seen (owlet1/decoder.py:285-288); this build keeps positions on the device so that graph
 * replays decode consecutive tokens. */
int mzk_sparse_mqa_advance(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                           int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                           int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                           int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                           const int32_t* idx, int64_t idx_row_stride, int topk, const float* sinks, int nsplit,
                           float* workspace, int64_t workspace_bytes, void* out, float* lse, const void* rope_cos,
                           const void* rope_sin, int rope_dim, void* stream);

/* One decode step's selection and attention in one launch (S = 1): the top-topk of the
 * indexer scores [B, score_stride] fp32 over G keys (owlet1/indexer.py:158-165 as
 * mzk_topk_rows: -inf never taken, lower index first among equal scores, ascending, then
 * -1) becomes the sparse list of mzk_sparse_mqa_rope over main_kv -- every attention
 * workgroup of a row selects the row's list itself, so the step has no top-k launch -- and
 * the list is also written to idx_out [B, idx_out_stride] int32.  With advance != 0 the
 * positions then advance as in mzk_sparse_mqa_advance.  In one launch for the FP8 latent
 * rows (fmt 1, D 576, nope 512) with G <= 8192 and topk <= 2048, both multiples of 4,
 * score_stride and idx_out_stride multiples of 4, scores / idx_out 16-byte aligned, and
 * splits of at most 1024 - 96 entries ((window + dense_cap + topk) / nsplit, the decode
 * kernel's entry tables); otherwise mzk_topk_rows and then the attention, same results.
 * out and lse NULL (nsplit > 1, advance 0): the split partials only, as mzk_sparse_mqa.  Other arguments
 * as mzk_sparse_mqa_rope (rope_cos / rope_sin may be NULL).  No counterpart in the
 * reference as one call: it is the reference's index_scores.topk followed by its sparse
 * attention (owlet1/attention.py:217-229). */
int mzk_sparse_mqa_select(const void* q, int64_t B, int H, int D, int fmt, int nope, int64_t* positions,
                          int advance, const void* win, int64_t win_batch_entries, int win_cap, int window,
                          const void* dense, int64_t dense_batch_entries, int dense_cap, int dense_ratio,
                          const void* main_kv, int64_t main_batch_entries, int64_t G, const float* scores,
                          int64_t score_stride, int topk, int32_t* idx_out, int64_t idx_out_stride,
                          const float* sinks, int nsplit, float* workspace, int64_t workspace_bytes, void* out,
                          float* lse, const void* rope_cos, const void* rope_sin, int rope_dim, void* stream);

/* The split partials of part of a row's entry list, for launches that share one workspace:
 * splits split_base .. split_base + nsplit - 1 of a workspace holding split_total splits
 * per row (rows*split_total*H*(2*D+8) bytes, laid out as for mzk_sparse_mqa), over the
 * sources this call is given -- e.g. the window and dense branches in one launch and the
 * top-k entries in another, which a caller can run concurrently when the top-k is not yet
 * known; mzk_sparse_mqa_combine(_rope) with nsplit = split_total then merges them as one
 * softmax (owlet1/attention.py:64-70 over the concatenated entries).  window may be 0 (no
 * window source); rope_cos / rope_sin (or NULL) as mzk_sparse_mqa_rope. */
int mzk_sparse_mqa_part(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                        const int64_t* positions, const void* win, int64_t win_batch_entries,
                        int win_cap, int window, const void* dense, int64_t dense_batch_entries,
                        int dense_cap, int dense_ratio, const void* main_kv,
                        int64_t main_batch_entries, int64_t G, const int32_t* idx,
                        int64_t idx_row_stride, int topk, int nsplit, int split_base,
                        int split_total, float* workspace, int64_t workspace_bytes,
                        const void* rope_cos, const void* rope_sin, int rope_dim, void* stream);

/* mzk_sparse_mqa_combine followed by the inverse RoPE of the merged bf16 output's trailing
 * rope_dim channels (owlet1/attention.py:226), cos / sin bf16 [rows, rope_dim/2]. */
int mzk_sparse_mqa_combine_rope(const float* workspace, int64_t B, int64_t S, int H, int D,
                                int nsplit, const float* sinks, const void* rope_cos,
                                const void* rope_sin, int rope_dim, void* out, float* lse,
                                void* stream);

/* mzk_sparse_mqa_rope without a workspace, for callers that cannot allocate (code under
 * HIP-graph capture that must not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference: it is mzk_sparse_mqa_rope with the split
 * partials kept in a file-scope device array of MZK_NOALLOC_SCRATCH_BYTES bytes (one copy
 * per GPU the library runs on, held until the process ends) instead of `workspace`; it
 * never allocates.  rope_cos / rope_sin may be NULL (then it is mzk_sparse_mqa); out and lse
 * are required (the partials stay in the private array).  Limit:
 * rows * nsplit * H * (2*D + 8) <= MZK_NOALLOC_SCRATCH_BYTES when nsplit > 1 (config 2:
 * 32 x 4 x 128 x 1160 = 19 MB), else MZK_EINVAL.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (concurrent streams, or host threads) race: the
 * caller must order them, e.g. on one stream.  The device address is looked up
 * (hipGetSymbolAddress) on the first call on each device: make that first call outside
 * graph capture. */
#define MZK_NOALLOC_SCRATCH_BYTES (32ll << 20)
int mzk_sparse_mqa_noalloc(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                           const int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                           int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                           int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                           const int32_t* idx, int64_t idx_row_stride, int topk, const float* sinks, int nsplit,
                           void* out, float* lse, const void* rope_cos, const void* rope_sin, int rope_dim,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MZK_H */

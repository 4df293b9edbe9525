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

#ifdef __cplusplus
}
#endif

#endif /* MZK_H */

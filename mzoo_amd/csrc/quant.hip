// Piece 1: block FP8-e4m3 / FP4-e2m1 quantizers and the packed cache formats.
//
// Semantics follow src/mzoo/archs/owlet1/quant.py (the reference's fake quantizers):
//   fp8:  amax = max(max|x|, 1e-4);  s = pow2ceil(amax * fp32(1/448));
//         y = e4m3(clamp(x / s, +-448)) * s                                   (:72-86)
//   fp4:  ue8m0: s = pow2ceil(max(amax, 6*2^-126) * fp32(1/6))
//         e4m3 : s = e4m3(max(amax, 6*2^-9) / 6)
//         y = e2m1(clamp(x / s, +-6)) * s                                     (:49-66)
// Layout: every kernel maps `G = block_size / 4` consecutive lanes to one block of
// `block_size` contiguous elements (4 per lane); the block amax is a xor-shuffle
// reduction inside that lane group.  One HBM read and one write per element.
#include "common.h"

namespace mzk {
namespace {

// ---- fake quant (value round trips) ------------------------------------------------

template <int DT, bool FP4>
__global__ void fake_quant_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t nthreads,
                                  int group, bool e4m3_scales) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= nthreads) return;  // whole lane groups are in or out (nthreads % group == 0)
  const int64_t base = t * 4;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = load_as_f32<DT>(x, base + i);
  float amax = abs_max4(v);
  amax = wave_max_group(amax, group);
  if constexpr (FP4) {
    const float s = fp4_scale_from_amax(amax, e4m3_scales);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = e2m1_code(clampf(div_rn(v[i], s), 6.0f));
      store_from_f32<DT>(y, base + i, e2m1_value(c) * s);
    }
  } else {
    const float s = fp8_scale_from_amax(amax);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = e4m3_encode(clampf(div_rn(v[i], s), 448.0f));
      store_from_f32<DT>(y, base + i, e4m3_decode(c) * s);
    }
  }
}

// Fallback for block sizes that are not a power of two in [4, 256]: one thread per block.
template <int DT, bool FP4>
__global__ void fake_quant_serial_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t nblocks,
                                         int bs, bool e4m3_scales) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= nblocks) return;
  const int64_t base = j * bs;
  float amax = 0.0f;
  for (int i = 0; i < bs; ++i) amax = nn_max(amax, fabsf(load_as_f32<DT>(x, base + i)));
  const float s = FP4 ? fp4_scale_from_amax(amax, e4m3_scales) : fp8_scale_from_amax(amax);
  for (int i = 0; i < bs; ++i) {
    const float v = load_as_f32<DT>(x, base + i);
    float r;
    if constexpr (FP4) r = e2m1_value(e2m1_code(clampf(div_rn(v, s), 6.0f))) * s;
    else r = e4m3_decode(e4m3_encode(clampf(div_rn(v, s), 448.0f))) * s;
    store_from_f32<DT>(y, base + i, r);
  }
}

// ---- packed encoders ---------------------------------------------------------------

// Thread t encodes elements 4t..4t+3; the `group` consecutive threads of a block share
// one amax (lane shuffles), so groups must not straddle a wave.
template <int DT>
__device__ __forceinline__ void quant_fp8_4(const void* __restrict__ x, uint8_t* __restrict__ codes,
                                            float* __restrict__ scales, int64_t t, int group, bool vec) {
  const int64_t base = t * 4;
  float v[4];
  load4_as_f32<DT>(x, base, vec, v);
  float amax = abs_max4(v);
  amax = group_max(amax, group);
  const float s = fp8_scale_from_amax(amax);
  // x / s == x * (1 / s) exactly (s is a power of two in [2^-22, 2^120] for finite input,
  // 1 / s a normal float), and v_cvt_pk_fp8_f32 is the e4m3 encoder (round to nearest even)
  // for |x| <= 448; an infinite amax keeps the division's behaviour through 1 / s
  const float inv = s <= 0x1p120f ? pow2_reciprocal(s) : 1.0f / s;
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(clampf(v[0] * inv, 448.0f), clampf(v[1] * inv, 448.0f), 0, false);
  const uint32_t word = static_cast<uint32_t>(
      __builtin_amdgcn_cvt_pk_fp8_f32(clampf(v[2] * inv, 448.0f), clampf(v[3] * inv, 448.0f), lo, true));
  reinterpret_cast<uint32_t*>(codes)[t] = word;
  if ((t % group) == 0) scales[t / group] = s;
}

template <int DT>
__device__ __forceinline__ void quant_mxfp4_4(const void* __restrict__ x, uint8_t* __restrict__ packed,
                                              uint8_t* __restrict__ e8m0, int64_t t, bool vec) {
  const int64_t base = t * 4;
  float v[4];
  load4_as_f32<DT>(x, base, vec, v);
  float amax = abs_max4(v);
  amax = wave_max_group(amax, 8);
  const float s = fp4_scale_from_amax(amax, false);
  const float inv = 1.0f / s;  // a power of two: x * inv == x / s exactly
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = e2m1_code(clampf(v[i] * inv, 6.0f));
  const uint16_t two = static_cast<uint16_t>(c[0] | (c[1] << 4) | (c[2] << 8) | (c[3] << 12));
  reinterpret_cast<uint16_t*>(packed)[t] = two;
  if ((t & 7) == 0) e8m0[t >> 3] = static_cast<uint8_t>(__float_as_uint(s) >> 23);
}

template <int DT>
__global__ void quant_fp8_block_kernel(const void* __restrict__ x, uint8_t* __restrict__ codes,
                                       float* __restrict__ scales, int64_t nthreads, int group, bool vec) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < nthreads) quant_fp8_4<DT>(x, codes, scales, t, group, vec);
}

template <int DT>
__global__ void quant_mxfp4_kernel(const void* __restrict__ x, uint8_t* __restrict__ packed,
                                   uint8_t* __restrict__ e8m0, int64_t nthreads, bool vec) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < nthreads) quant_mxfp4_4<DT>(x, packed, e8m0, t, vec);
}

template <int DT>
__global__ void dequant_fp8_block_kernel(const uint8_t* __restrict__ codes, const float* __restrict__ scales,
                                         int64_t nthreads, int bs, void* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= nthreads) return;
  const uint32_t word = reinterpret_cast<const uint32_t*>(codes)[t];
  const float s = scales[(t * 4) / bs];
#pragma unroll
  for (int i = 0; i < 4; ++i) store_from_f32<DT>(y, t * 4 + i, e4m3_decode((word >> (8 * i)) & 0xffu) * s);
}

template <int DT>
__global__ void dequant_mxfp4_kernel(const uint8_t* __restrict__ packed, const uint8_t* __restrict__ e8m0,
                                     int64_t nthreads, void* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= nthreads) return;
  const uint32_t two = reinterpret_cast<const uint16_t*>(packed)[t];
  const float s = __uint_as_float(static_cast<uint32_t>(e8m0[t >> 3]) << 23);
#pragma unroll
  for (int i = 0; i < 4; ++i) store_from_f32<DT>(y, t * 4 + i, e2m1_value((two >> (4 * i)) & 0xfu) * s);
}

// ---- DeepSeek-V4.1 cache entries (FlashMLA kv_cache_format) ---------------------------
// fp8: [D e4m3 codes][D/32 e8m0 scale bytes]    -- _fake_quant_fp8_block(x, 32), owlet1/quant.py:72-86
//      (the window cache's quantizer, owlet1/attention.py:154); D = 512 gives 528 bytes
// fp4: [D/2 e2m1 bytes, element 2i in the low nibble][D/16 e4m3 scale bytes]
//      -- _fake_quant_fp4_block(x, 16, e4m3_scales=True), quant.py:49-66 (the compressed
//      cache's quantizer, attention.py:183); D = 512 gives 288 bytes
// Thread t encodes elements 4t..4t+3 of the flattened [rows, D]; the 8 (fp8) or 4 (fp4)
// threads of a scale block are consecutive lanes of one wave.
__host__ __device__ constexpr int64_t v41_entry_bytes(int d, int fmt) { return fmt == 0 ? d + d / 32 : d / 2 + d / 16; }

template <int DT, int FMT>
__global__ void pack_v41_kernel(const void* __restrict__ x, int d, int64_t nthreads, const int64_t* __restrict__ dst,
                                uint8_t* __restrict__ out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= nthreads) return;
  const int64_t row = (t * 4) / d;
  const int c = static_cast<int>(t * 4 - row * d);
  uint8_t* e = out + (dst ? dst[row] : row) * v41_entry_bytes(d, FMT);
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = load_as_f32<DT>(x, t * 4 + i);
  float amax = abs_max4(v);
  if constexpr (FMT == 0) {
    amax = wave_max_group(amax, 8);
    const float sc = fp8_scale_from_amax(amax);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) word |= static_cast<uint32_t>(e4m3_encode(clampf(div_rn(v[i], sc), 448.0f))) << (8 * i);
    *reinterpret_cast<uint32_t*>(e + c) = word;
    if ((c & 31) == 0) e[d + c / 32] = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
  } else {
    amax = wave_max_group(amax, 4);
    const float sc = fp4_scale_from_amax(amax, true);
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = e2m1_code(clampf(div_rn(v[i], sc), 6.0f));
    *reinterpret_cast<uint16_t*>(e + c / 2) = static_cast<uint16_t>(q[0] | (q[1] << 4) | (q[2] << 8) | (q[3] << 12));
    if ((c & 15) == 0) e[d / 2 + c / 16] = e4m3_encode(sc);
  }
}

template <int DT, int FMT>
__global__ void unpack_v41_kernel(const uint8_t* __restrict__ cache, int d, int64_t nthreads, void* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= nthreads) return;
  const int64_t row = (t * 4) / d;
  const int c = static_cast<int>(t * 4 - row * d);
  const uint8_t* e = cache + row * v41_entry_bytes(d, FMT);
  if constexpr (FMT == 0) {
    const uint32_t word = *reinterpret_cast<const uint32_t*>(e + c);
    const float sc = __uint_as_float(static_cast<uint32_t>(e[d + c / 32]) << 23);
#pragma unroll
    for (int i = 0; i < 4; ++i) store_from_f32<DT>(y, t * 4 + i, e4m3_decode((word >> (8 * i)) & 0xffu) * sc);
  } else {
    const uint32_t two = *reinterpret_cast<const uint16_t*>(e + c / 2);
    const float sc = e4m3_decode(e[d / 2 + c / 16]);
#pragma unroll
    for (int i = 0; i < 4; ++i) store_from_f32<DT>(y, t * 4 + i, e2m1_value((two >> (4 * i)) & 0xfu) * sc);
  }
}

// ---- FP8-b128 latent entries ---------------------------------------------------------
// One workgroup per row; thread t < nope/4 quantizes nope channels 4t..4t+3 (32 lanes per
// 128-channel block), then the rope channels are rounded to bf16.

template <int DT>
__device__ __forceinline__ void pack_latent_row(const void* __restrict__ x, int nope, int rope, int64_t row,
                                                uint8_t* __restrict__ e, int t) {
  const int d = nope + rope;
  const int nb = nope / 128;
  const int64_t xrow = row * d;
  if (t < nope / 4) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = load_as_f32<DT>(x, xrow + 4 * t + i);
    float amax = abs_max4(v);
    amax = wave_max_group(amax, 32);
    const float s = fp8_scale_from_amax(amax);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) word |= static_cast<uint32_t>(e4m3_encode(clampf(div_rn(v[i], s), 448.0f))) << (8 * i);
    reinterpret_cast<uint32_t*>(e)[t] = word;
    if ((t & 31) == 0) reinterpret_cast<float*>(e + nope)[t >> 5] = s;
  }
  uint16_t* r = reinterpret_cast<uint16_t*>(e + nope + 4 * nb);
  for (int i = t; i < rope; i += blockDim.x) r[i] = f32_to_bf16(load_as_f32<DT>(x, xrow + nope + i));
}

template <int DT>
__global__ void pack_latent_kernel(const void* __restrict__ x, int nope, int rope, const int64_t* __restrict__ dst,
                                   uint8_t* __restrict__ cache) {
  const int64_t row = blockIdx.x;
  const int64_t entry_bytes = nope + 4 * (nope / 128) + 2 * rope;
  pack_latent_row<DT>(x, nope, rope, row, cache + (dst ? dst[row] : row) * entry_bytes, threadIdx.x);
}

// Decode-step prologue: blocks 0..B-1 write the new token of row b into its window-ring
// slot (b * win_batch_entries + positions[b] % win_cap); the remaining blocks quantize the
// indexer queries (FP8 b128 or MXFP4), 256 threads x 4 elements each.
template <int DT, int QDT, bool MX>
__global__ void __launch_bounds__(256) decode_prologue_kernel(
    const void* __restrict__ kv, int64_t B, int nope, int rope, const int64_t* __restrict__ positions,
    uint8_t* __restrict__ win, int64_t win_batch_entries, int win_cap, const void* __restrict__ q, int64_t qthreads,
    int qgroup, uint8_t* __restrict__ qcodes, float* __restrict__ qscales, uint8_t* __restrict__ qe8m0, bool qvec) {
  const int64_t blk = blockIdx.x;
  if (blk < B) {
    const int64_t entry_bytes = nope + 4 * (nope / 128) + 2 * rope;
    const int64_t pos = positions[blk];
    if (pos < 0) return;  // no ring slot for a negative position
    const int64_t slot = blk * win_batch_entries + pos % win_cap;
    pack_latent_row<DT>(kv, nope, rope, blk, win + slot * entry_bytes, threadIdx.x);
  } else {
    const int64_t t = (blk - B) * 256 + threadIdx.x;
    if (t < qthreads) {
      if constexpr (MX) quant_mxfp4_4<QDT>(q, qcodes, qe8m0, t, qvec);
      else quant_fp8_4<QDT>(q, qcodes, qscales, t, qgroup, qvec);
    }
  }
}

template <int DT>
__global__ void unpack_latent_kernel(const uint8_t* __restrict__ cache, int nope, int rope, void* __restrict__ y) {
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int d = nope + rope;
  const int nb = nope / 128;
  const uint8_t* e = cache + row * static_cast<int64_t>(nope + 4 * nb + 2 * rope);
  const int64_t yrow = row * d;
  if constexpr (DT == MZK_BF16) {
    // 8 channels per thread through the hardware e4m3 -> bf16 conversion (the same
    // routine the attention kernel dequantizes its tiles with)
    if (t < nope / 8) {
      const uint2 raw = reinterpret_cast<const uint2*>(e)[t];
      const float s = reinterpret_cast<const float*>(e + nope)[t >> 4];
      const uint4 v = dequant_fp8x8_bf16(raw, s);
      uint16_t* yy = static_cast<uint16_t*>(y) + yrow + 8 * t;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        yy[2 * i] = static_cast<uint16_t>(w[i] & 0xffffu);
        yy[2 * i + 1] = static_cast<uint16_t>(w[i] >> 16);
      }
    }
  } else {
    if (t < nope / 4) {
      const uint32_t word = reinterpret_cast<const uint32_t*>(e)[t];
      const float s = reinterpret_cast<const float*>(e + nope)[t >> 5];
#pragma unroll
      for (int i = 0; i < 4; ++i) store_from_f32<DT>(y, yrow + 4 * t + i, e4m3_decode((word >> (8 * i)) & 0xffu) * s);
    }
  }
  const uint16_t* r = reinterpret_cast<const uint16_t*>(e + nope + 4 * nb);
  for (int i = t; i < rope; i += blockDim.x) store_from_f32<DT>(y, yrow + nope + i, bf16_to_f32(r[i]));
}

bool pow2_in(int v, int lo, int hi) { return v >= lo && v <= hi && (v & (v - 1)) == 0; }

inline unsigned grid_for(int64_t n, int threads) { return static_cast<unsigned>((n + threads - 1) / threads); }

template <int DT>
void launch_fake(const void* x, void* y, int64_t rows, int64_t n, int bs, bool fp4, bool e4m3, hipStream_t s) {
  const int64_t total = rows * n;
  if (pow2_in(bs, 4, 256)) {
    const int64_t nthreads = total / 4;
    if (fp4)
      fake_quant_kernel<DT, true><<<grid_for(nthreads, 256), 256, 0, s>>>(x, y, nthreads, bs / 4, e4m3);
    else
      fake_quant_kernel<DT, false><<<grid_for(nthreads, 256), 256, 0, s>>>(x, y, nthreads, bs / 4, e4m3);
  } else {
    const int64_t nblocks = total / bs;
    if (fp4)
      fake_quant_serial_kernel<DT, true><<<grid_for(nblocks, 256), 256, 0, s>>>(x, y, nblocks, bs, e4m3);
    else
      fake_quant_serial_kernel<DT, false><<<grid_for(nblocks, 256), 256, 0, s>>>(x, y, nblocks, bs, e4m3);
  }
}

template <int DT>
void launch_quant_fp8(const void* x, int64_t rows, int64_t n, int bs, uint8_t* codes, float* scales, hipStream_t s) {
  const int64_t nthreads = rows * n / 4;
  quant_fp8_block_kernel<DT><<<grid_for(nthreads, 256), 256, 0, s>>>(x, codes, scales, nthreads, bs / 4, aligned16(x));
}

template <int DT>
void launch_pack_v41_fp8(const void* x, int d, int64_t n, const int64_t* dst, uint8_t* out, hipStream_t s) {
  pack_v41_kernel<DT, 0><<<grid_for(n, 256), 256, 0, s>>>(x, d, n, dst, out);
}
template <int DT>
void launch_pack_v41_fp4(const void* x, int d, int64_t n, const int64_t* dst, uint8_t* out, hipStream_t s) {
  pack_v41_kernel<DT, 1><<<grid_for(n, 256), 256, 0, s>>>(x, d, n, dst, out);
}
template <int DT>
void launch_unpack_v41_fp8(const uint8_t* cache, int d, int64_t n, void* y, hipStream_t s) {
  unpack_v41_kernel<DT, 0><<<grid_for(n, 256), 256, 0, s>>>(cache, d, n, y);
}
template <int DT>
void launch_unpack_v41_fp4(const uint8_t* cache, int d, int64_t n, void* y, hipStream_t s) {
  unpack_v41_kernel<DT, 1><<<grid_for(n, 256), 256, 0, s>>>(cache, d, n, y);
}

template <int DT>
void launch_quant_mxfp4(const void* x, int64_t rows, int64_t n, uint8_t* packed, uint8_t* e8m0, hipStream_t s) {
  const int64_t nthreads = rows * n / 4;
  quant_mxfp4_kernel<DT><<<grid_for(nthreads, 256), 256, 0, s>>>(x, packed, e8m0, nthreads, aligned16(x));
}

template <int DT>
void launch_dequant_fp8(const uint8_t* codes, const float* scales, int64_t rows, int64_t n, int bs, void* y, hipStream_t s) {
  const int64_t nthreads = rows * n / 4;
  dequant_fp8_block_kernel<DT><<<grid_for(nthreads, 256), 256, 0, s>>>(codes, scales, nthreads, bs, y);
}

template <int DT>
void launch_dequant_mxfp4(const uint8_t* packed, const uint8_t* e8m0, int64_t rows, int64_t n, void* y, hipStream_t s) {
  const int64_t nthreads = rows * n / 4;
  dequant_mxfp4_kernel<DT><<<grid_for(nthreads, 256), 256, 0, s>>>(packed, e8m0, nthreads, y);
}

inline int latent_threads(int nope, int rope) {
  int t = nope / 4;
  if (t < rope) t = rope;
  return ((t + 63) / 64) * 64;
}

template <int DT>
void launch_pack_latent(const void* x, int64_t rows, int nope, int rope, const int64_t* dst, uint8_t* cache, hipStream_t s) {
  pack_latent_kernel<DT><<<static_cast<unsigned>(rows), latent_threads(nope, rope), 0, s>>>(x, nope, rope, dst, cache);
}

template <int DT>
void launch_unpack_latent(const uint8_t* cache, int64_t rows, int nope, int rope, void* y, hipStream_t s) {
  unpack_latent_kernel<DT><<<static_cast<unsigned>(rows), latent_threads(nope, rope), 0, s>>>(cache, nope, rope, y);
}

template <int DT, int QDT>
int launch_prologue(const void* kv, int64_t B, int nope, int rope, const int64_t* positions, uint8_t* win,
                    int64_t wbe, int wcap, const void* q, int64_t qrows, int qdim, int qfmt, uint8_t* qcodes,
                    float* qscales, uint8_t* qe8m0, hipStream_t s) {
  const int64_t qthreads = qrows * qdim / 4;
  const unsigned grid = static_cast<unsigned>(B + (qthreads + 255) / 256);
  if (qfmt == 0)
    decode_prologue_kernel<DT, QDT, false><<<grid, 256, 0, s>>>(kv, B, nope, rope, positions, win, wbe, wcap, q,
                                                                 qthreads, 32, qcodes, qscales, qe8m0, aligned16(q));
  else
    decode_prologue_kernel<DT, QDT, true><<<grid, 256, 0, s>>>(kv, B, nope, rope, positions, win, wbe, wcap, q,
                                                                qthreads, 8, qcodes, qscales, qe8m0, aligned16(q));
  return MZK_OK;
}

template <int DT>
int launch_prologue_q(int qdt, const void* kv, int64_t B, int nope, int rope, const int64_t* positions, uint8_t* win,
                      int64_t wbe, int wcap, const void* q, int64_t qrows, int qdim, int qfmt, uint8_t* qcodes,
                      float* qscales, uint8_t* qe8m0, hipStream_t s) {
  switch (qdt) {
    case MZK_F32: return launch_prologue<DT, MZK_F32>(kv, B, nope, rope, positions, win, wbe, wcap, q, qrows, qdim, qfmt, qcodes, qscales, qe8m0, s);
    case MZK_BF16: return launch_prologue<DT, MZK_BF16>(kv, B, nope, rope, positions, win, wbe, wcap, q, qrows, qdim, qfmt, qcodes, qscales, qe8m0, s);
    case MZK_F16: return launch_prologue<DT, MZK_F16>(kv, B, nope, rope, positions, win, wbe, wcap, q, qrows, qdim, qfmt, qcodes, qscales, qe8m0, s);
    default: set_last_error("decode_prologue: unsupported query dtype %d", qdt); return MZK_EINVAL;
  }
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_decode_prologue(const void* kv, int kv_dtype, int64_t B, int nope, int rope,
                                   const int64_t* positions, uint8_t* win_cache, int64_t win_batch_entries,
                                   int win_cap, const void* q_idx, int q_dtype, int64_t q_rows, int q_dim,
                                   int q_format, uint8_t* q_codes, float* q_scales, uint8_t* q_e8m0, void* stream) {
  MZK_CHECK_ARG(B >= 0 && q_rows >= 0, "decode_prologue: bad sizes");
  MZK_CHECK_ARG(nope > 0 && nope % 128 == 0 && nope <= 1024 && rope >= 0 && rope % 2 == 0 && rope <= 256,
                "decode_prologue: nope must be a multiple of 128 (<= 1024), rope even (<= 256)");
  MZK_CHECK_ARG(win_cap >= 1 && win_batch_entries >= win_cap, "decode_prologue: bad window ring (cap %d)", win_cap);
  MZK_CHECK_ARG(q_format == 0 || q_format == 1, "decode_prologue: q_format must be 0 (FP8 b128) or 1 (MXFP4)");
  MZK_CHECK_ARG(q_format == 0 ? q_dim % 128 == 0 : q_dim % 32 == 0,
                "decode_prologue: q_dim must be a multiple of %d", q_format == 0 ? 128 : 32);
  if (B + q_rows == 0) return MZK_OK;
  MZK_CHECK_ARG(!B || (kv && positions && win_cache), "decode_prologue: null kv / positions / window");
  MZK_CHECK_ARG(!q_rows || (q_idx && q_codes && (q_format == 0 ? q_scales != nullptr : q_e8m0 != nullptr)),
                "decode_prologue: null query buffers");
  int rc;
  hipStream_t s = as_stream(stream);
  switch (kv_dtype) {
    case MZK_F32: rc = launch_prologue_q<MZK_F32>(q_dtype, kv, B, nope, rope, positions, win_cache, win_batch_entries, win_cap, q_idx, q_rows, q_dim, q_format, q_codes, q_scales, q_e8m0, s); break;
    case MZK_BF16: rc = launch_prologue_q<MZK_BF16>(q_dtype, kv, B, nope, rope, positions, win_cache, win_batch_entries, win_cap, q_idx, q_rows, q_dim, q_format, q_codes, q_scales, q_e8m0, s); break;
    case MZK_F16: rc = launch_prologue_q<MZK_F16>(q_dtype, kv, B, nope, rope, positions, win_cache, win_batch_entries, win_cap, q_idx, q_rows, q_dim, q_format, q_codes, q_scales, q_e8m0, s); break;
    default: set_last_error("decode_prologue: unsupported kv dtype %d", kv_dtype); return MZK_EINVAL;
  }
  if (rc) return rc;
  MZK_LAUNCH_CHECK("decode_prologue");
  return MZK_OK;
}

extern "C" int mzk_fake_quant_fp8_block(const void* x, void* y, int dtype, int64_t rows, int64_t n, int block_size,
                                        void* stream) {
  MZK_CHECK_ARG(x && y, "fake_quant_fp8_block: null pointer");
  MZK_CHECK_ARG(rows >= 0 && n > 0 && block_size > 0 && n % block_size == 0,
                "fake_quant_fp8_block: need n %% block_size == 0 (n=%lld, block_size=%d)", (long long)n, block_size);
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_fake, x, y, rows, n, block_size, false, false, as_stream(stream));
  MZK_LAUNCH_CHECK("fake_quant_fp8_block");
  return MZK_OK;
}

extern "C" int mzk_fake_quant_fp4_block(const void* x, void* y, int dtype, int64_t rows, int64_t n, int block_size,
                                        int e4m3_scales, void* stream) {
  MZK_CHECK_ARG(x && y, "fake_quant_fp4_block: null pointer");
  MZK_CHECK_ARG(rows >= 0 && n > 0 && block_size > 0 && n % block_size == 0,
                "fake_quant_fp4_block: need n %% block_size == 0 (n=%lld, block_size=%d)", (long long)n, block_size);
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_fake, x, y, rows, n, block_size, true, e4m3_scales != 0, as_stream(stream));
  MZK_LAUNCH_CHECK("fake_quant_fp4_block");
  return MZK_OK;
}

extern "C" int mzk_quant_fp8_block(const void* x, int dtype, int64_t rows, int64_t n, int block_size, uint8_t* codes,
                                   float* scales, void* stream) {
  MZK_CHECK_ARG(x && codes && scales, "quant_fp8_block: null pointer");
  MZK_CHECK_ARG(pow2_in(block_size, 4, 256) && n % block_size == 0 && rows >= 0,
                "quant_fp8_block: block_size must be a power of two in [4, 256] dividing n (n=%lld, block_size=%d)",
                (long long)n, block_size);
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_quant_fp8, x, rows, n, block_size, codes, scales, as_stream(stream));
  MZK_LAUNCH_CHECK("quant_fp8_block");
  return MZK_OK;
}

extern "C" int mzk_quant_mxfp4(const void* x, int dtype, int64_t rows, int64_t n, uint8_t* packed, uint8_t* e8m0,
                               void* stream) {
  MZK_CHECK_ARG(x && packed && e8m0, "quant_mxfp4: null pointer");
  MZK_CHECK_ARG(n % 32 == 0 && rows >= 0, "quant_mxfp4: n must be a multiple of 32 (n=%lld)", (long long)n);
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_quant_mxfp4, x, rows, n, packed, e8m0, as_stream(stream));
  MZK_LAUNCH_CHECK("quant_mxfp4");
  return MZK_OK;
}

extern "C" int mzk_dequant_fp8_block(const uint8_t* codes, const float* scales, int64_t rows, int64_t n, int block_size,
                                     void* y, int dtype, void* stream) {
  MZK_CHECK_ARG(codes && scales && y, "dequant_fp8_block: null pointer");
  MZK_CHECK_ARG(block_size >= 4 && block_size % 4 == 0 && n % block_size == 0 && rows >= 0,
                "dequant_fp8_block: need block_size %% 4 == 0 and n %% block_size == 0");
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_dequant_fp8, codes, scales, rows, n, block_size, y, as_stream(stream));
  MZK_LAUNCH_CHECK("dequant_fp8_block");
  return MZK_OK;
}

extern "C" int mzk_dequant_mxfp4(const uint8_t* packed, const uint8_t* e8m0, int64_t rows, int64_t n, void* y,
                                 int dtype, void* stream) {
  MZK_CHECK_ARG(packed && e8m0 && y, "dequant_mxfp4: null pointer");
  MZK_CHECK_ARG(n % 32 == 0 && rows >= 0, "dequant_mxfp4: n must be a multiple of 32");
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_dequant_mxfp4, packed, e8m0, rows, n, y, as_stream(stream));
  MZK_LAUNCH_CHECK("dequant_mxfp4");
  return MZK_OK;
}

extern "C" int mzk_pack_latent_fp8_b128(const void* x, int dtype, int64_t rows, int nope, int rope,
                                        const int64_t* dst_index, uint8_t* cache, void* stream) {
  MZK_CHECK_ARG(x && cache, "pack_latent_fp8_b128: null pointer");
  MZK_CHECK_ARG(nope > 0 && nope % 128 == 0 && nope <= 4096 && rope >= 0 && rope % 2 == 0 && rope <= 1024 && rows >= 0,
                "pack_latent_fp8_b128: nope must be a positive multiple of 128 (<= 4096), rope even (got %d, %d)",
                nope, rope);
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_pack_latent, x, rows, nope, rope, dst_index, cache, as_stream(stream));
  MZK_LAUNCH_CHECK("pack_latent_fp8_b128");
  return MZK_OK;
}

extern "C" int mzk_unpack_latent_fp8_b128(const uint8_t* cache, int64_t rows, int nope, int rope, void* y, int dtype,
                                          void* stream) {
  MZK_CHECK_ARG(cache && y, "unpack_latent_fp8_b128: null pointer");
  MZK_CHECK_ARG(nope > 0 && nope % 128 == 0 && nope <= 4096 && rope >= 0 && rope % 2 == 0 && rope <= 1024 && rows >= 0,
                "unpack_latent_fp8_b128: nope must be a positive multiple of 128, rope even");
  if (rows == 0) return MZK_OK;
  MZK_DISPATCH_DT(dtype, launch_unpack_latent, cache, rows, nope, rope, y, as_stream(stream));
  MZK_LAUNCH_CHECK("unpack_latent_fp8_b128");
  return MZK_OK;
}

extern "C" int mzk_pack_cache_v41(const void* x, int dtype, int64_t rows, int d, int fmt, uint8_t* out,
                                  const int64_t* dst_index, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && d >= 32 && d % 32 == 0, "pack_cache_v41: D must be a positive multiple of 32 (got %d)", d);
  MZK_CHECK_ARG(fmt == 0 || fmt == 1, "pack_cache_v41: fmt must be 0 (fp8, e8m0 per 32) or 1 (fp4, e4m3 per 16)");
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(x && out, "pack_cache_v41: null pointer");
  MZK_CHECK_ARG(aligned16(x) && reinterpret_cast<uintptr_t>(out) % 4 == 0, "pack_cache_v41: x 16-byte, out 4-byte aligned");
  const int64_t nthreads = rows * d / 4;
  hipStream_t s = as_stream(stream);
  if (fmt == 0) {
    MZK_DISPATCH_DT(dtype, launch_pack_v41_fp8, x, d, nthreads, dst_index, out, s);
  } else {
    MZK_DISPATCH_DT(dtype, launch_pack_v41_fp4, x, d, nthreads, dst_index, out, s);
  }
  MZK_LAUNCH_CHECK("pack_cache_v41");
  return MZK_OK;
}

extern "C" int mzk_unpack_cache_v41(const uint8_t* cache, int64_t rows, int d, int fmt, void* y, int dtype,
                                    void* stream) {
  MZK_CHECK_ARG(rows >= 0 && d >= 32 && d % 32 == 0, "unpack_cache_v41: D must be a positive multiple of 32 (got %d)",
                d);
  MZK_CHECK_ARG(fmt == 0 || fmt == 1, "unpack_cache_v41: fmt must be 0 (fp8) or 1 (fp4)");
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(cache && y, "unpack_cache_v41: null pointer");
  MZK_CHECK_ARG(reinterpret_cast<uintptr_t>(cache) % 4 == 0, "unpack_cache_v41: cache must be 4-byte aligned");
  const int64_t nthreads = rows * d / 4;
  hipStream_t s = as_stream(stream);
  if (fmt == 0) {
    MZK_DISPATCH_DT(dtype, launch_unpack_v41_fp8, cache, d, nthreads, y, s);
  } else {
    MZK_DISPATCH_DT(dtype, launch_unpack_v41_fp4, cache, d, nthreads, y, s);
  }
  MZK_LAUNCH_CHECK("unpack_cache_v41");
  return MZK_OK;
}

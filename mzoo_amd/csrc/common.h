// Shared device helpers and C-ABI plumbing for the mzoo_amd HIP library (gfx950).
//
// Numerics rules every kernel in this library follows (the build passes
// -ffp-contract=off, so a*b+c is two roundings unless written as fmaf):
//   * bf16 <-> fp32 conversion is done with integer arithmetic (round to nearest even),
//   * fp32 division and sqrt are the correctly rounded IEEE operations,
//   * fp32 denormals are kept (no flush to zero).
#pragma once

#include <hip/hip_runtime.h>
#include <atomic>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string>

#include "../../include/mzk.h"

namespace mzk {

// ------------------------------------------------------------------------------------
// error reporting
// ------------------------------------------------------------------------------------
void set_last_error(const char* fmt, ...);

#define MZK_CHECK_ARG(cond, ...)                                                   \
  do {                                                                              \
    if (!(cond)) {                                                                  \
      ::mzk::set_last_error(__VA_ARGS__);                                           \
      return MZK_EINVAL;                                                            \
    }                                                                               \
  } while (0)

// Vector loads and stores of 16 bytes need 16-byte aligned base pointers (null passes).
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define MZK_LAUNCH_CHECK(name)                                                      \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess) {                                                         \
      ::mzk::set_last_error("%s: launch failed: %s", name, hipGetErrorString(_e)); \
      return MZK_ELAUNCH;                                                           \
    }                                                                               \
  } while (0)

// Call FN<DT>(args...) for a runtime dtype code (inside a function returning int).
#define MZK_DISPATCH_DT(dtype, FN, ...)                               \
  switch (dtype) {                                                    \
    case MZK_F32: FN<MZK_F32>(__VA_ARGS__); break;                    \
    case MZK_BF16: FN<MZK_BF16>(__VA_ARGS__); break;                  \
    case MZK_F16: FN<MZK_F16>(__VA_ARGS__); break;                    \
    default: set_last_error("unsupported dtype %d", dtype); return MZK_EINVAL; \
  }

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kMaxDevices = 64;  // per-device one-time launch attributes (dynamic-LDS limits)

// ------------------------------------------------------------------------------------
// scalar conversions
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((b >> 16) | 0x40);  // quiet NaN
  b += 0x7fffu + ((b >> 16) & 1u);
  return static_cast<uint16_t>(b >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> fp16, round to nearest even, in integer arithmetic.  (A plain conversion lets
// the compiler fold a preceding multiply into v_fma_mix*_f16 with a +0 addend, which
// turns a -0.0 product into +0.0.)
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  const uint32_t b = __float_as_uint(f);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const uint32_t a = b & 0x7fffffffu;
  uint32_t h;
  if (a > 0x7f800000u) h = 0x7e00u;                         // NaN
  else if (a >= 0x477ff000u) h = 0x7c00u;                   // rounds to +-inf
  else if (a >= 0x38800000u) h = ((a + 0xfffu + ((a >> 13) & 1u)) >> 13) - (112u << 10);  // normal
  else h = static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 16777216.0f));      // 2^-24 steps
  return static_cast<uint16_t>(h | sign);
}

// Correctly rounded fp32 square root and division.  (HIP's __fsqrt_rn is the ~1 ulp
// hardware v_sqrt_f32 unless OCML_BASIC_ROUNDED_OPERATIONS is defined; the plain
// operators are correctly rounded under -fhip-fp32-correctly-rounded-divide-sqrt,
// which the build passes explicitly.)
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }

// Load element i of a tensor of the given dtype as fp32.
template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == MZK_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == MZK_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// Elements i .. i+3 (i a multiple of 4) as fp32: one 8- or 16-byte load when `vec` (the
// caller has checked that the base pointer is 16-byte aligned), else four element loads.
template <int DT>
__device__ __forceinline__ void load4_as_f32(const void* p, int64_t i, bool vec, float (&v)[4]) {
  if (vec) {
    if constexpr (DT == MZK_F32) {
      const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
      v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
      const uint16_t h[4] = {static_cast<uint16_t>(u.x & 0xffffu), static_cast<uint16_t>(u.x >> 16),
                             static_cast<uint16_t>(u.y & 0xffffu), static_cast<uint16_t>(u.y >> 16)};
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = DT == MZK_BF16 ? bf16_to_f32(h[k]) : f16_to_f32(h[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = load_as_f32<DT>(p, i + k);
  }
}

// Round fp32 to the dtype and store (the ".to(x.dtype)" of the reference).
template <int DT>
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v) {
  if constexpr (DT == MZK_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == MZK_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
}

// fp32 value rounded to the dtype, returned as fp32.
template <int DT>
__device__ __forceinline__ float round_to_dtype(float v) {
  if constexpr (DT == MZK_F32) return v;
  else if constexpr (DT == MZK_BF16) return bf16_to_f32(f32_to_bf16(v));
  else return f16_to_f32(f32_to_f16(v));
}

// 2^k for integer k in [-126, 127] built from the exponent field.
__device__ __forceinline__ float pow2i(int k) { return __uint_as_float(static_cast<uint32_t>(k + 127) << 23); }

// ue8m0 scale: 2^(E - 127 + (M != 0)) from the fp32 fields of t > 0 (power of two
// rounded up).  Results below 2^-126 are built exactly as subnormals.
__device__ __forceinline__ float pow2_ceil(float t) {
  uint32_t b = __float_as_uint(t);
  int k = static_cast<int>((b >> 23) & 0xffu) - 127 + ((b & 0x7fffffu) != 0u);
  if (k >= 128) return __uint_as_float(0x7f800000u);
  if (k >= -126) return pow2i(k);
  return __uint_as_float(1u << (k + 149));  // k in [-127, -126) only for t == 0 / subnormal t
}

// ------------------------------------------------------------------------------------
// FP8 e4m3 (OCP e4m3fn) encode/decode, integer arithmetic, round to nearest even.
// |x| >= 480 or NaN -> NaN code 0x7f (with sign); the sign of zero is kept.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ uint8_t e4m3_encode(float x) {
  uint32_t b = __float_as_uint(x);
  uint32_t sign = (b >> 24) & 0x80u;
  uint32_t a = b & 0x7fffffffu;
  uint32_t code;
  if (a >= 0x43f00000u) {               // >= 480.0f or NaN
    code = 0x7fu;
  } else if (a >= 0x3c800000u) {        // >= 2^-6: normal
    uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;  // 8-bit exp : 3-bit mantissa
    code = r - ((127u - 7u) << 3);
  } else {                              // subnormal: nearest multiple of 2^-9, ties to even
    float s = __uint_as_float(a) * 512.0f;                 // exact
    code = static_cast<uint32_t>(__builtin_rintf(s));      // 0..8 (8 = smallest normal)
  }
  return static_cast<uint8_t>(code | sign);
}

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  // place the 7 magnitude bits at the fp32 exponent/mantissa boundary, then rescale by
  // 2^120: exact for normals and subnormals alike (fp32 denormals are kept).
  uint32_t mag = (c & 0x7fu) << 20;
  float v = __uint_as_float(mag) * 1.329227995784916e+36f;  // 2^120
  if ((c & 0x7fu) == 0x7fu) v = __uint_as_float(0x7fc00000u);
  return (c & 0x80u) ? -v : v;
}

// FP8 block scale of the reference's fake quantizer (owlet1/quant.py:72-86):
// s = pow2ceil(max(amax, 1e-4) * fp32(1/448)); codes are e4m3(clamp(x / s, +-448)).
constexpr float kInv448 = 1.0f / 448.0f;  // the fp32-rounded reciprocal the reference multiplies by

// Maximum of two values that are >= 0 or NaN (block maxima of |x|), as the integer maximum
// of their bit patterns: for such values the patterns order as the values do, and a NaN
// (any payload, sign cleared by fabsf) sorts above +inf -- so a NaN anywhere in a block
// makes its maximum NaN, as torch's amax does (fmaxf would drop it).
__device__ __forceinline__ float nn_max(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// max |v[i]| over four values, NaN-propagating (see nn_max).
__device__ __forceinline__ float abs_max4(const float (&v)[4]) {
  return nn_max(nn_max(fabsf(v[0]), fabsf(v[1])), nn_max(fabsf(v[2]), fabsf(v[3])));
}

// The floors of the reference's scales are torch clamp_min calls, which keep a NaN amax:
// nn_max keeps it too.  pow2_ceil maps a NaN or infinite amax to an infinite scale, so
// x / s is 0 for finite x and the dequantized block is NaN (0 * inf), as in the reference.
__device__ __forceinline__ float fp8_scale_from_amax(float amax) {
  return pow2_ceil(nn_max(amax, 1e-4f) * kInv448);
}

// clamp(v, -lim, lim) keeping NaN, like torch's clamp (fminf / fmaxf would turn a NaN
// into one of the bounds).
__device__ __forceinline__ float clampf(float v, float lim) { return v != v ? v : fminf(fmaxf(v, -lim), lim); }

// FP4 block scale of the reference's fake quantizer (owlet1/quant.py:49-66): ue8m0
// pow2ceil(max(amax, 6*2^-126) * fp32(1/6)), or with e4m3 scales e4m3(max(amax, 6*2^-9) / 6).
constexpr float kInv6 = 1.0f / 6.0f;  // the fp32-rounded reciprocal the reference multiplies by

__device__ __forceinline__ float fp4_scale_from_amax(float amax, bool e4m3_scales) {
  if (e4m3_scales) return e4m3_decode(e4m3_encode(div_rn(nn_max(amax, 0x1.8p-7f /* 6*2^-9 */), 6.0f)));
  return pow2_ceil(nn_max(amax, 0x1.8p-124f /* 6*2^-126 */) * kInv6);
}

// ------------------------------------------------------------------------------------
// FP4 e2m1 codes.  code = number of thresholds <= |q| (ties at 0.25/1.25/2.5/5 round
// down, at 0.75/1.75/3.5 round up), sign in bit 3 from the sign bit (-0 -> 8).
// ------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t e2m1_code(float q) {
  float a = fabsf(q);
  uint32_t c = (a >= 0x1.000002p-2f) + (a >= 0.75f) + (a >= 0x1.400002p+0f) + (a >= 1.75f) +
               (a >= 0x1.400002p+1f) + (a >= 3.5f) + (a >= 0x1.400002p+2f);
  return c | ((__float_as_uint(q) >> 28) & 0x8u);
}

__device__ __forceinline__ float e2m1_value(uint32_t code) {
  // {0, .5, 1, 1.5, 2, 3, 4, 6}; code 8 decodes to +0.0
  const uint32_t m = code & 7u;
  float v = (m < 4u) ? 0.5f * static_cast<float>(m)
                     : static_cast<float>(1u << (((m - 4u) >> 1) + 1u)) * ((m & 1u) ? 1.5f : 1.0f);
  return ((code & 8u) && m) ? -v : v;
}

// ------------------------------------------------------------------------------------
// gfx950 hardware conversions
// ------------------------------------------------------------------------------------
typedef __bf16 mzk_v2bf __attribute__((ext_vector_type(2)));

// 8 e4m3 codes (little-endian in `raw`) times a power-of-two `scale` -> 8 bf16 (as 4
// dwords, element 2i in the low half of dword i), with v_cvt_scalef32_pk_bf16_fp8.  Exact:
// an e4m3 value has 4 significant bits, so code * 2^k is representable in bf16.
__device__ __forceinline__ uint4 dequant_fp8x8_bf16(uint2 raw, float scale) {
  const mzk_v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(raw.x), scale, false);
  const mzk_v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(raw.x), scale, true);
  const mzk_v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(raw.y), scale, false);
  const mzk_v2bf d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(raw.y), scale, true);
  return uint4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, c),
               __builtin_bit_cast(uint32_t, d)};
}

// Two fp32 -> packed bf16x2 (round to nearest even) with v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const mzk_v2bf v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// One RoPE pair of bf16 channels (even in the low half): bf16(e*c - o*s), bf16(e*s + o*c),
// each product and sum rounded to fp32 (no fused multiply-add), then to bf16 by the
// hardware's round-to-nearest-even pack -- owlet1/norm_rope.py:141-145.  The inverse
// rotation is the same call with -s (the reference negates sin).
__device__ __forceinline__ uint32_t rope_pair_bf16(uint32_t pair, float c, float s) {
  const float e = __uint_as_float(pair << 16);
  const float o = __uint_as_float(pair & 0xffff0000u);
  return pack_bf16x2(e * c - o * s, e * s + o * c);
}


// ------------------------------------------------------------------------------------
// The compressor's pinned float32 exp (the CPU restatement oracle/compressor.py evaluates
// the same operation sequence): n = rint(x*log2e), r = (x - n*ln2_hi) - n*ln2_lo, degree-7
// Taylor in Horner form, times 2^n through the exponent field (two steps below 2^-126);
// no fused operations.  Max error ~2 ulp.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float exp_pinned(float x) {
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.42860682030941723e-06f;
  const float c[8] = {1.0f, 1.0f, 0.5f, 1.0f / 6.0f, 1.0f / 24.0f, 1.0f / 120.0f, 1.0f / 720.0f, 1.0f / 5040.0f};
  float n = __builtin_rintf(x * kLog2e);
  n = fminf(fmaxf(n, -160.0f), 160.0f);
  const float r = (x - n * kLn2Hi) - n * kLn2Lo;
  float p = c[7];
#pragma unroll
  for (int i = 6; i >= 0; --i) p = p * r + c[i];
  const int ni = static_cast<int>(n);
  const int hi = ni < -126 ? -126 : (ni > 127 ? 127 : ni);
  float out = p * pow2i(hi);
  if (ni < -126) {
    int lo = ni + 64;
    lo = lo < -126 ? -126 : (lo > 127 ? 127 : lo);
    out = (p * pow2i(lo)) * 5.421010862427522e-20f;  // * 2^-64
  }
  if (x < -104.0f) out = 0.0f;
  if (x > 88.8f) out = __builtin_huge_valf();
  if (x != x) out = x;
  return out;
}

// ------------------------------------------------------------------------------------
// wave helpers (wave64)
// ------------------------------------------------------------------------------------
// Maximum of values >= 0 or NaN (block maxima of |x|; NaN wins, see nn_max) over aligned
// groups of `group` consecutive lanes.
__device__ __forceinline__ float wave_max_group(float v, int group) {
  for (int m = group >> 1; m >= 1; m >>= 1) v = nn_max(v, __shfl_xor(v, m, 64));
  return v;
}

// The value of lane (lane ^ M), exactly: DPP quad permutes for 1 and 2, DPP row shifts up
// or down (by lane bit M) for 4 and 8, a swizzle for 16, a permute through LDS for 32.
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "xor partner distance");
  const int x = __float_as_int(v);
  if constexpr (M == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4 || M == 8) {
    const int from_up = __builtin_amdgcn_mov_dpp(x, 0x100 + M, 0xF, 0xF, false);  // row_shl: lane + M
    const int from_dn = __builtin_amdgcn_mov_dpp(x, 0x110 + M, 0xF, 0xF, false);  // row_shr: lane - M
    return __int_as_float((threadIdx.x & M) ? from_dn : from_up);
  } else if constexpr (M == 16) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x401F));  // and 0x1f, xor 0x10
  } else {
    return __shfl_xor(v, 32, 64);
  }
}

// Maximum of values >= 0 or NaN (NaN wins, see nn_max) over aligned groups of `group`
// consecutive lanes (a power of two <= 32), by exact xor-partner exchanges; every lane of a
// group ends with the group's maximum.
__device__ __forceinline__ float group_max(float v, int group) {
  if (group > 16) v = nn_max(v, lane_xor<16>(v));
  if (group > 8) v = nn_max(v, lane_xor<8>(v));
  if (group > 4) v = nn_max(v, lane_xor<4>(v));
  if (group > 2) v = nn_max(v, lane_xor<2>(v));
  if (group > 1) v = nn_max(v, lane_xor<1>(v));
  return v;
}

// 1 / s for a power of two s in [2^-126, 2^126] (exact): the exponent negated
__device__ __forceinline__ float pow2_reciprocal(float s) { return __uint_as_float((254u << 23) - __float_as_uint(s)); }

// Maximum of v >= 0 or NaN (NaN wins, see nn_max) over the 16 lanes of each DPP row, in
// the row's last lane (lane 15 of the row); the shifts bring in 0 from beyond the row,
// which a maximum of values >= 0 ignores.
__device__ __forceinline__ float row_max_nonneg(float v) {
  v = nn_max(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x111, 0xF, 0xF, true)));
  v = nn_max(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x112, 0xF, 0xF, true)));
  v = nn_max(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x114, 0xF, 0xF, true)));
  v = nn_max(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x118, 0xF, 0xF, true)));
  return v;
}

// Maximum of v >= 0 or NaN over the wave, as a wave-uniform value.
__device__ __forceinline__ float wave_max_nonneg(float v) {
  const int r = __float_as_int(row_max_nonneg(v));
  return nn_max(nn_max(__int_as_float(__builtin_amdgcn_readlane(r, 15)), __int_as_float(__builtin_amdgcn_readlane(r, 31))),
                nn_max(__int_as_float(__builtin_amdgcn_readlane(r, 47)), __int_as_float(__builtin_amdgcn_readlane(r, 63))));
}

}  // namespace mzk

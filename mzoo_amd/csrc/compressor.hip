// Piece 2: the KV compressor (gated softmax pool over `ratio` tokens + RMSNorm) and the
// interleaved RoPE it is followed by.
//
//   latent[b, g, :] = RMSNorm( dtype( sum_r kv[b, g*ratio + r, :] * softmax_r(gate[b, g*ratio + r, :]) ) )
//   -- src/mzoo/archs/owlet1/cache.py:142-172 (DeepseekV41Compressor.forward, fp32 pooling),
//      owlet1/norm_rope.py:25-30 (RMSNorm: h * rsqrt(mean(h^2) + eps), dtype, weight * h).
//   ratio 1: latent = RMSNorm(dtype(kv)) (the un-gated per-token projection).
//   rope: owlet1/norm_rope.py:126-145 (pairs (even, odd) of the trailing rope channels,
//   fp32 math, inverse = conjugate rotation).
//
// Bit-exact by construction against the CPU restatement (oracle/compressor.py): both
// evaluate the same float32 operation sequence --
//   exp: n = rint(x*log2e), r = (x - n*ln2_hi) - n*ln2_lo, degree-7 Taylor in Horner form,
//        times 2^n through the exponent field (two steps below 2^-126); no fused ops;
//   softmax over r: running max, exp(g_r - max), sum from 0 in r order, divide;
//   pooled: sum from 0 in r order of kv_r * p_r;
//   RMSNorm: lane l of the wave sums channels l, l+64, ... in order from 0, then the xor
//   butterfly (32, 16, 8, 4, 2, 1); var = sum / D; rsqrt = 1 / sqrt (correctly rounded).
// Layout: one wave per (b, group); lane l owns channels l + 64 i (coalesced 256 B rows).
#include "common.h"

namespace mzk {
namespace {

constexpr int kMaxPerLane = 16;  // D <= 1024

template <int ODT, int WDT>
__global__ void __launch_bounds__(256) compress_kernel(const float* __restrict__ kv, const float* __restrict__ gate,
                                                       int64_t B, int64_t n_groups, int ratio, int D,
                                                       int64_t tokens_per_batch, const void* __restrict__ weight,
                                                       float eps, void* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t rid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (rid >= B * n_groups) return;  // whole waves
  const int64_t b = rid / n_groups;
  const int64_t g = rid - b * n_groups;
  const float* kvb = kv + (b * tokens_per_batch + g * ratio) * D;
  const float* gtb = gate ? gate + (b * tokens_per_batch + g * ratio) * D : nullptr;

  float h[kMaxPerLane];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int d = lane + 64 * i;
    h[i] = 0.0f;
    if (d < D) {
      float v;
      if (ratio == 1) {
        v = kvb[d];
      } else {
        float m = gtb[d];
        for (int r = 1; r < ratio; ++r) m = fmaxf(m, gtb[static_cast<int64_t>(r) * D + d]);
        float s = 0.0f;
        for (int r = 0; r < ratio; ++r) s = s + exp_pinned(gtb[static_cast<int64_t>(r) * D + d] - m);
        float acc = 0.0f;
        for (int r = 0; r < ratio; ++r) {
          const float e = exp_pinned(gtb[static_cast<int64_t>(r) * D + d] - m);
          acc = acc + kvb[static_cast<int64_t>(r) * D + d] * div_rn(e, s);
        }
        v = acc;
      }
      v = round_to_dtype<ODT>(v);  // latent.to(dtype) before the norm
      h[i] = v;
      ss = ss + v * v;
    }
  }
  // xor butterfly: every lane ends with the same total
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss = ss + __shfl_xor(ss, m, 64);
  const float var = div_rn(ss, static_cast<float>(D));
  const float inv = div_rn(1.0f, sqrt_rn(var + eps));
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int d = lane + 64 * i;
    if (d < D) {
      const float normed = round_to_dtype<ODT>(h[i] * inv);
      const float w = load_as_f32<WDT>(weight, d);
      store_from_f32<ODT>(out, rid * D + d, w * normed);
    }
  }
}

// DeepseekV41RMSNorm (owlet1/norm_rope.py:25-30) of any width: one wave per row, the sum
// of squares in the pinned order above (lane l sums channels l, l+64, ... from 0, then the
// xor butterfly), var = sum / D, inv = 1 / sqrt(var + eps); normed = IDT(h * inv) (the
// ".to(input_dtype)"), out = ODT(weight * normed).  Two passes over the row (L2-resident).
template <int IDT, int WDT, int ODT>
__global__ void __launch_bounds__(256) rms_norm_kernel(const void* __restrict__ x, int64_t rows, int D,
                                                       int64_t x_stride, const void* __restrict__ weight, float eps,
                                                       void* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int64_t base = row * x_stride;
  float ss = 0.0f;
  for (int d = lane; d < D; d += 64) {
    const float v = load_as_f32<IDT>(x, base + d);
    ss = ss + v * v;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss = ss + __shfl_xor(ss, m, 64);
  const float var = div_rn(ss, static_cast<float>(D));
  const float inv = div_rn(1.0f, sqrt_rn(var + eps));
  for (int d = lane; d < D; d += 64) {
    const float normed = round_to_dtype<IDT>(load_as_f32<IDT>(x, base + d) * inv);
    store_from_f32<ODT>(out, row * D + d, load_as_f32<WDT>(weight, d) * normed);
  }
}

template <int IDT, int WDT>
int launch_rms_norm_o(int odt, const void* x, int64_t rows, int D, int64_t xs, const void* w, float eps, void* out,
                      hipStream_t s) {
  const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
  switch (odt) {
    case MZK_F32: rms_norm_kernel<IDT, WDT, MZK_F32><<<grid, 256, 0, s>>>(x, rows, D, xs, w, eps, out); break;
    case MZK_BF16: rms_norm_kernel<IDT, WDT, MZK_BF16><<<grid, 256, 0, s>>>(x, rows, D, xs, w, eps, out); break;
    case MZK_F16: rms_norm_kernel<IDT, WDT, MZK_F16><<<grid, 256, 0, s>>>(x, rows, D, xs, w, eps, out); break;
    default: set_last_error("rms_norm: unsupported out dtype %d", odt); return MZK_EINVAL;
  }
  return MZK_OK;
}

template <int IDT>
int launch_rms_norm(int wdt, int odt, const void* x, int64_t rows, int D, int64_t xs, const void* w, float eps,
                    void* out, hipStream_t s) {
  switch (wdt) {
    case MZK_F32: return launch_rms_norm_o<IDT, MZK_F32>(odt, x, rows, D, xs, w, eps, out, s);
    case MZK_BF16: return launch_rms_norm_o<IDT, MZK_BF16>(odt, x, rows, D, xs, w, eps, out, s);
    case MZK_F16: return launch_rms_norm_o<IDT, MZK_F16>(odt, x, rows, D, xs, w, eps, out, s);
    default: set_last_error("rms_norm: unsupported weight dtype %d", wdt); return MZK_EINVAL;
  }
}

// rows x D (dtype DT); cos/sin [rows / heads, rd/2] fp32, broadcast over `heads`
// consecutive rows.  Nope channels are copied through unchanged.
template <int DT>
__global__ void rope_kernel(const void* __restrict__ x, const float* __restrict__ cosv, const float* __restrict__ sinv,
                            int64_t rows, int D, int rd, int heads, int inverse, void* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int half = rd / 2;
  const int per_row = (D - rd) + half;  // nope channels + rope pairs
  if (t >= rows * per_row) return;
  const int64_t row = t / per_row;
  const int k = static_cast<int>(t - row * per_row);
  const int64_t base = row * D;
  if (k < D - rd) {
    store_from_f32<DT>(y, base + k, load_as_f32<DT>(x, base + k));
    return;
  }
  const int i = k - (D - rd);
  const int64_t crow = row / heads;
  const float c = cosv[crow * half + i];
  const float s = inverse ? -sinv[crow * half + i] : sinv[crow * half + i];
  const float ev = load_as_f32<DT>(x, base + (D - rd) + 2 * i);
  const float od = load_as_f32<DT>(x, base + (D - rd) + 2 * i + 1);
  store_from_f32<DT>(y, base + (D - rd) + 2 * i, ev * c - od * s);
  store_from_f32<DT>(y, base + (D - rd) + 2 * i + 1, ev * s + od * c);
}

template <int ODT>
int launch_compress_w(int wdt, const float* kv, const float* gate, int64_t B, int64_t n, int ratio, int D, int64_t tpb,
                      const void* w, float eps, void* out, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>((B * n + 3) / 4);
  switch (wdt) {
    case MZK_F32: compress_kernel<ODT, MZK_F32><<<grid, 256, 0, s>>>(kv, gate, B, n, ratio, D, tpb, w, eps, out); break;
    case MZK_BF16: compress_kernel<ODT, MZK_BF16><<<grid, 256, 0, s>>>(kv, gate, B, n, ratio, D, tpb, w, eps, out); break;
    case MZK_F16: compress_kernel<ODT, MZK_F16><<<grid, 256, 0, s>>>(kv, gate, B, n, ratio, D, tpb, w, eps, out); break;
    default: set_last_error("compress: unsupported weight dtype %d", wdt); return MZK_EINVAL;
  }
  return MZK_OK;
}

template <int DT>
void launch_rope(const void* x, const float* c, const float* sn, int64_t rows, int D, int rd, int heads, int inverse,
                 void* y, hipStream_t s) {
  const int64_t n = rows * ((D - rd) + rd / 2);
  rope_kernel<DT><<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(x, c, sn, rows, D, rd, heads, inverse, y);
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_compress(const float* kv, const float* gate, int64_t B, int64_t n_groups, int ratio, int D,
                            int64_t tokens_per_batch, const void* norm_weight, int weight_dtype, float eps, void* out,
                            int out_dtype, void* stream) {
  MZK_CHECK_ARG(B >= 0 && n_groups >= 0 && ratio >= 1 && D >= 1 && D <= 64 * kMaxPerLane,
                "compress: bad sizes (ratio >= 1, 1 <= D <= %d)", 64 * kMaxPerLane);
  MZK_CHECK_ARG(tokens_per_batch >= n_groups * ratio, "compress: tokens_per_batch < n_groups * ratio");
  if (B * n_groups == 0) return MZK_OK;
  MZK_CHECK_ARG(kv && norm_weight && out && (ratio == 1 || gate), "compress: null pointer");
  int rc;
  hipStream_t s = as_stream(stream);
  switch (out_dtype) {
    case MZK_F32: rc = launch_compress_w<MZK_F32>(weight_dtype, kv, gate, B, n_groups, ratio, D, tokens_per_batch,
                                                  norm_weight, eps, out, s); break;
    case MZK_BF16: rc = launch_compress_w<MZK_BF16>(weight_dtype, kv, gate, B, n_groups, ratio, D, tokens_per_batch,
                                                    norm_weight, eps, out, s); break;
    case MZK_F16: rc = launch_compress_w<MZK_F16>(weight_dtype, kv, gate, B, n_groups, ratio, D, tokens_per_batch,
                                                  norm_weight, eps, out, s); break;
    default: set_last_error("compress: unsupported out dtype %d", out_dtype); return MZK_EINVAL;
  }
  if (rc) return rc;
  MZK_LAUNCH_CHECK("compress");
  return MZK_OK;
}

extern "C" int mzk_rope(const void* x, int dtype, const float* cos_t, const float* sin_t, int64_t rows, int D,
                        int rope_dim, int heads, int inverse, void* y, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && D >= 1 && rope_dim >= 0 && rope_dim <= D && rope_dim % 2 == 0 && heads >= 1,
                "rope: bad sizes (even rope_dim <= D, heads >= 1)");
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(x && y && (rope_dim == 0 || (cos_t && sin_t)), "rope: null pointer");
  MZK_DISPATCH_DT(dtype, launch_rope, x, cos_t, sin_t, rows, D, rope_dim, heads, inverse, y, as_stream(stream));
  MZK_LAUNCH_CHECK("rope");
  return MZK_OK;
}

extern "C" int mzk_rms_norm(const void* x, int x_dtype, int64_t rows, int D, int64_t x_row_stride,
                            const void* weight, int weight_dtype, float eps, void* out, int out_dtype, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && D >= 1 && x_row_stride >= D, "rms_norm: bad sizes (D >= 1, row stride >= D)");
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(x && weight && out, "rms_norm: null pointer");
  hipStream_t s = as_stream(stream);
  int rc;
  switch (x_dtype) {
    case MZK_F32: rc = launch_rms_norm<MZK_F32>(weight_dtype, out_dtype, x, rows, D, x_row_stride, weight, eps, out, s); break;
    case MZK_BF16: rc = launch_rms_norm<MZK_BF16>(weight_dtype, out_dtype, x, rows, D, x_row_stride, weight, eps, out, s); break;
    case MZK_F16: rc = launch_rms_norm<MZK_F16>(weight_dtype, out_dtype, x, rows, D, x_row_stride, weight, eps, out, s); break;
    default: set_last_error("rms_norm: unsupported input dtype %d", x_dtype); return MZK_EINVAL;
  }
  if (rc) return rc;
  MZK_LAUNCH_CHECK("rms_norm");
  return MZK_OK;
}

// Compressed-group emission inside the decode step: the per-token work of
// DeepseekV41Compressor / DeepseekV41CSACache / the indexer's key publication / the
// compressed-cache append (owlet1/cache.py:96-124, :159-172; owlet1/indexer.py:96-117;
// owlet1/attention.py:173-192), for one new token per batch row, with all state on the
// device so the step can be recorded into a graph and replayed with advancing positions.
//
// One workgroup (256 threads) per batch row, one launch per compressed branch.  Every step:
//   * the token's fp32 compressor projections (kv, gate) go to slot pos % ratio of the
//     row's carry ring (the partial group the reference buffers with torch.cat);
//   * optionally, the token's RoPE tables, row `pos` of a position-indexed table, are copied
//     into the step's cos / sin buffers (the later launches of the step read them).
// When the token completes a group ((pos + 1) % ratio == 0), group g = (pos+1)/ratio - 1:
//   * pool: softmax over the ratio tokens of the gate, per channel, weighted sum of kv
//     (fp32, the compressor kernel's pinned order), rounded to bf16 -> RMSNorm (pinned sum
//     of squares) -> bf16 latent;
//   * main entry: RoPE of the trailing 64 channels at the group's position g * ratio, the
//     FP8-b128 entry (656 B) written to entry g of the row's cache;
//   * index key (branches with one): k = bf16(latent . wk^T) with a pinned order (each output
//     sums channels [0, D/2) and [D/2, D) sequentially, then adds the halves), k_norm, RoPE of
//     the trailing 64 channels at g * ratio, quantized (FP8 b128 + fp32 scale, or MXFP4 +
//     e8m0) to key g.
// Layout constants: latent 512 + 64 (nope + rope), index key 128; bf16 activations.
#include "common.h"

namespace mzk {
namespace {

constexpr int kD = 576;
constexpr int kNope = 512;
constexpr int kRopePairs = 32;  // rope 64
constexpr int kDi = 128;
constexpr int kEntryBytes = kNope + 4 * (kNope / 128) + 2 * 2 * kRopePairs;  // 656
constexpr int kHalf = kD / 2;

struct EmitBranch {
  const float* kv;        // [B, D] fp32: this token's compressor kv projection
  const float* gate;      // [B, D] fp32: its gate projection (unused at ratio 1)
  float* carry_kv;        // [B, ratio, D] fp32
  float* carry_gate;      // [B, ratio, D] fp32
  int ratio;
  const uint16_t* norm_w;  // bf16 [D]: the compressor's RMSNorm weight
  float eps;
  uint8_t* cache;          // FP8-b128 entries, row b's entry g at b * cache_batch + g
  int64_t cache_batch;
  int64_t cache_cap;       // groups a row can hold
  const uint16_t* wk;      // bf16 [Di, D] (nn.Linear layout) or nullptr: no index key
  const uint16_t* kn_w;    // bf16 [Di]: k_norm weight
  float k_eps;
  int key_fmt;             // 0: FP8 b128 (codes [.., 128] + fp32 scale), 1: MXFP4 (packed [.., 64] + e8m0 [.., 4])
  uint8_t* k_codes;
  void* k_scales;
  int64_t key_batch;
};

struct EmitParams {
  EmitBranch br;
  const int64_t* positions;  // [B]
  const uint16_t* tab;       // bf16 [tab_rows, 64]: cos (32) | sin (32) of position p in row p
  int64_t tab_rows;
  uint16_t* step_cos;        // [B, 32] bf16 or nullptr
  uint16_t* step_sin;
};

__device__ __forceinline__ float bf(float v) { return round_to_dtype<MZK_BF16>(v); }

// One RoPE pair (fp32 math, no fused operations, rounded to bf16) -- norm_rope.py:141-145.
__device__ __forceinline__ void rope_pair(float& e, float& o, float c, float s) {
  const float a = e * c - o * s;
  const float b = e * s + o * c;
  e = bf(a);
  o = bf(b);
}

__global__ void __launch_bounds__(256) emit_kernel(EmitParams p) {
  __shared__ float lat[kD];
  __shared__ float part[2][kDi];
  __shared__ float kvec[kDi];
  __shared__ float inv_s[2];
  const int t = threadIdx.x;
  const int64_t b = blockIdx.x;
  const EmitBranch& br = p.br;
  const int64_t pos = p.positions[b];
  if (pos < 0) return;  // an inactive row: nothing to carry or emit
  if (p.step_cos && t < 2 * kRopePairs && pos < p.tab_rows) {
    const uint16_t v = p.tab[pos * 2 * kRopePairs + t];
    if (t < kRopePairs) p.step_cos[b * kRopePairs + t] = v;
    else p.step_sin[b * kRopePairs + (t - kRopePairs)] = v;
  }
  const int r = br.ratio;
  const int slot = static_cast<int>(pos % r);
  const float* kvb = br.kv + b * kD;
  const float* gtb = br.gate + b * kD;
  float* ckv = br.carry_kv + b * static_cast<int64_t>(r) * kD;
  float* cgt = br.carry_gate + b * static_cast<int64_t>(r) * kD;
  for (int d = t; d < kD; d += 256) {
    ckv[slot * kD + d] = kvb[d];
    if (r > 1) cgt[slot * kD + d] = gtb[d];
  }
  if ((pos + 1) % r != 0) return;  // uniform over the workgroup
  const int64_t g = (pos + 1) / r - 1;
  const int64_t gp = g * r;  // the group's position (its first token)
  if (g >= br.cache_cap || gp >= p.tab_rows) return;

  // ---- pool (slot r - 1 is this token: read from the input, not the carry just written)
  for (int d = t; d < kD; d += 256) {
    float v;
    if (r == 1) {
      v = kvb[d];
    } else {
      float m = cgt[d];
      for (int i = 1; i < r; ++i) m = fmaxf(m, i == r - 1 ? gtb[d] : cgt[i * kD + d]);
      float s = 0.0f;
      for (int i = 0; i < r; ++i) s = s + exp_pinned((i == r - 1 ? gtb[d] : cgt[i * kD + d]) - m);
      float acc = 0.0f;
      for (int i = 0; i < r; ++i) {
        const float e = exp_pinned((i == r - 1 ? gtb[d] : cgt[i * kD + d]) - m);
        acc = acc + (i == r - 1 ? kvb[d] : ckv[i * kD + d]) * div_rn(e, s);
      }
      v = acc;
    }
    lat[d] = bf(v);  // latent.to(dtype) before the norm
  }
  __syncthreads();
  // ---- RMSNorm of the latent (wave 0, pinned order)
  if (t < 64) {
    float ss = 0.0f;
    for (int d = t; d < kD; d += 64) ss = ss + lat[d] * lat[d];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss = ss + __shfl_xor(ss, m, 64);
    if (t == 0) inv_s[0] = div_rn(1.0f, sqrt_rn(div_rn(ss, static_cast<float>(kD)) + br.eps));
  }
  __syncthreads();
  {
    const float inv = inv_s[0];
    for (int d = t; d < kD; d += 256) lat[d] = bf(bf16_to_f32(br.norm_w[d]) * bf(lat[d] * inv));
  }
  __syncthreads();

  // ---- the main cache entry: FP8-b128 nope blocks + rotated bf16 rope channels
  const uint16_t* tg = p.tab + gp * 2 * kRopePairs;
  uint8_t* ent = br.cache + (b * br.cache_batch + g) * kEntryBytes;
  if (t < kNope / 4) {
    float v[4] = {lat[4 * t], lat[4 * t + 1], lat[4 * t + 2], lat[4 * t + 3]};
    float amax = abs_max4(v);
    amax = wave_max_group(amax, 32);
    const float sc = fp8_scale_from_amax(amax);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) word |= static_cast<uint32_t>(e4m3_encode(clampf(div_rn(v[i], sc), 448.0f))) << (8 * i);
    reinterpret_cast<uint32_t*>(ent)[t] = word;
    if ((t & 31) == 0) reinterpret_cast<float*>(ent + kNope)[t >> 5] = sc;
  } else if (t < kNope / 4 + kRopePairs) {
    const int i = t - kNope / 4;
    float e = lat[kNope + 2 * i], o = lat[kNope + 2 * i + 1];
    rope_pair(e, o, bf16_to_f32(tg[i]), bf16_to_f32(tg[kRopePairs + i]));
    uint16_t* rp = reinterpret_cast<uint16_t*>(ent + kNope + 4 * (kNope / 128));
    rp[2 * i] = f32_to_bf16(e);
    rp[2 * i + 1] = f32_to_bf16(o);
  }
  if (br.wk == nullptr) return;

  // ---- the index key: k = bf16(latent . wk^T), pinned halves
  {
    const int o = t & (kDi - 1);
    const int h = t >> 7;  // 256 threads: two halves of D per output
    const uint16_t* wrow = br.wk + static_cast<int64_t>(o) * kD + h * kHalf;
    float acc = 0.0f;
#pragma unroll 4
    for (int c = 0; c < kHalf / 8; ++c) {
      const uint4 w8 = reinterpret_cast<const uint4*>(wrow)[c];
      const uint32_t ws[4] = {w8.x, w8.y, w8.z, w8.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = h * kHalf + 8 * c + 2 * j;
        acc = acc + lat[i] * __uint_as_float(ws[j] << 16);
        acc = acc + lat[i + 1] * __uint_as_float(ws[j] & 0xffff0000u);
      }
    }
    part[h][o] = acc;
  }
  __syncthreads();
  if (t < kDi) kvec[t] = bf(part[0][t] + part[1][t]);
  __syncthreads();
  if (t < 64) {  // k_norm: lane l sums channels l, l + 64
    float ss = 0.0f;
    ss = ss + kvec[t] * kvec[t];
    ss = ss + kvec[t + 64] * kvec[t + 64];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss = ss + __shfl_xor(ss, m, 64);
    if (t == 0) inv_s[1] = div_rn(1.0f, sqrt_rn(div_rn(ss, static_cast<float>(kDi)) + br.k_eps));
  }
  __syncthreads();
  if (t < kDi) kvec[t] = bf(bf16_to_f32(br.kn_w[t]) * bf(kvec[t] * inv_s[1]));
  __syncthreads();
  if (t < kRopePairs) {  // RoPE of channels 64..127
    float e = kvec[kDi - 2 * kRopePairs + 2 * t], o = kvec[kDi - 2 * kRopePairs + 2 * t + 1];
    rope_pair(e, o, bf16_to_f32(tg[t]), bf16_to_f32(tg[kRopePairs + t]));
    kvec[kDi - 2 * kRopePairs + 2 * t] = e;
    kvec[kDi - 2 * kRopePairs + 2 * t + 1] = o;
  }
  __syncthreads();
  if (t < kDi / 4) {  // wave 0, lanes 0..31: four channels each
    float v[4] = {kvec[4 * t], kvec[4 * t + 1], kvec[4 * t + 2], kvec[4 * t + 3]};
    float amax = abs_max4(v);
    const int64_t key = b * br.key_batch + g;
    if (br.key_fmt == 0) {
      amax = wave_max_group(amax, 32);
      const float sc = fp8_scale_from_amax(amax);
      uint32_t word = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) word |= static_cast<uint32_t>(e4m3_encode(clampf(div_rn(v[i], sc), 448.0f))) << (8 * i);
      reinterpret_cast<uint32_t*>(br.k_codes + key * kDi)[t] = word;
      if (t == 0) static_cast<float*>(br.k_scales)[key] = sc;
    } else {
      amax = wave_max_group(amax, 8);
      const float sc = fp4_scale_from_amax(amax, false);
      uint32_t c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = e2m1_code(clampf(div_rn(v[i], sc), 6.0f));
      reinterpret_cast<uint16_t*>(br.k_codes + key * (kDi / 2))[t] =
          static_cast<uint16_t>(c[0] | (c[1] << 4) | (c[2] << 8) | (c[3] << 12));
      if ((t & 7) == 0) static_cast<uint8_t*>(br.k_scales)[key * (kDi / 32) + (t >> 3)] =
          static_cast<uint8_t>(__float_as_uint(sc) >> 23);
    }
  }
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_decode_emit(const int64_t* positions, int64_t B, const float* kv, const float* gate,
                               float* carry_kv, float* carry_gate, int ratio, const void* norm_weight, float eps,
                               uint8_t* cache, int64_t cache_batch_entries, int64_t cache_cap, const void* wk,
                               const void* k_norm_weight, float k_eps, int key_format, uint8_t* k_codes,
                               void* k_scales, int64_t key_batch_entries, const void* rope_table, int64_t table_rows,
                               void* step_cos, void* step_sin, void* stream) {
  MZK_CHECK_ARG(B >= 0 && B <= 0x7fffffff, "decode_emit: bad B");
  MZK_CHECK_ARG(ratio >= 1 && ratio <= 1024, "decode_emit: ratio %d not in [1, 1024]", ratio);
  if (B == 0) return MZK_OK;
  MZK_CHECK_ARG(positions && kv && carry_kv && norm_weight && cache && rope_table && (ratio == 1 || (gate && carry_gate)),
                "decode_emit: null pointer");
  MZK_CHECK_ARG(table_rows >= 1, "decode_emit: empty RoPE table");
  MZK_CHECK_ARG((step_cos == nullptr) == (step_sin == nullptr), "decode_emit: step cos and sin go together");
  MZK_CHECK_ARG(aligned16(cache) && cache_cap >= 0 && cache_batch_entries >= cache_cap,
                "decode_emit: the cache must be 16-byte aligned with cache_batch_entries >= cache_cap");
  EmitParams p{};
  EmitBranch& br = p.br;
  br.kv = kv;
  br.gate = gate;
  br.carry_kv = carry_kv;
  br.carry_gate = carry_gate;
  br.ratio = ratio;
  br.norm_w = static_cast<const uint16_t*>(norm_weight);
  br.eps = eps;
  br.cache = cache;
  br.cache_batch = cache_batch_entries;
  br.cache_cap = cache_cap;
  br.wk = nullptr;
  if (wk) {
    MZK_CHECK_ARG(k_norm_weight && k_codes && k_scales && (key_format == 0 || key_format == 1),
                  "decode_emit: the index key needs k_norm_weight, k_codes, k_scales and key_format 0 / 1");
    MZK_CHECK_ARG(aligned16(wk) && aligned16(k_codes) && key_batch_entries >= cache_cap,
                  "decode_emit: wk and k_codes 16-byte aligned, key_batch_entries >= cache_cap");
    br.wk = static_cast<const uint16_t*>(wk);
    br.kn_w = static_cast<const uint16_t*>(k_norm_weight);
    br.k_eps = k_eps;
    br.key_fmt = key_format;
    br.k_codes = k_codes;
    br.k_scales = k_scales;
    br.key_batch = key_batch_entries;
  }
  p.positions = positions;
  p.tab = static_cast<const uint16_t*>(rope_table);
  p.tab_rows = table_rows;
  p.step_cos = static_cast<uint16_t*>(step_cos);
  p.step_sin = static_cast<uint16_t*>(step_sin);
  emit_kernel<<<static_cast<unsigned>(B), 256, 0, as_stream(stream)>>>(p);
  MZK_LAUNCH_CHECK("decode_emit");
  return MZK_OK;
}

// Piece 3: lightning-indexer scores on MFMA.
//
//   score[row, g] = Di^-0.5 * sum_h w[row,h] * relu(q[row,h,:] . k[b,g,:])     (g <  vis)
//                 = -inf                                                       (g >= vis)
//   vis = min(G, (pos[row] + 1) // ratio)
// -- src/mzoo/archs/owlet1/indexer.py:124-143, layers/attn/golden_ref.py:213-227,
//    layers/attn/indexer/fwd.py:48-132.  `w` arrives already multiplied by Hi^-0.5.
//
// Operand formats (FMT):
//   kFp8  : e4m3 codes + one power-of-two fp32 scale per q head row and per key
//           (FP8 b128 at Di=128, the SGLang/DeepSeek V3.2 indexer layout).  Because the
//           scales are positive, relu(sq*sk*dot) = sq*sk*relu(dot): the MFMA runs on raw
//           codes and sq folds into the head weight, sk into the per-key epilogue.
//   kMxfp4: e2m1 nibbles + one e8m0 scale per 32 channels; the block scales go straight
//           into v_mfma_scale_f32_32x32x64_f8f6f4 (lane = one 32-element block).
//   kBf16 : bf16 q/k (the reference kernel-level `indexer.fwd` contract).
//
// Tiling (one workgroup = 4 waves = one query row x 4*kNkb*32 keys):
//   MFMA 32x32: M = 32 heads, N = 32 keys, K = Di.  A (queries) stays in VGPRs for the
//   whole workgroup; each wave streams kNkb 32-key tiles of B straight from HBM.
//   The 32x32 f32 result holds, in lane l, key column l%32 and 16 head rows, so the
//   ReLU-weighted head sum is lane-local, then one xor-32 shuffle adds the other half.
//   For each operand a lane holds a contiguous run of channels; A and B use the same
//   lane/slot -> channel assignment, so the K-order inside the MFMA is irrelevant.
#include "common.h"

namespace mzk {
namespace {

enum { kFp8 = 0, kMxfp4 = 1, kBf16 = 2 };

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kWaves = 4;
constexpr int kNkb = 4;                          // 32-key tiles per wave
constexpr int kKeysPerWg = kWaves * kNkb * 32;   // 512

// channels consumed by one MFMA step, per format
template <int FMT> struct Step;
template <> struct Step<kFp8> { static constexpr int K = 64; };     // 32x32x64, 32 B per lane
template <> struct Step<kMxfp4> { static constexpr int K = 64; };   // 32x32x64, 16 B per lane
template <> struct Step<kBf16> { static constexpr int K = 16; };    // 32x32x16, 16 B per lane

// bytes of one row (Di channels) in the operand storage
template <int FMT> __host__ __device__ constexpr int row_bytes(int di) {
  return FMT == kFp8 ? di : (FMT == kMxfp4 ? di / 2 : 2 * di);
}

struct Frag {
  v8i v;
  int scale;  // e8m0 byte (kMxfp4 only)
};

// Load the operand fragment of step `st` for a row `r` of length Di.  Lane half `hi`
// (lane / 32) selects which half of the step's channels the lane carries.
template <int FMT, int DI>
__device__ __forceinline__ Frag load_frag(const uint8_t* __restrict__ rowp, const uint8_t* __restrict__ e8m0row,
                                          int st, int hi, bool valid) {
  Frag f;
  f.v = v8i{0, 0, 0, 0, 0, 0, 0, 0};
  f.scale = 127;
  if (!valid) return f;
  if constexpr (FMT == kFp8) {
    const uint4* p = reinterpret_cast<const uint4*>(rowp + st * 64 + hi * 32);
    const uint4 a = p[0], b = p[1];
    f.v = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
  } else if constexpr (FMT == kMxfp4) {
    const uint4 a = *reinterpret_cast<const uint4*>(rowp + st * 32 + hi * 16);
    f.v = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    f.scale = e8m0row[st * 2 + hi];
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(rowp + st * 32 + hi * 16);
    f.v = v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  }
  return f;
}

template <int FMT>
__device__ __forceinline__ v16f mma(const Frag& a, const Frag& b, v16f c) {
  if constexpr (FMT == kFp8) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a.v, b.v, c, 0, 0, 0, 127, 0, 127);
  } else if constexpr (FMT == kMxfp4) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a.v, b.v, c, 4, 4, 0, a.scale, 0, b.scale);
  } else {
    const v8bf av = __builtin_bit_cast(v8bf, v4i{a.v[0], a.v[1], a.v[2], a.v[3]});
    const v8bf bv = __builtin_bit_cast(v8bf, v4i{b.v[0], b.v[1], b.v[2], b.v[3]});
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
  }
}

// head row held by value j of a 32x32 f32 accumulator in lane l (of m-block mb)
__device__ __forceinline__ int acc_row(int j, int lane) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }

template <int FMT, int DI, int MB>
__global__ void __launch_bounds__(kWaves * 64)
indexer_scores_kernel(const uint8_t* __restrict__ q, const float* __restrict__ q_scale, const uint8_t* __restrict__ q_e8m0,
                      const float* __restrict__ w, const uint8_t* __restrict__ k, const float* __restrict__ k_scale,
                      const uint8_t* __restrict__ k_e8m0, int64_t S, int Hi, int64_t G, int64_t k_batch_stride,
                      const int64_t* __restrict__ positions, int ratio, float* __restrict__ scores, int64_t score_stride) {
  constexpr int NST = DI / Step<FMT>::K;
  constexpr int RB = row_bytes<FMT>(DI);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hi = lane >> 5;
  const int64_t row = blockIdx.y;
  const int64_t b = row / S;
  const int64_t pos = positions ? positions[row] : row % S;
  int64_t vis = (pos + 1) / ratio;
  if (vis > G) vis = G;
  if (vis < 0) vis = 0;
  const float inv_sqrt_di = 1.0f / sqrt_rn(static_cast<float>(DI));

  const uint8_t* kb_base = k + b * k_batch_stride * RB;
  const float* ks_base = FMT == kFp8 ? k_scale + b * k_batch_stride : nullptr;
  const uint8_t* ke_base = FMT == kMxfp4 ? k_e8m0 + b * k_batch_stride * (DI / 32) : nullptr;
  float* out = scores + row * score_stride;

  const int64_t wave_key0 = static_cast<int64_t>(blockIdx.x) * kKeysPerWg + wave * (kNkb * 32);
  // all key fragments of the wave's tiles are requested first -- before the query rows and
  // head weights, and without waiting for the row's position -- so the workgroup pays one
  // HBM round trip instead of three dependent ones (keys below G are always readable;
  // invisible ones are masked at the end)
  Frag bf[kNkb][NST];
  float ksv[kNkb];  // FP8: the per-key scales
#pragma unroll
  for (int t = 0; t < kNkb; ++t) {
    const int64_t g0 = wave_key0 + t * 32;
    const int64_t g = g0 + (lane & 31);
    const bool kv = g < G;
    const uint8_t* krow = kb_base + (kv ? g : 0) * RB;
    const uint8_t* kerow = FMT == kMxfp4 ? ke_base + (kv ? g : 0) * (DI / 32) : nullptr;
#pragma unroll
    for (int st = 0; st < NST; ++st) bf[t][st] = load_frag<FMT, DI>(krow, kerow, st, hi, kv);
    ksv[t] = (FMT == kFp8 && kv) ? ks_base[g] : 1.0f;
  }
  // per-head coefficients w (x the FP8 query scale): one lane per head, through LDS, so
  // a lane issues one load instead of one per accumulator row it needs
  __shared__ float coef_s[64];
  if (wave == 0) {
    float c = 0.0f;
    if (lane < Hi) {
      c = w[row * Hi + lane];
      if constexpr (FMT == kFp8) c = c * q_scale[row * Hi + lane];
    }
    coef_s[lane] = c;
  }
  // A fragments (queries), resident for the whole workgroup
  Frag a[MB][NST];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int h = mb * 32 + (lane & 31);
    const bool hv = h < Hi;
    const uint8_t* qrow = q + (row * Hi + (hv ? h : 0)) * static_cast<int64_t>(RB);
    const uint8_t* erow = FMT == kMxfp4 ? q_e8m0 + (row * Hi + (hv ? h : 0)) * (DI / 32) : nullptr;
#pragma unroll
    for (int st = 0; st < NST; ++st) a[mb][st] = load_frag<FMT, DI>(qrow, erow, st, hi, hv);
  }
  __syncthreads();
  float coef[MB][16];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 16; ++j) coef[mb][j] = coef_s[mb * 32 + acc_row(j, lane)];

#pragma unroll
  for (int t = 0; t < kNkb; ++t) {
    const int64_t g0 = wave_key0 + t * 32;
    const int64_t g = g0 + (lane & 31);
    if (g0 >= G) break;
    if (g0 >= vis) {  // nothing in this tile is visible to the row
      if (lane < 32 && g < G) out[g] = -__builtin_huge_valf();
      continue;
    }
    float part = 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      v16f acc = {};
#pragma unroll
      for (int st = 0; st < NST; ++st) acc = mma<FMT>(a[mb][st], bf[t][st], acc);
#pragma unroll
      for (int j = 0; j < 16; ++j) part = part + coef[mb][j] * fmaxf(acc[j], 0.0f);
    }
    const float total = part + __shfl_xor(part, 32, 64);
    if (lane < 32 && g < G) {
      float s = total * inv_sqrt_di;
      if constexpr (FMT == kFp8) s = s * ksv[t];
      out[g] = (g < vis) ? s : -__builtin_huge_valf();
    }
  }
}

template <int FMT, int DI>
int launch_di(const uint8_t* q, const float* qs, const uint8_t* qe, const float* w, const uint8_t* k, const float* ks,
              const uint8_t* ke, int64_t rows, int64_t S, int Hi, int64_t G, int64_t kbs, const int64_t* pos, int ratio,
              float* scores, int64_t sstride, hipStream_t s) {
  dim3 grid(static_cast<unsigned>((G + kKeysPerWg - 1) / kKeysPerWg), static_cast<unsigned>(rows));
  if (Hi <= 32)
    indexer_scores_kernel<FMT, DI, 1><<<grid, kWaves * 64, 0, s>>>(q, qs, qe, w, k, ks, ke, S, Hi, G, kbs, pos, ratio,
                                                                  scores, sstride);
  else
    indexer_scores_kernel<FMT, DI, 2><<<grid, kWaves * 64, 0, s>>>(q, qs, qe, w, k, ks, ke, S, Hi, G, kbs, pos, ratio,
                                                                  scores, sstride);
  return MZK_OK;
}

template <int FMT>
int launch(const uint8_t* q, const float* qs, const uint8_t* qe, const float* w, const uint8_t* k, const float* ks,
           const uint8_t* ke, int64_t B, int64_t S, int Hi, int Di, int64_t G, int64_t kbs, const int64_t* pos, int ratio,
           float* scores, int64_t sstride, hipStream_t s) {
  const int64_t rows = B * S;
  switch (Di) {
    case 64: return launch_di<FMT, 64>(q, qs, qe, w, k, ks, ke, rows, S, Hi, G, kbs, pos, ratio, scores, sstride, s);
    case 128: return launch_di<FMT, 128>(q, qs, qe, w, k, ks, ke, rows, S, Hi, G, kbs, pos, ratio, scores, sstride, s);
    case 256: return launch_di<FMT, 256>(q, qs, qe, w, k, ks, ke, rows, S, Hi, G, kbs, pos, ratio, scores, sstride, s);
    default:
      if constexpr (FMT == kBf16) {
        if (Di == 96) return launch_di<FMT, 96>(q, qs, qe, w, k, ks, ke, rows, S, Hi, G, kbs, pos, ratio, scores, sstride, s);
        if (Di == 32) return launch_di<FMT, 32>(q, qs, qe, w, k, ks, ke, rows, S, Hi, G, kbs, pos, ratio, scores, sstride, s);
      }
      set_last_error("indexer_scores: unsupported index head dim %d", Di);
      return MZK_EUNSUPPORTED;
  }
}

int check_common(int64_t B, int64_t S, int Hi, int Di, int64_t G, int64_t kbs, int ratio, int64_t sstride) {
  MZK_CHECK_ARG(B >= 0 && S >= 0 && G >= 0, "indexer_scores: negative size");
  MZK_CHECK_ARG(Hi >= 1 && Hi <= 64, "indexer_scores: index heads must be in [1, 64] (got %d)", Hi);
  MZK_CHECK_ARG(ratio >= 1, "indexer_scores: compress_ratio must be >= 1 (got %d)", ratio);
  MZK_CHECK_ARG(kbs >= G && sstride >= G, "indexer_scores: key batch stride / score stride smaller than G");
  MZK_CHECK_ARG(B * S <= 0x7fffffff, "indexer_scores: too many query rows");
  (void)Di;
  return MZK_OK;
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_indexer_scores_fp8(const uint8_t* q_codes, const float* q_scales, const float* w, const uint8_t* k_codes,
                                      const float* k_scales, int64_t B, int64_t S, int Hi, int Di, int64_t G,
                                      int64_t k_batch_stride, const int64_t* positions, int ratio, float* scores,
                                      int64_t score_stride, void* stream) {
  int rc = check_common(B, S, Hi, Di, G, k_batch_stride, ratio, score_stride);
  if (rc) return rc;
  if (B * S == 0 || G == 0) return MZK_OK;
  MZK_CHECK_ARG(q_codes && q_scales && w && k_codes && k_scales && scores, "indexer_scores_fp8: null pointer");
  MZK_CHECK_ARG(Di % 64 == 0, "indexer_scores_fp8: Di must be a multiple of 64 (got %d)", Di);
  rc = launch<kFp8>(q_codes, q_scales, nullptr, w, k_codes, k_scales, nullptr, B, S, Hi, Di, G, k_batch_stride, positions,
                    ratio, scores, score_stride, as_stream(stream));
  if (rc) return rc;
  MZK_LAUNCH_CHECK("indexer_scores_fp8");
  return MZK_OK;
}

extern "C" int mzk_indexer_scores_mxfp4(const uint8_t* q_packed, const uint8_t* q_e8m0, const float* w,
                                        const uint8_t* k_packed, const uint8_t* k_e8m0, int64_t B, int64_t S, int Hi,
                                        int Di, int64_t G, int64_t k_batch_stride, const int64_t* positions, int ratio,
                                        float* scores, int64_t score_stride, void* stream) {
  int rc = check_common(B, S, Hi, Di, G, k_batch_stride, ratio, score_stride);
  if (rc) return rc;
  if (B * S == 0 || G == 0) return MZK_OK;
  MZK_CHECK_ARG(q_packed && q_e8m0 && w && k_packed && k_e8m0 && scores, "indexer_scores_mxfp4: null pointer");
  MZK_CHECK_ARG(Di % 64 == 0, "indexer_scores_mxfp4: Di must be a multiple of 64 (got %d)", Di);
  rc = launch<kMxfp4>(q_packed, nullptr, q_e8m0, w, k_packed, nullptr, k_e8m0, B, S, Hi, Di, G, k_batch_stride,
                      positions, ratio, scores, score_stride, as_stream(stream));
  if (rc) return rc;
  MZK_LAUNCH_CHECK("indexer_scores_mxfp4");
  return MZK_OK;
}

extern "C" int mzk_indexer_scores_bf16(const void* q, const float* w, const void* k, int64_t B, int64_t S, int Hi, int Di,
                                       int64_t G, int64_t k_batch_stride, const int64_t* positions, int ratio,
                                       float* scores, int64_t score_stride, void* stream) {
  int rc = check_common(B, S, Hi, Di, G, k_batch_stride, ratio, score_stride);
  if (rc) return rc;
  if (B * S == 0 || G == 0) return MZK_OK;
  MZK_CHECK_ARG(q && w && k && scores, "indexer_scores_bf16: null pointer");
  rc = launch<kBf16>(static_cast<const uint8_t*>(q), nullptr, nullptr, w, static_cast<const uint8_t*>(k), nullptr, nullptr,
                     B, S, Hi, Di, G, k_batch_stride, positions, ratio, scores, score_stride, as_stream(stream));
  if (rc) return rc;
  MZK_LAUNCH_CHECK("indexer_scores_bf16");
  return MZK_OK;
}

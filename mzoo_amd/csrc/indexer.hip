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
// Tiling (one workgroup = 4 waves = one query row x 4*NKB*32 keys, NKB = kNkb = 4 tiles
// per wave, 5 in the merged emission launch):
//   MFMA 32x32: M = 32 heads, N = 32 keys, K = Di.  A (queries) stays in VGPRs for the
//   whole workgroup; each wave streams NKB 32-key tiles of B straight from HBM.
//   The 32x32 f32 result holds, in lane l, key column l%32 and 16 head rows, so the
//   ReLU-weighted head sum is lane-local, then one xor-32 shuffle adds the other half.
//   For each operand a lane holds a contiguous run of channels; A and B use the same
//   lane/slot -> channel assignment, so the K-order inside the MFMA is irrelevant.
#include "common.h"
#include "emit_core.h"

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

// Load the operand fragment of step `st` from a (valid) row of length Di.  Lane half `hi`
// (lane / 32) selects which half of the step's channels the lane carries.  No branch: the
// callers clamp out-of-range rows to a readable one, so every load is issued on every lane
// and the in-order wait counts stay exact.
template <int FMT, int DI>
__device__ __forceinline__ Frag load_frag(const uint8_t* __restrict__ rowp, const uint8_t* __restrict__ e8m0row,
                                          int st, int hi) {
  Frag f;
  f.scale = 127;
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

// The zero fragment in place of `f` where `keep` is false (rows beyond the operand).
__device__ __forceinline__ Frag keep_or_zero(Frag f, bool keep) {
#pragma unroll
  for (int i = 0; i < 8; ++i) f.v[i] = keep ? f.v[i] : 0;
  f.scale = keep ? f.scale : 127;
  return f;
}

// One term of the ReLU-weighted head sum: part + c * max(x, 0), as one fused multiply-add.
// max(x, 0) is an integer max on the bits (a negative float's bit pattern is a negative
// integer, so it becomes +0; a positive one is kept): one instruction, where fmaxf also
// canonicalizes its operand.
__device__ __forceinline__ float relu_fma(float c, float x, float part) {
  const float r = __int_as_float(__builtin_elementwise_max(__float_as_int(x), 0));
  return __builtin_fmaf(c, r, part);
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

struct IdxParams {
  const uint8_t* q;  // quantized / bf16 query operand [rows, Hi, row_bytes]
  const float* q_scale;
  const uint8_t* q_e8m0;
  const float* w;
  const uint8_t* k;
  const float* k_scale;
  const uint8_t* k_e8m0;
  int64_t S;
  int Hi;
  int64_t G, kbs;
  const int64_t* positions;
  int ratio;
  float* scores;
  int64_t sstride;
  // fused decode prologue (Di = 128): the bf16 query is quantized in the kernel (FP8 b128
  // or MXFP4), and workgroup 0 of each row stores the codes / scales and appends the new
  // latent
  const uint16_t* q_raw;  // [rows, Hi, 128] bf16
  uint8_t* q_codes_out;   // FP8: [rows, Hi, 128] e4m3; MXFP4: [rows, Hi, 64] e2m1 pairs; or null
  float* q_scales_out;    // FP8: [rows, Hi], or null
  uint8_t* q_e8m0_out;    // MXFP4: [rows, Hi, 4], or null
  const uint16_t* kv;     // [rows, nope + rope] bf16 (APPEND: rotated; FUSE: the kv projection)
  int nope, rope;
  uint8_t* win;
  int64_t win_batch_entries;
  int win_cap;
  // FUSE (Di = 128, latent 512 + 64): the query's trailing q_rope_dim channels are rotated
  // with q_cos / q_sin [rows, q_rope_dim / 2] bf16 before quantization, and one extra
  // workgroup per row normalizes kv (RMSNorm, weight kv_w [576] bf16, kv_eps), rotates its
  // rope slice with kv_cos / kv_sin [rows, 32] bf16 and appends the FP8-b128 entry
  const uint16_t* q_cos;
  const uint16_t* q_sin;
  int q_rope_dim;
  const uint16_t* kv_w;
  float kv_eps;
  const uint16_t* kv_cos;
  const uint16_t* kv_sin;
  // GATHER (level two of the two-level selection): the score axis is the row's candidate
  // slots j < cand_nb * cand_bs; slot j is key cand[row][j / cand_bs] * cand_bs + j % cand_bs
  // (a block index < 0 or a key >= G is empty: -inf)
  const int32_t* cand;
  int64_t cand_stride;
  int cand_nb, cand_bs;
  int64_t cand_keys;  // keys per batch row (the slots' key range)
  // EMIT: the grid is one-dimensional, rows x lead workgroups, then rows x scoring workgroups
  int64_t rows;
};

constexpr int kFuseNope = 512, kFuseRope = 64, kFuseChunks = (kFuseNope + kFuseRope) / 64;

// The fused kv prologue (owlet1/attention.py:150-154 with the 656-byte window entry), done
// by wave 0 of each row's first workgroup: lane l holds channels l + 64 i.  Its loads are
// issued between the query's and the keys', and the work runs once the query is quantized,
// while the key loads are in flight.
//   RMSNorm (norm_rope.py:25-30): sum of squares in 64 partials (lane l over its channels in
//   order) combined by the xor butterfly 32 .. 1, var = sum / 576, inv = 1 / sqrt(var + eps),
//   y = bf16(w * bf16(h * inv));
//   RoPE of channels 512 .. 575 (pairs (2j, 2j+1) = lanes 2j, 2j+1 of chunk 8) at the row's
//   cos / sin;
//   pack: FP8 e4m3 codes of the 4 nope blocks of 128 with their power-of-two scales, then the
//   rotated rope slice in bf16, into ring slot b * win_batch_entries + pos % win_cap.
typedef unsigned short mzk_u16x2 __attribute__((ext_vector_type(2)));

struct FusedKv {
  // two 16-bit values per register (d16 / d16_hi loads): kv and weight channels
  // lane + 64 i, i = 0 .. 8, then cos / sin of the lane's rope pair
  static constexpr int kRegs = (2 * kFuseChunks + 2 + 1) / 2;
  mzk_u16x2 v[kRegs];

  __device__ __forceinline__ void load(const IdxParams& p, int64_t row, int lane) {
    const uint16_t* kvrow = p.kv + row * (kFuseNope + kFuseRope);
#pragma unroll
    for (int i = 0; i < kFuseChunks; ++i) {
      v[i / 2][i & 1] = kvrow[lane + 64 * i];
      v[(kFuseChunks + i) / 2][(kFuseChunks + i) & 1] = p.kv_w[lane + 64 * i];
    }
    v[kFuseChunks][0] = p.kv_cos[row * (kFuseRope / 2) + (lane >> 1)];
    v[kFuseChunks][1] = p.kv_sin[row * (kFuseRope / 2) + (lane >> 1)];
  }
  __device__ __forceinline__ uint16_t at(int k) const { return v[k / 2][k & 1]; }

  __device__ __forceinline__ void append(const IdxParams& p, int64_t b, int64_t pos, int lane) const {
    if (pos < 0) return;  // no ring slot for a negative position
    float h[kFuseChunks];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kFuseChunks; ++i) {
      h[i] = bf16_to_f32(at(i));
      ss = ss + h[i] * h[i];
    }
    // p[l] + p[l ^ m] for m = 32 .. 1: every lane ends with the same total
    ss = ss + lane_xor<32>(ss);
    ss = ss + lane_xor<16>(ss);
    ss = ss + lane_xor<8>(ss);
    ss = ss + lane_xor<4>(ss);
    ss = ss + lane_xor<2>(ss);
    ss = ss + lane_xor<1>(ss);
    const float var = div_rn(ss, static_cast<float>(kFuseNope + kFuseRope));
    const float inv = div_rn(1.0f, sqrt_rn(var + p.kv_eps));
    float y[kFuseChunks];
#pragma unroll
    for (int i = 0; i < kFuseChunks; ++i)
      y[i] = bf16_to_f32(f32_to_bf16(bf16_to_f32(at(kFuseChunks + i)) * bf16_to_f32(f32_to_bf16(h[i] * inv))));
    // rope slice: lane 2j holds the even channel of pair j, lane 2j+1 the odd one
    const float cf = bf16_to_f32(at(2 * kFuseChunks)), sf = bf16_to_f32(at(2 * kFuseChunks + 1));
    const float partner = lane_xor<1>(y[kFuseChunks - 1]);
    const bool odd = lane & 1;
    const float e = odd ? partner : y[kFuseChunks - 1];
    const float o = odd ? y[kFuseChunks - 1] : partner;
    const uint16_t rot = f32_to_bf16(odd ? e * sf + o * cf : e * cf - o * sf);
    uint8_t* ent =
        p.win + (b * p.win_batch_entries + pos % p.win_cap) * (kFuseNope + 4 * (kFuseNope / 128) + 2 * kFuseRope);
    static_assert(kFuseNope / 128 == 4, "four nope blocks");
    float scs[4], invs[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      scs[k] = fp8_scale_from_amax(wave_max_nonneg(nn_max(fabsf(y[2 * k]), fabsf(y[2 * k + 1]))));
      // x / sc == x * (1 / sc) exactly: sc is a power of two in [2^-22, 2^127]
      invs[k] = 1.0f / scs[k];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // v_cvt_pk_fp8_f32 is the quantizer's e4m3 encoder for |x| <= 448
      const int code = __builtin_amdgcn_cvt_pk_fp8_f32(clampf(y[i] * invs[i >> 1], 448.0f), 0.0f, 0, false);
      ent[lane + 64 * i] = static_cast<uint8_t>(code & 0xff);
    }
    if (lane < 4) reinterpret_cast<float*>(ent + kFuseNope)[lane] =
        lane == 0 ? scs[0] : lane == 1 ? scs[1] : lane == 2 ? scs[2] : scs[3];
    reinterpret_cast<uint16_t*>(ent + kFuseNope + 4 * (kFuseNope / 128))[lane] = rot;
  }
};

// LDS bytes per quantized head row (padding spreads banks)
template <int FMT>
constexpr int q_pitch() { return FMT == kFp8 ? 128 + 16 : 64 + 16; }

// The raw query's quantization (QRAW): thread t holds 32 channels of head t / 4 (bf16, already
// rotated) in qr; they are quantized into LDS (FP8 b128 per head, or MXFP4 per 32 channels),
// then every lane reads back its A fragments and, FP8, its head's scale into cq.  Thread t
// owns head qh = t / 4, channels 32 qc .. 32 qc + 31 (qc = t % 4).
//   amax: the magnitudes' bf16 bits compared as integers (two per word, v_pk_max_u16) -- the
//   float order of values >= 0 with NaN above infinity, as nn_max;
//   FP8: codes of clamp(x / s, +-448) by v_cvt_pk_fp8_f32 (s a power of two, x / s == x *
//   (1 / s) exactly); with a finite amax every x * (1 / s) is finite and the clamp is a
//   median, else the NaN-keeping clamp;
//   MXFP4: with a finite amax, v_cvt_scalef32_pk_fp4_bf16 (x / s to e2m1, nearest even,
//   saturating at 6), which equals e2m1_code(clamp(x * (1 / s), +-6)) for every finite bf16 x
//   and power-of-two s in [2^-126, 2^127] (checked on the hardware for all bf16 inputs); a
//   block with a NaN or an infinity takes the software encoder.
typedef unsigned short mzk_u16x2v __attribute__((ext_vector_type(2)));
typedef __bf16 mzk_bf16x2v __attribute__((ext_vector_type(2)));

// The MFMA A fragments of the query codes quantize_query left in LDS, and (FP8) the lane's
// head scale.
template <int FMT, int DI, int MB>
__device__ __forceinline__ void query_frags(int lane, int hi, int hl, const uint8_t* q_lds, const float* qs_lds,
                                            const uint8_t* qe_lds, Frag (&a)[MB][DI / Step<FMT>::K], float& cq) {
  constexpr int QP = q_pitch<FMT>();
  constexpr int NST = DI / Step<FMT>::K;
  if constexpr (FMT == kMxfp4) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int h = mb * 32 + (lane & 31);
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const uint4 u = *reinterpret_cast<const uint4*>(q_lds + h * QP + st * 32 + hi * 16);
        a[mb][st].v = v8i{(int)u.x, (int)u.y, (int)u.z, (int)u.w, 0, 0, 0, 0};
        a[mb][st].scale = qe_lds[h * 4 + st * 2 + hi];
      }
    }
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint4* src = reinterpret_cast<const uint4*>(q_lds + (mb * 32 + (lane & 31)) * QP);
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const uint4 u = src[4 * st + 2 * hi], v = src[4 * st + 2 * hi + 1];
        a[mb][st].v = v8i{(int)u.x, (int)u.y, (int)u.z, (int)u.w, (int)v.x, (int)v.y, (int)v.z, (int)v.w};
        a[mb][st].scale = 127;
      }
    }
    cq = qs_lds[hl];
  }
}

// READ false: the codes (and scales) into LDS and the barrier only; query_frags reads them.
template <int FMT, int DI, int MB, bool READ = true>
__device__ __forceinline__ void quantize_query(const uint4 (&qr)[4], int qh, int qc, int Hi, int lane, int hi, int hl,
                                               uint8_t* q_lds, float* qs_lds, uint8_t* qe_lds,
                                               Frag (&a)[MB][DI / Step<FMT>::K], float& cq) {
  constexpr int QP = q_pitch<FMT>();
  constexpr int NST = DI / Step<FMT>::K;
  // the thread's channels, two bf16 per word (the even channel low); heads beyond Hi are zeros
  uint32_t wv[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wv[4 * i] = qr[i].x;
    wv[4 * i + 1] = qr[i].y;
    wv[4 * i + 2] = qr[i].z;
    wv[4 * i + 3] = qr[i].w;
  }
  if (qh >= Hi) {
#pragma unroll
    for (int k = 0; k < 16; ++k) wv[k] = 0u;
  }
  mzk_u16x2v m = __builtin_bit_cast(mzk_u16x2v, wv[0] & 0x7fff7fffu);
#pragma unroll
  for (int k = 1; k < 16; ++k) m = __builtin_elementwise_max(m, __builtin_bit_cast(mzk_u16x2v, wv[k] & 0x7fff7fffu));
  float amax = __uint_as_float(static_cast<uint32_t>(m.x > m.y ? m.x : m.y) << 16);
  if constexpr (FMT == kMxfp4) {
    // one MXFP4 block of 32 channels per thread: scale, then e2m1 codes (element 2i in the
    // low nibble of byte i), as the quantizer's packed form
    const float sc = fp4_scale_from_amax(amax, false);
    uint32_t wd[4];
    if (amax <= 0x1.fffffep127f) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t word = 0;
        word = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(word, __builtin_bit_cast(mzk_bf16x2v, wv[4 * i]), sc, 0);
        word = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(word, __builtin_bit_cast(mzk_bf16x2v, wv[4 * i + 1]), sc, 1);
        word = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(word, __builtin_bit_cast(mzk_bf16x2v, wv[4 * i + 2]), sc, 2);
        word = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(word, __builtin_bit_cast(mzk_bf16x2v, wv[4 * i + 3]), sc, 3);
        wd[i] = word;
      }
    } else {
      // x / sc == x * (1 / sc) exactly: sc is a power of two (here infinite: 1 / sc = 0)
      const float inv = 1.0f / sc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = __uint_as_float(wv[4 * i + j] << 16);
          const float hi2 = __uint_as_float(wv[4 * i + j] & 0xffff0000u);
          word |= e2m1_code(clampf(lo * inv, 6.0f)) << (8 * j);
          word |= e2m1_code(clampf(hi2 * inv, 6.0f)) << (8 * j + 4);
        }
        wd[i] = word;
      }
    }
    *reinterpret_cast<uint4*>(q_lds + qh * QP + 16 * qc) = uint4{wd[0], wd[1], wd[2], wd[3]};
    qe_lds[qh * 4 + qc] = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
    __syncthreads();
    if constexpr (READ) query_frags<FMT, DI, MB>(lane, hi, hl, q_lds, qs_lds, qe_lds, a, cq);
  } else {
    amax = group_max(amax, 4);  // the 4 threads of a head are consecutive lanes
    const float sc = fp8_scale_from_amax(amax);
    // x / sc == x * (1 / sc) exactly: sc is a power of two, in [2^-22, 2^120] for finite input
    const float inv = sc <= 0x1p120f ? pow2_reciprocal(sc) : 1.0f / sc;
    uint32_t wd[8];
    if (amax <= 0x1.fffffep127f) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x[4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          x[2 * j] = __builtin_amdgcn_fmed3f(__uint_as_float(wv[2 * i + j] << 16) * inv, -448.0f, 448.0f);
          x[2 * j + 1] = __builtin_amdgcn_fmed3f(__uint_as_float(wv[2 * i + j] & 0xffff0000u) * inv, -448.0f, 448.0f);
        }
        const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
        wd[i] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], lo, true));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x[4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          x[2 * j] = clampf(__uint_as_float(wv[2 * i + j] << 16) * inv, 448.0f);
          x[2 * j + 1] = clampf(__uint_as_float(wv[2 * i + j] & 0xffff0000u) * inv, 448.0f);
        }
        const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
        wd[i] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], lo, true));
      }
    }
    uint4* dst = reinterpret_cast<uint4*>(q_lds + qh * QP + 32 * qc);
    dst[0] = uint4{wd[0], wd[1], wd[2], wd[3]};
    dst[1] = uint4{wd[4], wd[5], wd[6], wd[7]};
    if (qc == 0) qs_lds[qh] = sc;
    __syncthreads();
    if constexpr (READ) query_frags<FMT, DI, MB>(lane, hi, hl, q_lds, qs_lds, qe_lds, a, cq);
  }
}

// ---- the merged emission + scores launch (EMIT) ------------------------------------------

// The emission branches of a merged launch: the fine one (ratio 4, with the index key and
// the kv prologue) and, with COARSE, a keyless coarse one (coarse_body's form).
struct EmitSet {
  EmitParams fine;
  EmitParams coarse;
};

// Loads through the constant address space: with a workgroup-uniform address they become
// scalar loads, which wait on their own counter and leave the in-order vector loads (and the
// waits the score loop counts on them) alone.  Only for data no launch of the step writes
// before this one ends (the positions, the position table).
typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;
typedef const __attribute__((address_space(4))) int64_t* const_i64_ptr;

// Row `pos` of the position table (clamped into it: the host refuses positions beyond the
// table) as 32 words: cos of pairs 0..31 (bf16, pair j in the low half of word j / 2 for even
// j) in words 0..15, sin in words 16..31; scalar loads.
__device__ __forceinline__ void load_table_row(const EmitParams& e, int64_t pos, uint32_t (&tw)[kRopePairs]) {
  const int64_t r = pos < 0 ? 0 : (pos >= e.tab_rows ? e.tab_rows - 1 : pos);
  const const_u32_ptr src = (const_u32_ptr)(e.tab + r * 2 * kRopePairs);
#pragma unroll
  for (int i = 0; i < kRopePairs; ++i) tw[i] = src[i];
}

// The merged launch's compress ratio (emit_row<kEmitRatio>).
constexpr int kEmitRatio = 4;

// The group whose index key the step at position pos emits (emit_row's condition), or -1.
__device__ __forceinline__ int64_t emitted_group(const EmitParams& e, int64_t pos) {
  if (pos < 0 || (pos + 1) % kEmitRatio != 0 || e.br.wk == nullptr) return -1;
  const int64_t g = (pos + 1) / kEmitRatio - 1;
  return (g < e.br.cache_cap && g * kEmitRatio < e.tab_rows) ? g : -1;
}

// RoPE of the query's trailing 64 channels (owlet1/indexer.py:126-128) with the table row's
// words: thread (head, qc) holds channels 32 qc .. 32 qc + 31, so qc = 2 rotates pairs 0..15
// and qc = 3 pairs 16..31 (pair j = channels 64 + 2j, 65 + 2j) -- the fused prologue's
// per-pair arithmetic (rope_pair_bf16).
__device__ __forceinline__ void rope_query_table(uint4 (&qr)[4], int qc, const uint32_t (&tw)[kRopePairs]) {
  if (qc < 2) return;
  const bool upper = qc == 3;
  uint32_t* wq = reinterpret_cast<uint32_t*>(qr);
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t cp = upper ? tw[8 + (k >> 1)] : tw[k >> 1];
    const uint32_t sp = upper ? tw[24 + (k >> 1)] : tw[16 + (k >> 1)];
    wq[k] = rope_pair_bf16(wq[k], __uint_as_float((k & 1) ? cp & 0xffff0000u : cp << 16),
                           __uint_as_float((k & 1) ? sp & 0xffff0000u : sp << 16));
  }
}

// Workgroup 0 of a row in the merged launch: the row's emission (emit_row), then, when the
// step emitted index key g (< G), that key's score.  The score is computed as a scoring
// workgroup computes it -- the same query quantization into the same A fragments, one 32x32
// MFMA tile whose 32 key columns all hold key g (its codes straight from LDS), the same
// ReLU-weighted head sum -- so its bits are those the separate emission + scores launches
// give.
template <int FMT, int MB>
__device__ __forceinline__ void emit_and_score(const IdxParams& p, const EmitParams& e, int64_t row) {
  constexpr int NST = kDi / Step<FMT>::K;
  __shared__ __align__(16) uint8_t key_lds[kDi + 16];
  __shared__ __align__(16) uint8_t q_lds[64 * q_pitch<FMT>()];
  __shared__ float qs_lds[FMT == kFp8 ? 64 : 1];
  __shared__ uint8_t qe_lds[FMT == kMxfp4 ? 256 : 4];
  const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5;
  const int qh = tid >> 2, qc = tid & 3;
  const int Hi = p.Hi;
  // the query, its head weight and the token's RoPE tables are requested before the
  // emission, so they have arrived when it ends
  const int64_t pos = *(const_i64_ptr)(e.positions + row);
  uint4 qr[4];
  const int hq = qh < Hi ? qh : Hi - 1;
  const uint4* src = reinterpret_cast<const uint4*>(p.q_raw + (row * Hi + hq) * kDi + 32 * qc);
#pragma unroll
  for (int i = 0; i < 4; ++i) qr[i] = src[i];
  const int hl = lane < Hi ? lane : Hi - 1;
  float cw = p.w[row * Hi + hl];
  uint32_t tw[kRopePairs];
  load_table_row(e, pos, tw);
  // the query is rotated and quantized into LDS first, while the emission's operands (the
  // key weights last) are still arriving; its fragments are read after the emission
  cw = lane < Hi ? cw : 0.0f;
  rope_query_table(qr, qc, tw);
  Frag a[MB][NST];
  float cq = 1.0f;
  quantize_query<FMT, kDi, MB, false>(qr, qh, qc, Hi, lane, hi, hl, q_lds, qs_lds, qe_lds, a, cq);
  if (!emit_row<kEmitRatio, true, 1>(e, row, key_lds)) return;  // uniform
  const int64_t g = (pos + 1) / kEmitRatio - 1;
  if (g >= p.G) return;  // uniform
  __syncthreads();  // the key bytes in key_lds
  if (tid >= 64) return;  // one wave scores the key
  query_frags<FMT, kDi, MB>(lane, hi, hl, q_lds, qs_lds, qe_lds, a, cq);
  const float cwq = cw * cq;
  float coef[MB][16];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 16; ++j) coef[mb][j] = __shfl(cwq, mb * 32 + acc_row(j, lane), 64);
  Frag bk[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) bk[st] = load_frag<FMT, kDi>(key_lds, key_lds + kDi / 2, st, hi);
  float part = 0.0f;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    v16f acc = {};
#pragma unroll
    for (int st = 0; st < NST; ++st) acc = mma<FMT>(a[mb][st], bk[st], acc);
#pragma unroll
    for (int j = 0; j < 16; ++j) part = relu_fma(coef[mb][j], acc[j], part);
  }
  const float total = part + __shfl_xor(part, 32, 64);
  float s = total * (1.0f / sqrt_rn(static_cast<float>(kDi)));
  if constexpr (FMT == kFp8) s = s * *reinterpret_cast<const float*>(key_lds + kDi);
  if (lane == 0) p.scores[row * p.sstride + g] = s;
}

// One workgroup = 4 waves = one query row x 4 * NKB * 32 keys (see the tiling note above).
// QRAW: the query arrives as bf16 [Hi, 128] and each workgroup quantizes it into LDS --
// thread t owns head t/4, channels 32(t%4)..+31 (quantize_query).  FP8 b128
// (owlet1/quant.py:72-86: one power-of-two scale per head) uses v_cvt_pk_fp8_f32, which
// equals the e4m3 encoder of the quantizer (round to nearest even, subnormals kept) for
// every |x| <= 448.  MXFP4 (quant.py:49-66 with block 32 and ue8m0 scales): a thread's 32
// channels are one scale block and exactly one lane's MFMA fragment (16 bytes of nibbles +
// the e8m0 byte).
// APPEND: workgroup 0 of the row also writes the new token's FP8-b128 latent into its
// window-ring slot (b * win_batch_entries + pos % win_cap).
// FUSE: the query is rotated before it is quantized, and wave 0 of each row's workgroup 0
// runs the kv prologue (FusedKv): loads before the keys', the work after the query's
// quantization.
// EMIT (with FUSE; one query row per batch row, ratio 4): the step's group emission joins
// the launch.  Per row, lead workgroup 0 runs the emission (emit_row: carry slot, step
// tables, and on a group step the group's entry and index key) and then scores the new key
// itself (emit_and_score), lead workgroup 1 writes the token's window entry (kv_prologue),
// and the scoring workgroups take the query's RoPE tables from row `pos` of the position
// table and leave the new key's score to lead workgroup 0.  The grid is one-dimensional:
// rows x lead workgroups, then rows x scoring workgroups; xw below is the workgroup's place
// in its row, leads first.
template <int FMT, int DI, int MB, bool QRAW, bool APPEND, bool FUSE = false, bool GATHER = false, bool EMIT = false,
          int NKB = kNkb, bool COARSE = false>
__global__ void __launch_bounds__(kWaves * 64) indexer_scores_kernel(const IdxParams p, const EmitSet es) {
  static_assert(!QRAW || ((FMT == kFp8 || FMT == kMxfp4) && DI == 128), "in-kernel quantization: Di = 128");
  static_assert(!FUSE || (QRAW && !APPEND), "the fused prologue quantizes the raw query and appends on its own");
  static_assert(!GATHER || !QRAW, "the candidate scorer takes the quantized query");
  static_assert(!EMIT || (FUSE && DI == kDi), "the merged emission takes the fused prologue's query, Di = 128");
  static_assert(!COARSE || EMIT, "the coarse branch joins the merged emission");
  const EmitParams& e = es.fine;
  // EMIT: workgroups before the scoring ones (emitter, window entry, coarse parts)
  constexpr int kLead = EMIT ? 2 + (COARSE ? kCoarseParts : 0) : 0;
  constexpr int QP = q_pitch<FMT>();
  constexpr int NST = DI / Step<FMT>::K;
  constexpr int RB = row_bytes<FMT>(DI);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;
  // the row and the workgroup's place in it: xw < kLead a lead workgroup (EMIT), else the
  // scoring workgroup xw - kLead of the row
  int64_t row = blockIdx.y;
  int64_t xw = blockIdx.x;
  if constexpr (EMIT) {
    const int64_t nsw = (p.G + kWaves * NKB * 32 - 1) / (kWaves * NKB * 32);
    const int64_t l = blockIdx.x;
    if (l < p.rows * kLead) {
      row = l / kLead;
      xw = l % kLead;
    } else {
      row = (l - p.rows * kLead) / nsw;
      xw = kLead + (l - p.rows * kLead) % nsw;
    }
  }
  const int64_t b = row / p.S;
  const int Hi = p.Hi;
  const int64_t G = p.G;
  const float inv_sqrt_di = 1.0f / sqrt_rn(static_cast<float>(DI));

  const uint8_t* kb_base = p.k + b * p.kbs * RB;
  const float* ks_base = FMT == kFp8 ? p.k_scale + b * p.kbs : nullptr;
  const uint8_t* ke_base = FMT == kMxfp4 ? p.k_e8m0 + b * p.kbs * (DI / 32) : nullptr;
  float* out = p.scores + row * p.sstride;

  if constexpr (EMIT) {
    if (xw == 0) {  // uniform: the row's emission
      // a step that completes no group has nothing here (its carry slot is lead workgroup
      // 1's): leave before requesting anything, so the compute unit's key stream is not
      // queued behind this workgroup's loads
      if (emitted_group(e, *(const_i64_ptr)(e.positions + row)) >= 0) emit_and_score<FMT, MB>(p, e, row);
      return;
    }
    if (xw == 1) {  // uniform: the token's window entry and its carry slot
      if (tid < 64) kv_prologue(e, row, tid);
      else carry_slot<kWaves * 64 - 64>(e, row, tid - 64);
      // on a group step then the key projection's second half, which the emission workgroup
      // waits for
      if (emitted_group(e, *(const_i64_ptr)(e.positions + row)) >= 0) emit_row<kEmitRatio, true, 2>(e, row, nullptr);
      return;
    }
    if (COARSE && xw < kLead) {  // uniform: a part of the coarse branch's group step
      coarse_body(es.coarse, row * kCoarseParts + (xw - 2));
      return;
    }
  }
  const int64_t wave_key0 =
      (xw - kLead) * (kWaves * NKB * 32) + wave * (NKB * 32);
  // Load order.  Vector-memory loads complete in issue order, so the small operands every
  // tile needs -- the query (fragments, or the bf16 rows to quantize) and the head
  // weights -- go first; then all key fragments of the wave's tiles, so tile 0's MFMAs
  // start while the later tiles are still arriving.  No load waits for the row's position
  // and none sits behind a branch (out-of-range rows are clamped to readable ones), so the
  // compiler's in-order wait counts stay exact.
  Frag a[MB][NST];
  uint4 qr[4];  // QRAW: 32 bf16 channels of head tid/4
  uint4 qtab = uint4{0u, 0u, 0u, 0u};  // FUSE: 16 bytes of the row's query cos / sin tables
  uint32_t tw[EMIT ? kRopePairs : 1];  // EMIT: the row's table row (cos | sin), uniform
  int64_t epos = 0;                     // EMIT: the row's position (a scalar load)
  const int qh = tid >> 2, qc = tid & 3;
  if constexpr (QRAW) {
    const int hq = qh < Hi ? qh : Hi - 1;
    const uint4* src = reinterpret_cast<const uint4*>(p.q_raw + (row * Hi + hq) * 128 + 32 * qc);
#pragma unroll
    for (int i = 0; i < 4; ++i) qr[i] = src[i];
    if constexpr (FUSE && !EMIT) {
      // the row's cos then sin tables (q_rope_dim / 16 pieces of 16 bytes each), one piece
      // per thread of the first 2 * q_rope_dim / 16; the rest read piece 0 and drop it
      const int n4 = p.q_rope_dim / 16;
      const int t = tid < 2 * n4 ? tid : 0;
      const uint16_t* tab = t < n4 ? p.q_cos : p.q_sin;
      qtab = reinterpret_cast<const uint4*>(tab + row * (p.q_rope_dim / 2))[t < n4 ? t : t - n4];
    }
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int h = mb * 32 + (lane & 31);
      const bool hv = h < Hi;
      const uint8_t* qrow = p.q + (row * Hi + (hv ? h : 0)) * static_cast<int64_t>(RB);
      const uint8_t* erow = FMT == kMxfp4 ? p.q_e8m0 + (row * Hi + (hv ? h : 0)) * (DI / 32) : nullptr;
#pragma unroll
      for (int st = 0; st < NST; ++st) a[mb][st] = keep_or_zero(load_frag<FMT, DI>(qrow, erow, st, hi), hv);
    }
  }
  // per-head coefficients w (x the FP8 query scale): lane h loads head h's, and every lane
  // then gathers the 16 rows of its accumulators with cross-lane reads
  const int hl = lane < Hi ? lane : Hi - 1;
  float cw = p.w[row * Hi + hl];
  float cq = 1.0f;
  if constexpr (FMT == kFp8 && !QRAW) cq = p.q_scale[row * Hi + hl];
  cw = lane < Hi ? cw : 0.0f;
  // FUSE: the kv prologue's operands come after the query's (whose wait ends in a barrier of
  // the whole workgroup) and before the keys (which the score loop waits for)
  FusedKv fkv;
  if constexpr (FUSE && !EMIT) {
    if (xw == 0 && tid < 64) fkv.load(p, row, tid);
  }
  // Key fragments: up to five tiles per wave are all requested here; more (a wave of 8 or 16
  // tiles, EMIT's long-row forms) stream through a ring of NBUF tile slots, tile t + NBUF
  // requested into tile t's slot once tile t is scored, so NBUF tiles stay in flight: 8 KB of
  // keys per wave, two FP8 tiles or four MXFP4 ones (measured best of 2 .. 7 slots for both:
  // more in flight was slower).  Every request is unconditional (rows clamped), which keeps
  // the in-order wait counts exact.
  constexpr int NBUF = NKB > 5 ? (FMT == kFp8 ? 2 : 4) : NKB;
  static_assert(NBUF == NKB || (EMIT && !GATHER), "the tile ring serves the merged emission's scorer");
  Frag bf[NBUF][NST];
  float ksv[NBUF];  // FP8: the per-key scales
  int32_t cblk[NKB];  // GATHER: the candidate block of each tile's slot, all loaded first
  if constexpr (GATHER) {
    // (loads complete in order: list entries issued between key loads would make each
    // tile's key loads wait for the previous tile's keys)
#pragma unroll
    for (int t = 0; t < NKB; ++t) {
      const int64_t g = wave_key0 + t * 32 + (lane & 31);
      const int64_t gc = g < G ? g : G - 1;  // slots at or beyond G: the row's last slot
      cblk[t] = p.cand[row * p.cand_stride + gc / p.cand_bs];
    }
  }
  auto issue = [&](int t) __attribute__((always_inline)) {
    // keys at or beyond G read row G-1 instead: their score columns are never written
    const int64_t g = wave_key0 + t * 32 + (lane & 31);
    int64_t gc = g < G ? g : G - 1;
    if constexpr (GATHER) {
      // candidate slot gc -> its key (an empty slot reads key 0: its score is never written)
      const int64_t kg = static_cast<int64_t>(cblk[t]) * p.cand_bs + gc % p.cand_bs;
      gc = (cblk[t] >= 0 && kg < p.cand_keys) ? kg : 0;
    }
    const uint8_t* krow = kb_base + gc * RB;
    const uint8_t* kerow = FMT == kMxfp4 ? ke_base + gc * (DI / 32) : nullptr;
#pragma unroll
    for (int st = 0; st < NST; ++st) bf[t % NBUF][st] = load_frag<FMT, DI>(krow, kerow, st, hi);
    ksv[t % NBUF] = FMT == kFp8 ? ks_base[gc] : 1.0f;
  };
#pragma unroll
  for (int t = 0; t < NBUF; ++t) issue(t);
  // APPEND: thread t's share of the new latent (nope channels 4t..4t+3, rope channel t),
  // loaded by every workgroup (clamped), packed by workgroup 0 at the end
  uint2 kv_nope = uint2{0u, 0u};
  uint16_t kv_rope = 0;
  if constexpr (APPEND) {
    const uint16_t* kvrow = p.kv + row * (p.nope + p.rope);
    const int tn = tid < p.nope / 4 ? tid : p.nope / 4 - 1;
    const int tr = tid < p.rope ? tid : p.rope - 1;
    kv_nope = *reinterpret_cast<const uint2*>(kvrow + 4 * tn);
    kv_rope = kvrow[p.nope + tr];
  }
  if constexpr (EMIT) {
    // the row's position and RoPE tables, scalar loads issued behind the vector loads above
    epos = *(const_i64_ptr)(p.positions + row);
    load_table_row(e, epos, tw);
  }
  const int64_t pos = EMIT ? epos : (p.positions ? p.positions[row] : row % p.S);
  int64_t vis = EMIT ? (pos + 1) / kEmitRatio : (pos + 1) / p.ratio;
  const int64_t nkeys = GATHER ? p.cand_keys : G;
  if (vis > nkeys) vis = nkeys;
  if (vis < 0) vis = 0;
  // EMIT: the key the row's emission workgroup scores (-1: none), as emit_row decides
  const int64_t g_own = EMIT ? emitted_group(e, pos) : -1;

  __shared__ __align__(16) uint8_t q_lds[QRAW ? 64 * QP : 16];
  __shared__ float qs_lds[QRAW && FMT == kFp8 ? 64 : 1];
  __shared__ uint8_t qe_lds[QRAW && FMT == kMxfp4 ? 256 : 4];
  __shared__ uint4 qtab_lds[FUSE && !EMIT ? 16 : 1];
  if constexpr (EMIT) {
    rope_query_table(qr, qc, tw);
    // the step's RoPE tables (row pos of the position table, which the later launches of
    // the step read) from the row's first scoring workgroup, which holds the row already
    // (emit_row<R, true> leaves them to it): cos in words 0..15 of tw, sin in 16..31
    if (xw == kLead && tid == 0 && e.step_cos && epos >= 0 && epos < e.tab_rows) {
      uint4* dc = reinterpret_cast<uint4*>(e.step_cos + row * kRopePairs);
      uint4* ds = reinterpret_cast<uint4*>(e.step_sin + row * kRopePairs);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        dc[k] = uint4{tw[4 * k], tw[4 * k + 1], tw[4 * k + 2], tw[4 * k + 3]};
        ds[k] = uint4{tw[16 + 4 * k], tw[16 + 4 * k + 1], tw[16 + 4 * k + 2], tw[16 + 4 * k + 3]};
      }
    }
  } else if constexpr (FUSE) {
    // RoPE of the query's rope channels (owlet1/indexer.py:126-128, compress cos / sin),
    // bf16 in and out as the reference's rotated query.  q_rope_dim is a multiple of 32, so
    // a thread's 32 channels are all rope or all nope.
    const int n4 = p.q_rope_dim / 16;
    if (tid < 2 * n4) qtab_lds[tid] = qtab;
    __syncthreads();
    const int first = 32 * qc - (128 - p.q_rope_dim);
    if (first >= 0) {
      // this thread's 16 pairs: 32 bytes of cos and of sin (two 16-byte pieces each)
      const uint4* ct = qtab_lds + first / 16;
      const uint4* st = ct + p.q_rope_dim / 16;
      const uint4 c0 = ct[0], c1 = ct[1], s0 = st[0], s1 = st[1];
      const uint32_t cw_[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const uint32_t sw_[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      uint32_t* wq = reinterpret_cast<uint32_t*>(qr);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const uint32_t cp = cw_[k >> 1], sp = sw_[k >> 1];
        wq[k] = rope_pair_bf16(wq[k], __uint_as_float((k & 1) ? cp & 0xffff0000u : cp << 16),
                               __uint_as_float((k & 1) ? sp & 0xffff0000u : sp << 16));
      }
    }
  }
  if constexpr (QRAW) quantize_query<FMT, DI, MB>(qr, qh, qc, Hi, lane, hi, hl, q_lds, qs_lds, qe_lds, a, cq);
  if constexpr (FUSE && !EMIT) {
    // the row's kv prologue, while the key loads are still in flight (its registers are
    // free again before the score loop)
    if (xw == 0 && tid < 64) fkv.append(p, b, pos, tid);
  }
  const float cwq = cw * cq;
  float coef[MB][16];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 16; ++j) coef[mb][j] = __shfl(cwq, mb * 32 + acc_row(j, lane), 64);

  // the scores of tile t (a tile that starts below G)
  auto score = [&](int t) __attribute__((always_inline)) {
    const int64_t g0 = wave_key0 + t * 32;
    const int64_t g = g0 + (lane & 31);
    if (!GATHER && g0 >= vis) {  // nothing in this tile is visible to the row
      if (lane < 32 && g < G) out[g] = -__builtin_huge_valf();
      return;
    }
    float part = 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      v16f acc = {};
#pragma unroll
      for (int st = 0; st < NST; ++st) acc = mma<FMT>(a[mb][st], bf[t % NBUF][st], acc);
#pragma unroll
      for (int j = 0; j < 16; ++j) part = relu_fma(coef[mb][j], acc[j], part);
    }
    const float total = part + __shfl_xor(part, 32, 64);
    if (lane < 32 && g < G && (!EMIT || g != g_own)) {
      float s = total * inv_sqrt_di;
      if constexpr (FMT == kFp8) s = s * ksv[t % NBUF];
      int64_t kpos = g;
      if constexpr (GATHER) {  // g < G here, so cblk[t] is slot g's block
        kpos = static_cast<int64_t>(cblk[t]) * p.cand_bs + g % p.cand_bs;
        if (cblk[t] < 0) kpos = -1;
      }
      out[g] = (kpos >= 0 && kpos < vis) ? s : -__builtin_huge_valf();
    }
  };
  if constexpr (NBUF == NKB) {
#pragma unroll
    for (int t = 0; t < NKB; ++t) {
      if (wave_key0 + t * 32 >= G) break;
      score(t);
    }
  } else {
    // the ring: the next request into this tile's slot follows its scores, whether or not the
    // tile lies inside the row (so every wave issues the same requests)
#pragma unroll
    for (int t = 0; t < NKB; ++t) {
      if (wave_key0 + t * 32 < G) score(t);
      if (t + NBUF < NKB) issue(t + NBUF);
    }
  }

  if constexpr (QRAW) {
    if (xw == 0) {
      // the quantized query, for callers that keep it (the codes are still in LDS)
      if constexpr (FMT == kFp8) {
        if (p.q_codes_out && qh < Hi) {
          const uint4* src = reinterpret_cast<const uint4*>(q_lds + qh * QP + 32 * qc);
          uint4* dst = reinterpret_cast<uint4*>(p.q_codes_out + (row * Hi + qh) * 128 + 32 * qc);
          dst[0] = src[0];
          dst[1] = src[1];
          if (qc == 0) p.q_scales_out[row * Hi + qh] = qs_lds[qh];
        }
      } else {
        if (p.q_codes_out && qh < Hi) {
          *reinterpret_cast<uint4*>(p.q_codes_out + (row * Hi + qh) * 64 + 16 * qc) =
              *reinterpret_cast<const uint4*>(q_lds + qh * QP + 16 * qc);
          p.q_e8m0_out[(row * Hi + qh) * 4 + qc] = qe_lds[qh * 4 + qc];
        }
      }
      if constexpr (APPEND) {
        // FP8-b128 latent entry (as pack_latent_row): threads t < nope/4 hold 4 nope
        // channels each (32 lanes per 128-channel block), threads t < rope one rope channel;
        // a negative position has no ring slot
        if (pos >= 0) {
          const int64_t entry_bytes = p.nope + 4 * (p.nope / 128) + 2 * p.rope;
          uint8_t* ent = p.win + (b * p.win_batch_entries + pos % p.win_cap) * entry_bytes;
          if (tid < p.nope / 4) {
            const float v[4] = {bf16_to_f32(static_cast<uint16_t>(kv_nope.x & 0xffffu)),
                                bf16_to_f32(static_cast<uint16_t>(kv_nope.x >> 16)),
                                bf16_to_f32(static_cast<uint16_t>(kv_nope.y & 0xffffu)),
                                bf16_to_f32(static_cast<uint16_t>(kv_nope.y >> 16))};
            float am = abs_max4(v);
            am = wave_max_group(am, 32);
            const float sc = fp8_scale_from_amax(am);
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) word |= static_cast<uint32_t>(e4m3_encode(clampf(div_rn(v[i], sc), 448.0f))) << (8 * i);
            reinterpret_cast<uint32_t*>(ent)[tid] = word;
            if ((tid & 31) == 0) reinterpret_cast<float*>(ent + p.nope)[tid >> 5] = sc;
          }
          if (tid < p.rope) reinterpret_cast<uint16_t*>(ent + p.nope + 4 * (p.nope / 128))[tid] = kv_rope;
        }
      }
    }
  }
}


// ------------------------------------------------------------------------------------
// Prefill form (FP8, Di = 128): many query rows against the same keys.  The decode tiling
// re-streams every key for every query row; here one workgroup takes kPfQb query rows and
// walks the key blocks of 512: per block a wave holds 128 keys (4 N-blocks of 32, two
// 64-channel steps) as the MFMA B operand and runs the rows through them (A = a row's 64
// heads as two 32-row M-blocks).  The rows' codes are staged in LDS once, at the start (one
// memory round trip; 144-byte row pitch against bank conflicts), with the per-head weights
// w * q_scale next to them; each lane reads the 16 accumulator rows it holds.  Within a
// row the next key tile's MFMAs are issued while the current tile's ReLU-weighted head sum
// runs (the two take about as long).  Keys a row cannot see (at or beyond (pos + 1) //
// ratio) are written as -inf without MFMA work, blocks beyond every row's visibility
// without loading them, and the workgroups with the most visible keys are dispatched first
// (the grid runs the query blocks from the last to the first).  The head sum runs in the
// row kernel's order, so the scores are the row kernel's bit for bit.
// ------------------------------------------------------------------------------------
constexpr int kPfQb = 8;               // query rows per workgroup
constexpr int kPfPrefillMinRows = 64;  // rows per batch from which the prefill form is used
constexpr int kPfPitch = 144;          // LDS bytes per staged head row
constexpr int kPfLds = kPfQb * 64 * kPfPitch + kPfQb * 64 * 4 + kPfQb * 8;

__global__ void __launch_bounds__(kWaves * 64, 2) indexer_prefill_fp8_kernel(const IdxParams p, int64_t nqb) {
  constexpr int DI = 128, NST = 2;
  extern __shared__ __align__(16) uint8_t pf_smem[];
  uint8_t* q_lds = pf_smem;                                                   // [qb][64][kPfPitch]
  float* coef_lds = reinterpret_cast<float*>(pf_smem + kPfQb * 64 * kPfPitch);  // [qb][64]
  int64_t* vis_lds = reinterpret_cast<int64_t*>(coef_lds + kPfQb * 64);        // [qb]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;
  const int64_t nkb = (p.G + kKeysPerWg - 1) / kKeysPerWg;
  const int64_t qb_all = static_cast<int64_t>(gridDim.x) - 1 - blockIdx.x;  // last query block first
  const int64_t b = qb_all / nqb;
  const int64_t s0 = (qb_all % nqb) * kPfQb;
  const int Hi = p.Hi;
  const int64_t G = p.G, S = p.S;
  const float inv_sqrt_di = 1.0f / sqrt_rn(static_cast<float>(DI));
  const int nq = static_cast<int>(S - s0 < kPfQb ? S - s0 : kPfQb);
  const uint8_t* kb_base = p.k + b * p.kbs * DI;
  const float* ks_base = p.k_scale + b * p.kbs;
  // the rows' codes: 16-byte piece i = (row, head, piece) of the block, every load issued
  // before any is stored (rows beyond the block and heads beyond Hi read row 0 / head 0 and
  // store zeros)
  constexpr int kPieces = kPfQb * 64 * (DI / 16);
  constexpr int kPerThread = kPieces / (kWaves * 64);
  uint4 pc[kPerThread];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int i = tid + k * kWaves * 64;
    const int qi = i / (64 * (DI / 16)), h = (i / (DI / 16)) % 64, c = i % (DI / 16);
    const bool ok = qi < nq && h < Hi;
    const int64_t r = b * S + s0 + (ok ? qi : 0);
    pc[k] = *reinterpret_cast<const uint4*>(p.q + (r * Hi + (ok ? h : 0)) * DI + 16 * c);
  }
  for (int i = tid; i < kPfQb * 64; i += kWaves * 64) {
    const int qi = i >> 6, h = i & 63;
    float c = 0.0f;
    if (qi < nq && h < Hi) {
      const int64_t r = b * S + s0 + qi;
      c = p.w[r * Hi + h] * p.q_scale[r * Hi + h];
    }
    coef_lds[i] = c;
  }
  if (tid < kPfQb) {
    int64_t v = 0;
    if (tid < nq) {
      const int64_t r = b * S + s0 + tid;
      const int64_t pos = p.positions ? p.positions[r] : s0 + tid;
      v = (pos + 1) / p.ratio;
      v = v > G ? G : (v < 0 ? 0 : v);
    }
    vis_lds[tid] = v;
  }
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int i = tid + k * kWaves * 64;
    const int qi = i / (64 * (DI / 16)), h = (i / (DI / 16)) % 64, c = i % (DI / 16);
    const bool ok = qi < nq && h < Hi;
    *reinterpret_cast<uint4*>(q_lds + (qi * 64 + h) * kPfPitch + 16 * c) = ok ? pc[k] : uint4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  int64_t vis_max = 0;
  for (int qi = 0; qi < nq; ++qi) vis_max = vis_lds[qi] > vis_max ? vis_lds[qi] : vis_max;

  // the key blocks in turn: every block with a visible key is scored, and the blocks
  // beyond every row's visibility are written as -inf
  for (int64_t kb = 0; kb < nkb; ++kb) {
    const int64_t key0 = kb * kKeysPerWg + wave * (kNkb * 32);
    if (kb * kKeysPerWg >= vis_max) {
      if (lane < 32) {
        for (int qi = 0; qi < nq; ++qi) {
          float* out = p.scores + (b * S + s0 + qi) * p.sstride;
#pragma unroll
          for (int t = 0; t < kNkb; ++t) {
            const int64_t g = key0 + t * 32 + lane;
            if (g < G) out[g] = -__builtin_huge_valf();
          }
        }
      }
      continue;
    }
    // the wave's keys: B fragments and per-key scales (keys at or beyond G read key G-1;
    // their score columns are never written)
    Frag bf[kNkb][NST];
    float ksv[kNkb];
#pragma unroll
    for (int t = 0; t < kNkb; ++t) {
      const int64_t g = key0 + t * 32 + (lane & 31);
      const int64_t gc = g < G ? g : G - 1;
#pragma unroll
      for (int st = 0; st < NST; ++st) bf[t][st] = load_frag<kFp8, DI>(kb_base + gc * DI, nullptr, st, hi);
      ksv[t] = ks_base[gc];
    }
    for (int qi = 0; qi < nq; ++qi) {
      const int64_t vis = vis_lds[qi];
      float* out = p.scores + (b * S + s0 + qi) * p.sstride;
      if (key0 < vis) {
        Frag a[2][NST];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int st = 0; st < NST; ++st) {
            const uint4* src =
                reinterpret_cast<const uint4*>(q_lds + (qi * 64 + mb * 32 + (lane & 31)) * kPfPitch + st * 64 + hi * 32);
            const uint4 u = src[0], v = src[1];
            a[mb][st].v = v8i{(int)u.x, (int)u.y, (int)u.z, (int)u.w, (int)v.x, (int)v.y, (int)v.z, (int)v.w};
            a[mb][st].scale = 127;
          }
        // this lane's 16 accumulator rows of each M-block: 4 runs of 4 consecutive heads
        float cf[2][16];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const float4 c4 = *reinterpret_cast<const float4*>(coef_lds + qi * 64 + mb * 32 + 8 * r4 + 4 * hi);
            cf[mb][4 * r4 + 0] = c4.x;
            cf[mb][4 * r4 + 1] = c4.y;
            cf[mb][4 * r4 + 2] = c4.z;
            cf[mb][4 * r4 + 3] = c4.w;
          }
        // Software pipeline over the 4 key tiles: the MFMAs of tile t+1 are issued while the
        // head sum of tile t runs (one MFMA per 16 VALU operations, about one MFMA's duration),
        // so the matrix and vector units work at the same time; the stores come after.
        float total[kNkb];
        v16f acc[2][2];  // [tile parity][M-block]
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          acc[0][mb] = v16f{};
#pragma unroll
          for (int st = 0; st < NST; ++st) acc[0][mb] = mma<kFp8>(a[mb][st], bf[0][st], acc[0][mb]);
        }
#pragma unroll
        for (int t = 0; t < kNkb; ++t) {
          const int cur = t & 1, nxt = cur ^ 1;
          if (t + 1 < kNkb) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
              acc[nxt][mb] = v16f{};
#pragma unroll
              for (int st = 0; st < NST; ++st) acc[nxt][mb] = mma<kFp8>(a[mb][st], bf[t + 1][st], acc[nxt][mb]);
            }
          }
          float part = 0.0f;
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int j = 0; j < 16; ++j) part = relu_fma(cf[mb][j], acc[cur][mb][j], part);
          if (t + 1 < kNkb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // sixteen VALU
            }
          }
          total[t] = part + __shfl_xor(part, 32, 64);
        }
        if (lane < 32) {
#pragma unroll
          for (int t = 0; t < kNkb; ++t) {
            const int64_t g = key0 + t * 32 + lane;
            if (g < G) out[g] = g < vis ? (total[t] * inv_sqrt_di) * ksv[t] : -__builtin_huge_valf();
          }
        }
      } else if (lane < 32) {
#pragma unroll
        for (int t = 0; t < kNkb; ++t) {
          const int64_t g = key0 + t * 32 + lane;
          if (g < G) out[g] = -__builtin_huge_valf();
        }
      }
    }
  }

}

template <int FMT, int DI>
int launch_di(const IdxParams& p, int64_t rows, hipStream_t s) {
  dim3 grid(static_cast<unsigned>((p.G + kKeysPerWg - 1) / kKeysPerWg), static_cast<unsigned>(rows));
  if (p.Hi <= 32) indexer_scores_kernel<FMT, DI, 1, false, false><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  else indexer_scores_kernel<FMT, DI, 2, false, false><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  return MZK_OK;
}

// The candidate scorer: p.G is the row's slot count (n_blocks * block_size).
template <int FMT>
int launch_gather(const IdxParams& p, int64_t rows, int Di, hipStream_t s) {
  dim3 grid(static_cast<unsigned>((p.G + kKeysPerWg - 1) / kKeysPerWg), static_cast<unsigned>(rows));
  if (Di != 128) {
    set_last_error("indexer_candidate_scores: index head dim must be 128 (got %d)", Di);
    return MZK_EUNSUPPORTED;
  }
  if (p.Hi <= 32) indexer_scores_kernel<FMT, 128, 1, false, false, false, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  else indexer_scores_kernel<FMT, 128, 2, false, false, false, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  return MZK_OK;
}

// Slot indices of the candidate axis -> key positions (in place allowed): one thread per
// entry; -1 and empty slots stay -1.  Ascending slots give ascending positions, since the
// candidate blocks are ascending.
__global__ void candidate_positions_kernel(const int32_t* __restrict__ slot_idx, int64_t rows, int k,
                                           int64_t idx_stride, const int32_t* __restrict__ cand, int64_t cand_stride,
                                           int n_blocks, int block_size, int32_t* __restrict__ pos, int64_t pos_stride) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows * k) return;
  const int64_t row = t / k, j = t - row * k;
  const int32_t sl = slot_idx[row * idx_stride + j];
  int32_t out = -1;
  if (sl >= 0 && sl < n_blocks * block_size) {
    const int32_t blk = cand[row * cand_stride + sl / block_size];
    if (blk >= 0) out = blk * block_size + sl % block_size;
  }
  pos[row * pos_stride + j] = out;
}

template <int FMT>
int launch(const IdxParams& p, int64_t rows, int Di, hipStream_t s) {
  switch (Di) {
    case 64: return launch_di<FMT, 64>(p, rows, s);
    case 128: return launch_di<FMT, 128>(p, rows, s);
    case 256: return launch_di<FMT, 256>(p, rows, s);
    default:
      if constexpr (FMT == kBf16) {
        if (Di == 96) return launch_di<FMT, 96>(p, rows, s);
        if (Di == 32) return launch_di<FMT, 32>(p, rows, s);
      }
      set_last_error("indexer_scores: unsupported index head dim %d", Di);
      return MZK_EUNSUPPORTED;
  }
}

// Workgroups resident at once on the current device at `per_cu` per compute unit (the
// count read once per device; 256 compute units if the query fails).
int resident_workgroups(int per_cu) {
  static int cus[16] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return per_cu * cus[dev];
}

IdxParams make_params(const uint8_t* q, const float* qs, const uint8_t* qe, const float* w, const uint8_t* k,
                      const float* ks, const uint8_t* ke, int64_t S, int Hi, int64_t G, int64_t kbs, const int64_t* pos,
                      int ratio, float* scores, int64_t sstride) {
  IdxParams p{};
  p.q = q;
  p.q_scale = qs;
  p.q_e8m0 = qe;
  p.w = w;
  p.k = k;
  p.k_scale = ks;
  p.k_e8m0 = ke;
  p.S = S;
  p.Hi = Hi;
  p.G = G;
  p.kbs = kbs;
  p.positions = pos;
  p.ratio = ratio;
  p.scores = scores;
  p.sstride = sstride;
  return p;
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

int check_candidates(int64_t B, int64_t S, int64_t G, const int32_t* cand, int64_t cand_stride, int n_blocks,
                     int block_size, int64_t slots_stride) {
  MZK_CHECK_ARG(n_blocks >= 0 && block_size >= 1 && cand_stride >= n_blocks,
                "indexer_candidate_scores: bad candidate list shape");
  MZK_CHECK_ARG(static_cast<int64_t>(n_blocks) * block_size <= (int64_t(1) << 30),
                "indexer_candidate_scores: more than 2^30 candidate slots");
  MZK_CHECK_ARG(static_cast<int64_t>(n_blocks) * block_size <= slots_stride,
                "indexer_candidate_scores: score stride smaller than n_blocks * block_size");
  MZK_CHECK_ARG(G < (int64_t(1) << 31), "indexer_candidate_scores: key count must fit int32");
  MZK_CHECK_ARG(B * S <= 65535, "indexer_candidate_scores: at most 65535 query rows (got %lld)", (long long)(B * S));
  MZK_CHECK_ARG(n_blocks == 0 || cand != nullptr, "indexer_candidate_scores: null candidate list");
  return MZK_OK;
}

IdxParams with_candidates(IdxParams p, int64_t G, const int32_t* cand, int64_t cand_stride, int n_blocks,
                          int block_size) {
  p.G = static_cast<int64_t>(n_blocks) * block_size;
  p.cand = cand;
  p.cand_stride = cand_stride;
  p.cand_nb = n_blocks;
  p.cand_bs = block_size;
  p.cand_keys = G;
  return p;
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
  const IdxParams prm = make_params(q_codes, q_scales, nullptr, w, k_codes, k_scales, nullptr, S, Hi, G, k_batch_stride,
                                    positions, ratio, scores, score_stride);
  if (Di == 128 && S >= kPfPrefillMinRows) {
    // prefill: query rows stream through key tiles held in registers
    const int64_t nqb = (S + kPfQb - 1) / kPfQb;
    const int64_t nblocks = B * nqb;
    MZK_CHECK_ARG(nblocks <= 0x7fffffff, "indexer_scores_fp8: %lld workgroups exceed the grid limit", (long long)nblocks);
    // the staged query rows need more than the default dynamic-LDS limit: set once per device
    static std::atomic<bool> attr_set[kMaxDevices] = {};  // setting it twice is harmless
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
      set_last_error("indexer_scores_fp8: no usable current device");
      return MZK_ELAUNCH;
    }
    if (!attr_set[dev].load(std::memory_order_acquire)) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(indexer_prefill_fp8_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kPfLds) != hipSuccess) {
        set_last_error("indexer_scores_fp8: cannot raise the prefill kernel's LDS limit to %d bytes", kPfLds);
        return MZK_ELAUNCH;
      }
      attr_set[dev].store(true, std::memory_order_release);
    }
    indexer_prefill_fp8_kernel<<<static_cast<unsigned>(nblocks), kWaves * 64, kPfLds, as_stream(stream)>>>(prm, nqb);
  } else {
    rc = launch<kFp8>(prm, B * S, Di, as_stream(stream));
  }
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
  rc = launch<kMxfp4>(make_params(q_packed, nullptr, q_e8m0, w, k_packed, nullptr, k_e8m0, S, Hi, G, k_batch_stride,
                                  positions, ratio, scores, score_stride),
                      B * S, Di, as_stream(stream));
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
  rc = launch<kBf16>(make_params(static_cast<const uint8_t*>(q), nullptr, nullptr, w, static_cast<const uint8_t*>(k),
                                 nullptr, nullptr, S, Hi, G, k_batch_stride, positions, ratio, scores, score_stride),
                     B * S, Di, as_stream(stream));
  if (rc) return rc;
  MZK_LAUNCH_CHECK("indexer_scores_bf16");
  return MZK_OK;
}

extern "C" int mzk_indexer_decode_fp8(const void* q_idx, const float* w, const uint8_t* k_codes, const float* k_scales,
                                      int64_t B, int Hi, int Di, int64_t G, int64_t k_batch_stride,
                                      const int64_t* positions, int ratio, float* scores, int64_t score_stride,
                                      uint8_t* q_codes, float* q_scales, const void* kv, int nope, int rope,
                                      uint8_t* win_cache, int64_t win_batch_entries, int win_cap, void* stream) {
  int rc = check_common(B, 1, Hi, Di, G, k_batch_stride, ratio, score_stride);
  if (rc) return rc;
  MZK_CHECK_ARG(Di == 128, "indexer_decode_fp8: the fused decode form needs Di = 128 (got %d)", Di);
  MZK_CHECK_ARG(positions != nullptr, "indexer_decode_fp8: positions are required");
  MZK_CHECK_ARG((q_codes == nullptr) == (q_scales == nullptr), "indexer_decode_fp8: q_codes and q_scales go together");
  if (kv) {
    MZK_CHECK_ARG(win_cache && win_cap >= 1 && win_batch_entries >= win_cap, "indexer_decode_fp8: bad window ring");
    MZK_CHECK_ARG(nope >= 128 && nope % 128 == 0 && nope <= 4 * kWaves * 64 && rope >= 1 && rope <= kWaves * 64 &&
                      rope % 2 == 0,
                  "indexer_decode_fp8: latent %d+%d unsupported (nope a multiple of 128 up to 1024, rope even up to 256)",
                  nope, rope);
  }
  if (B == 0) return MZK_OK;
  MZK_CHECK_ARG(G >= 1, "indexer_decode_fp8: at least one key group is required");
  MZK_CHECK_ARG(q_idx && w && k_codes && k_scales && scores, "indexer_decode_fp8: null pointer");
  MZK_CHECK_ARG(aligned16(q_idx) && aligned16(k_codes) && aligned16(q_codes) && aligned16(kv) && aligned16(win_cache),
                "indexer_decode_fp8: q_idx, k_codes, q_codes, kv and the window cache must be 16-byte aligned");
  IdxParams p = make_params(nullptr, nullptr, nullptr, w, k_codes, k_scales, nullptr, 1, Hi, G, k_batch_stride,
                            positions, ratio, scores, score_stride);
  p.q_raw = static_cast<const uint16_t*>(q_idx);
  p.q_codes_out = q_codes;
  p.q_scales_out = q_scales;
  p.kv = static_cast<const uint16_t*>(kv);
  p.nope = nope;
  p.rope = rope;
  p.win = win_cache;
  p.win_batch_entries = win_batch_entries;
  p.win_cap = win_cap;
  dim3 grid(static_cast<unsigned>((G + kKeysPerWg - 1) / kKeysPerWg), static_cast<unsigned>(B));
  hipStream_t s = as_stream(stream);
  if (Hi <= 32) {
    if (kv) indexer_scores_kernel<kFp8, 128, 1, true, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
    else indexer_scores_kernel<kFp8, 128, 1, true, false><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  } else {
    if (kv) indexer_scores_kernel<kFp8, 128, 2, true, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
    else indexer_scores_kernel<kFp8, 128, 2, true, false><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  }
  MZK_LAUNCH_CHECK("indexer_decode_fp8");
  return MZK_OK;
}

extern "C" int mzk_indexer_decode_mxfp4(const void* q_idx, const float* w, const uint8_t* k_packed,
                                        const uint8_t* k_e8m0, int64_t B, int Hi, int Di, int64_t G,
                                        int64_t k_batch_stride, const int64_t* positions, int ratio, float* scores,
                                        int64_t score_stride, uint8_t* q_packed, uint8_t* q_e8m0, const void* kv,
                                        int nope, int rope, uint8_t* win_cache, int64_t win_batch_entries,
                                        int win_cap, void* stream) {
  int rc = check_common(B, 1, Hi, Di, G, k_batch_stride, ratio, score_stride);
  if (rc) return rc;
  MZK_CHECK_ARG(Di == 128, "indexer_decode_mxfp4: the fused decode form needs Di = 128 (got %d)", Di);
  MZK_CHECK_ARG(positions != nullptr, "indexer_decode_mxfp4: positions are required");
  MZK_CHECK_ARG((q_packed == nullptr) == (q_e8m0 == nullptr), "indexer_decode_mxfp4: q_packed and q_e8m0 go together");
  if (kv) {
    MZK_CHECK_ARG(win_cache && win_cap >= 1 && win_batch_entries >= win_cap, "indexer_decode_mxfp4: bad window ring");
    MZK_CHECK_ARG(nope >= 128 && nope % 128 == 0 && nope <= 4 * kWaves * 64 && rope >= 1 && rope <= kWaves * 64 &&
                      rope % 2 == 0,
                  "indexer_decode_mxfp4: latent %d+%d unsupported (nope a multiple of 128 up to 1024, rope even up to 256)",
                  nope, rope);
  }
  if (B == 0) return MZK_OK;
  MZK_CHECK_ARG(G >= 1, "indexer_decode_mxfp4: at least one key group is required");
  MZK_CHECK_ARG(q_idx && w && k_packed && k_e8m0 && scores, "indexer_decode_mxfp4: null pointer");
  MZK_CHECK_ARG(aligned16(q_idx) && aligned16(k_packed) && aligned16(q_packed) && aligned16(kv) && aligned16(win_cache),
                "indexer_decode_mxfp4: q_idx, k_packed, q_packed, kv and the window cache must be 16-byte aligned");
  IdxParams p = make_params(nullptr, nullptr, nullptr, w, k_packed, nullptr, k_e8m0, 1, Hi, G, k_batch_stride,
                            positions, ratio, scores, score_stride);
  p.q_raw = static_cast<const uint16_t*>(q_idx);
  p.q_codes_out = q_packed;
  p.q_e8m0_out = q_e8m0;
  p.kv = static_cast<const uint16_t*>(kv);
  p.nope = nope;
  p.rope = rope;
  p.win = win_cache;
  p.win_batch_entries = win_batch_entries;
  p.win_cap = win_cap;
  dim3 grid(static_cast<unsigned>((G + kKeysPerWg - 1) / kKeysPerWg), static_cast<unsigned>(B));
  hipStream_t s = as_stream(stream);
  if (Hi <= 32) {
    if (kv) indexer_scores_kernel<kMxfp4, 128, 1, true, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
    else indexer_scores_kernel<kMxfp4, 128, 1, true, false><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  } else {
    if (kv) indexer_scores_kernel<kMxfp4, 128, 2, true, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
    else indexer_scores_kernel<kMxfp4, 128, 2, true, false><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  }
  MZK_LAUNCH_CHECK("indexer_decode_mxfp4");
  return MZK_OK;
}

extern "C" int mzk_indexer_decode_fused(int q_format, const void* q_idx, const float* w, const uint8_t* k_codes,
                                        const void* k_scales, int64_t B, int Hi, int Di, int64_t G,
                                        int64_t k_batch_stride, const int64_t* positions, int ratio, float* scores,
                                        int64_t score_stride, uint8_t* q_codes, void* q_scales, const void* q_cos,
                                        const void* q_sin, int q_rope_dim, const void* kv, const void* kv_weight,
                                        float kv_eps, const void* kv_cos, const void* kv_sin, int nope, int rope,
                                        uint8_t* win_cache, int64_t win_batch_entries, int win_cap, void* stream) {
  int rc = check_common(B, 1, Hi, Di, G, k_batch_stride, ratio, score_stride);
  if (rc) return rc;
  MZK_CHECK_ARG(q_format == 0 || q_format == 1, "indexer_decode_fused: q_format must be 0 (FP8) or 1 (MXFP4), got %d",
                q_format);
  MZK_CHECK_ARG(Di == 128, "indexer_decode_fused: the fused decode form needs Di = 128 (got %d)", Di);
  MZK_CHECK_ARG(q_rope_dim >= 32 && q_rope_dim <= 128 && q_rope_dim % 32 == 0,
                "indexer_decode_fused: q_rope_dim must be 32, 64, 96 or 128 (got %d)", q_rope_dim);
  MZK_CHECK_ARG(nope == kFuseNope && rope == kFuseRope, "indexer_decode_fused: latent %d+%d unsupported (needs 512+64)",
                nope, rope);
  MZK_CHECK_ARG(kv_eps >= 0.0f, "indexer_decode_fused: negative eps");
  MZK_CHECK_ARG(positions != nullptr, "indexer_decode_fused: positions are required");
  MZK_CHECK_ARG((q_codes == nullptr) == (q_scales == nullptr), "indexer_decode_fused: q_codes and q_scales go together");
  MZK_CHECK_ARG(win_cap >= 1 && win_batch_entries >= win_cap, "indexer_decode_fused: bad window ring");
  if (B == 0) return MZK_OK;
  MZK_CHECK_ARG(G >= 1, "indexer_decode_fused: at least one key group is required");
  MZK_CHECK_ARG(q_idx && w && k_codes && k_scales && scores && q_cos && q_sin && kv && kv_weight && kv_cos && kv_sin &&
                    win_cache,
                "indexer_decode_fused: null pointer");
  MZK_CHECK_ARG(aligned16(q_idx) && aligned16(k_codes) && aligned16(q_codes) && aligned16(q_cos) && aligned16(q_sin),
                "indexer_decode_fused: q_idx, k_codes, q_codes, q_cos and q_sin must be 16-byte aligned");
  MZK_CHECK_ARG(B <= 65535, "indexer_decode_fused: at most 65535 rows (got %lld)", (long long)B);
  const bool fp8 = q_format == 0;
  IdxParams p = make_params(nullptr, nullptr, nullptr, w, k_codes, fp8 ? static_cast<const float*>(k_scales) : nullptr,
                            fp8 ? nullptr : static_cast<const uint8_t*>(k_scales), 1, Hi, G, k_batch_stride, positions,
                            ratio, scores, score_stride);
  p.q_raw = static_cast<const uint16_t*>(q_idx);
  p.q_codes_out = q_codes;
  if (fp8) p.q_scales_out = static_cast<float*>(q_scales);
  else p.q_e8m0_out = static_cast<uint8_t*>(q_scales);
  p.q_cos = static_cast<const uint16_t*>(q_cos);
  p.q_sin = static_cast<const uint16_t*>(q_sin);
  p.q_rope_dim = q_rope_dim;
  p.kv = static_cast<const uint16_t*>(kv);
  p.kv_w = static_cast<const uint16_t*>(kv_weight);
  p.kv_eps = kv_eps;
  p.kv_cos = static_cast<const uint16_t*>(kv_cos);
  p.kv_sin = static_cast<const uint16_t*>(kv_sin);
  p.nope = nope;
  p.rope = rope;
  p.win = win_cache;
  p.win_batch_entries = win_batch_entries;
  p.win_cap = win_cap;
  dim3 grid(static_cast<unsigned>((G + kKeysPerWg - 1) / kKeysPerWg), static_cast<unsigned>(B));
  hipStream_t s = as_stream(stream);
  if (fp8) {
    if (Hi <= 32) indexer_scores_kernel<kFp8, 128, 1, true, false, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
    else indexer_scores_kernel<kFp8, 128, 2, true, false, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  } else {
    if (Hi <= 32) indexer_scores_kernel<kMxfp4, 128, 1, true, false, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
    else indexer_scores_kernel<kMxfp4, 128, 2, true, false, true><<<grid, kWaves * 64, 0, s>>>(p, EmitSet{});
  }
  MZK_LAUNCH_CHECK("indexer_decode_fused");
  return MZK_OK;
}

// The decode step's group emission and indexer scores in one launch (the EMIT scorer):
// mzk_decode_emit's arguments for the fine branch (ratio 4, with the index key and the kv
// prologue; the scoring workgroups quantize the indexer query themselves, so it has no
// q_codes / q_scales outputs), then the scorer's: q_idx bf16 [B, Hi, 128] (unrotated; its
// RoPE from the table row of the token's position), w fp32 [B, Hi], G keys per row (key
// batch stride key_batch_entries, the key format of the emission), scores fp32 [B,
// score_stride]; then, with c_kv, a keyless coarse branch (mzk_decode_emit_pair's c_*
// arguments; ratio 2 .. 128, B <= 1024).
extern "C" int mzk_decode_emit_scores(const int64_t* positions, int64_t B, const float* kv, const float* gate,
                                      float* carry_kv, float* carry_gate, int ratio, const void* norm_weight, float eps,
                                      uint8_t* cache, int64_t cache_batch_entries, int64_t cache_cap, const void* wk,
                                      const void* k_norm_weight, float k_eps, int key_format, uint8_t* k_codes,
                                      void* k_scales, int64_t key_batch_entries, const void* rope_table,
                                      int64_t table_rows, void* step_cos, void* step_sin, const void* kv_proj,
                                      const void* kv_weight, float kv_eps, uint8_t* win_cache, int64_t win_batch_entries,
                                      int win_cap, const void* q_idx, const float* w, int Hi, int64_t G, float* scores,
                                      int64_t score_stride, const float* c_kv, const float* c_gate, float* c_carry_kv,
                                      float* c_carry_gate, int c_ratio, const void* c_norm_weight, float c_eps,
                                      uint8_t* c_cache, int64_t c_cache_batch_entries, int64_t c_cache_cap,
                                      void* key_half, void* stream) {
  MZK_CHECK_ARG(ratio == kEmitRatio, "decode_emit_scores: the merged launch takes compress ratio 4 (got %d)", ratio);
  MZK_CHECK_ARG(wk && kv_proj && q_idx && w && scores,
                "decode_emit_scores: needs the index key weights, the kv prologue, q_idx, w and scores");
  MZK_CHECK_ARG(key_half != nullptr && aligned16(key_half),
                "decode_emit_scores: key_half (a zeroed, 16-byte aligned [B, %d] int64 buffer) is required",
                kKeyHalfWords);
  EmitSet es;
  int rc = build_emit(positions, B, kv, gate, carry_kv, carry_gate, ratio, norm_weight, eps, cache,
                      cache_batch_entries, cache_cap, wk, k_norm_weight, k_eps, key_format, k_codes, k_scales,
                      key_batch_entries, rope_table, table_rows, step_cos, step_sin, kv_proj, kv_weight, kv_eps,
                      win_cache, win_batch_entries, win_cap, nullptr, 0, nullptr, nullptr, es.fine);
  if (rc) return rc;
  es.fine.key_half = static_cast<uint64_t*>(key_half);
  const bool coarse = c_kv != nullptr;
  if (coarse) {
    rc = build_emit(positions, B, c_kv, c_gate, c_carry_kv, c_carry_gate, c_ratio, c_norm_weight, c_eps, c_cache,
                    c_cache_batch_entries, c_cache_cap, nullptr, nullptr, 0.0f, 0, nullptr, nullptr, 0, rope_table,
                    table_rows, nullptr, nullptr, nullptr, nullptr, 0.0f, nullptr, 0, 0, nullptr, 0, nullptr, nullptr,
                    es.coarse);
    if (rc) return rc;
    MZK_CHECK_ARG(B == 0 || coarse_form(es.coarse),
                  "decode_emit_scores: the coarse branch needs a ratio of 2 .. %d and at most %d rows", kCoarseMaxRatio,
                  kCoarseMaxRows);
  }
  rc = check_common(B, 1, Hi, kDi, G, key_batch_entries, ratio, score_stride);
  if (rc) return rc;
  if (B == 0) return MZK_OK;
  MZK_CHECK_ARG(G >= 1, "decode_emit_scores: at least one key group is required");
  MZK_CHECK_ARG(B <= 65535, "decode_emit_scores: at most 65535 rows (got %lld)", (long long)B);
  MZK_CHECK_ARG(aligned16(q_idx), "decode_emit_scores: q_idx must be 16-byte aligned");
  const bool fp8 = key_format == 0;
  IdxParams p = make_params(nullptr, nullptr, nullptr, w, k_codes, fp8 ? static_cast<const float*>(k_scales) : nullptr,
                            fp8 ? nullptr : static_cast<const uint8_t*>(k_scales), 1, Hi, G, key_batch_entries,
                            positions, ratio, scores, score_stride);
  p.q_raw = static_cast<const uint16_t*>(q_idx);
  p.q_rope_dim = 2 * kRopePairs;
  // Key tiles per wave: the fewest of 4, 8 and 16 (512, 1024, 2048 keys per workgroup) that
  // leave at most one scoring workgroup per compute unit.  The key stream is what a compute
  // unit's time goes to, so the scoring workgroups carry equal shares, one per unit.  The lead
  // workgroups (emission, window entry, coarse parts) come first in the grid: they share
  // units with scoring workgroups, and a group step's emission, dispatched first, has its
  // loads (the key weights) served ahead of its neighbour's key stream.  (Config 2: the 64
  // lead workgroups, then 32 rows x 8 scoring workgroups of 1024 keys on the 256 units.)
  const int lead = 2 + (coarse ? kCoarseParts : 0);
  const int64_t cus = resident_workgroups(1);
  int nkb = 16;
  for (int c : {4, 8}) {
    if (B * ((G + kWaves * 32 * c - 1) / (kWaves * 32 * c)) <= cus) {
      nkb = c;
      break;
    }
  }
  const int64_t nsw = (G + kWaves * 32 * nkb - 1) / (kWaves * 32 * nkb);
  const int64_t nwg = B * (nsw + lead);
  MZK_CHECK_ARG(nwg <= 0x7fffffff, "decode_emit_scores: %lld workgroups exceed the grid limit", (long long)nwg);
  p.rows = B;
  dim3 grid(static_cast<unsigned>(nwg));
  hipStream_t s = as_stream(stream);
#define MZK_EMIT_LAUNCH(F, M, C)                                                                                       \
  do {                                                                                                                \
    if (nkb == 4) indexer_scores_kernel<F, kDi, M, true, false, true, false, true, 4, C><<<grid, kWaves * 64, 0, s>>>(p, es);  \
    else if (nkb == 8) indexer_scores_kernel<F, kDi, M, true, false, true, false, true, 8, C><<<grid, kWaves * 64, 0, s>>>(p, es); \
    else indexer_scores_kernel<F, kDi, M, true, false, true, false, true, 16, C><<<grid, kWaves * 64, 0, s>>>(p, es);  \
  } while (0)
  if (fp8) {
    if (coarse) {
      if (Hi <= 32) MZK_EMIT_LAUNCH(kFp8, 1, true);
      else MZK_EMIT_LAUNCH(kFp8, 2, true);
    } else {
      if (Hi <= 32) MZK_EMIT_LAUNCH(kFp8, 1, false);
      else MZK_EMIT_LAUNCH(kFp8, 2, false);
    }
  } else {
    if (coarse) {
      if (Hi <= 32) MZK_EMIT_LAUNCH(kMxfp4, 1, true);
      else MZK_EMIT_LAUNCH(kMxfp4, 2, true);
    } else {
      if (Hi <= 32) MZK_EMIT_LAUNCH(kMxfp4, 1, false);
      else MZK_EMIT_LAUNCH(kMxfp4, 2, false);
    }
  }
#undef MZK_EMIT_LAUNCH
  MZK_LAUNCH_CHECK("decode_emit_scores");
  return MZK_OK;
}

// ---- two-level selection, level two: the candidate scorer ------------------------------
//
// tickets/0009-indexer-hierarchical.md:29-32 (layers after the candidate source score only
// the candidates; owlet1/indexer.py:150-151 applies it as
// index_scores.masked_fill(~candidates, -inf) before the top-k).  Scores go to the candidate axis, slot j of a row holding key
// cand_blocks[row][j / block_size] * block_size + j % block_size, so the cost follows the
// candidate count, not the key count.  A slot's score has the same bits as the dense row
// kernel's score of its key.

namespace mzk {
namespace {
template <int FMT>
int candidate_scores(const char* name, const IdxParams& base, int64_t B, int64_t S, int Hi, int Di, int64_t G,
                     int64_t kbs, int ratio, const int32_t* cand, int64_t cand_stride, int n_blocks, int block_size,
                     int64_t sstride, hipStream_t s) {
  MZK_CHECK_ARG(B >= 0 && S >= 0 && G >= 0, "%s: negative size", name);
  MZK_CHECK_ARG(Hi >= 1 && Hi <= 64, "%s: index heads must be in [1, 64] (got %d)", name, Hi);
  MZK_CHECK_ARG(ratio >= 1, "%s: compress_ratio must be >= 1 (got %d)", name, ratio);
  MZK_CHECK_ARG(kbs >= G, "%s: key batch stride smaller than G", name);
  int rc = check_candidates(B, S, G, cand, cand_stride, n_blocks, block_size, sstride);
  if (rc) return rc;
  if (B * S == 0 || n_blocks == 0) return MZK_OK;
  MZK_CHECK_ARG(G > 0, "%s: candidates over an empty key cache", name);
  rc = launch_gather<FMT>(with_candidates(base, G, cand, cand_stride, n_blocks, block_size), B * S, Di, s);
  if (rc) return rc;
  MZK_LAUNCH_CHECK(name);
  return MZK_OK;
}
}  // namespace
}  // namespace mzk

extern "C" int mzk_indexer_candidate_scores_fp8(const uint8_t* q_codes, const float* q_scales, const float* w,
                                                const uint8_t* k_codes, const float* k_scales, int64_t B, int64_t S,
                                                int Hi, int Di, int64_t G, int64_t k_batch_stride,
                                                const int64_t* positions, int ratio, const int32_t* cand_blocks,
                                                int64_t cand_stride, int n_blocks, int block_size, float* scores,
                                                int64_t score_stride, void* stream) {
  MZK_CHECK_ARG(B * S == 0 || n_blocks == 0 || (q_codes && q_scales && w && k_codes && k_scales && scores),
                "indexer_candidate_scores_fp8: null pointer");
  return candidate_scores<kFp8>("indexer_candidate_scores_fp8",
                                make_params(q_codes, q_scales, nullptr, w, k_codes, k_scales, nullptr, S, Hi, G,
                                            k_batch_stride, positions, ratio, scores, score_stride),
                                B, S, Hi, Di, G, k_batch_stride, ratio, cand_blocks, cand_stride, n_blocks, block_size,
                                score_stride, as_stream(stream));
}

extern "C" int mzk_indexer_candidate_scores_mxfp4(const uint8_t* q_packed, const uint8_t* q_e8m0, const float* w,
                                                  const uint8_t* k_packed, const uint8_t* k_e8m0, int64_t B, int64_t S,
                                                  int Hi, int Di, int64_t G, int64_t k_batch_stride,
                                                  const int64_t* positions, int ratio, const int32_t* cand_blocks,
                                                  int64_t cand_stride, int n_blocks, int block_size, float* scores,
                                                  int64_t score_stride, void* stream) {
  MZK_CHECK_ARG(B * S == 0 || n_blocks == 0 || (q_packed && q_e8m0 && w && k_packed && k_e8m0 && scores),
                "indexer_candidate_scores_mxfp4: null pointer");
  return candidate_scores<kMxfp4>("indexer_candidate_scores_mxfp4",
                                  make_params(q_packed, nullptr, q_e8m0, w, k_packed, nullptr, k_e8m0, S, Hi, G,
                                              k_batch_stride, positions, ratio, scores, score_stride),
                                  B, S, Hi, Di, G, k_batch_stride, ratio, cand_blocks, cand_stride, n_blocks,
                                  block_size, score_stride, as_stream(stream));
}

extern "C" int mzk_candidate_positions(const int32_t* slot_idx, int64_t rows, int k, int64_t idx_stride,
                                       const int32_t* cand_blocks, int64_t cand_stride, int n_blocks, int block_size,
                                       int32_t* pos_out, int64_t out_stride, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && k >= 0 && n_blocks >= 0 && block_size >= 1 && idx_stride >= k && out_stride >= k &&
                    cand_stride >= n_blocks,
                "candidate_positions: bad sizes");
  MZK_CHECK_ARG(static_cast<int64_t>(n_blocks) * block_size <= (int64_t(1) << 30),
                "candidate_positions: more than 2^30 candidate slots");
  if (rows == 0 || k == 0) return MZK_OK;
  MZK_CHECK_ARG(slot_idx && pos_out && (n_blocks == 0 || cand_blocks), "candidate_positions: null pointer");
  MZK_CHECK_ARG(slot_idx == pos_out ? idx_stride == out_stride : true,
                "candidate_positions: in place needs equal strides");
  const int64_t n = rows * k;
  MZK_CHECK_ARG((n + 255) / 256 <= 0x7fffffff, "candidate_positions: too many entries");
  candidate_positions_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, as_stream(stream)>>>(
      slot_idx, rows, k, idx_stride, cand_blocks, cand_stride, n_blocks, block_size, pos_out, out_stride);
  MZK_LAUNCH_CHECK("candidate_positions");
  return MZK_OK;
}

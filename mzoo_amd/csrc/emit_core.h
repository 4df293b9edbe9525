// Compressed-group emission for one decode token per batch row: the device code shared by
// the emission launch (emit.hip) and the merged emission + scores launch (indexer.hip).
// The per-token work of DeepseekV41Compressor / DeepseekV41CSACache / the indexer's key
// publication / the compressed-cache append (owlet1/cache.py:96-124, :159-172;
// owlet1/indexer.py:96-117; owlet1/attention.py:173-192), with all state on the device so the
// step can be recorded into a graph and replayed with advancing positions.
//
// Per row, every step (one 256-thread workgroup, emit_row):
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
//   * index key (branches with one): k = bf16(latent . wk^T) with a pinned order (8 lanes per
//     output: lane j sums the 16-byte chunks j, j+8, ..., j+64 of the weight row, 8 channels
//     each in order, then the 8 partials meet in an xor butterfly 4, 2, 1), k_norm, RoPE of
//     the trailing 64 channels at g * ratio, quantized (FP8 b128 + fp32 scale, or MXFP4 +
//     e8m0) to key g.
// The step's prologue: the token's window entry (kv_prologue, one wave) and the indexer
// query's RoPE + quantization (query_prologue, kQBlocks workgroups per row).
// Layout constants: latent 512 + 64 (nope + rope), index key 128; bf16 activations.
#pragma once
#include "common.h"

namespace mzk {
namespace {

constexpr int kD = 576;
constexpr int kNope = 512;
constexpr int kRopePairs = 32;  // rope 64
constexpr int kDi = 128;
constexpr int kEntryBytes = kNope + 4 * (kNope / 128) + 2 * 2 * kRopePairs;  // 656
constexpr int kChunks = kD / 8;      // 16-byte chunks of a weight row (72)
constexpr int kLanesPerOut = 8;      // lanes per key output
constexpr int kChunksPerLane = kChunks / kLanesPerOut;  // 9

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
  // the step's prologue (kv_raw null: none), at the token's RoPE (row pos of the table)
  const uint16_t* kv_raw;    // [B, 576] bf16: the wkv projection
  const uint16_t* kv_w;      // [576] bf16: kv_norm weight
  float kv_eps;
  uint8_t* win;              // window ring of FP8-b128 entries, slot b * win_batch + pos % win_cap
  int64_t win_batch;
  int win_cap;
  // MERGED: [B, kKeyHalfWords] the key projection's handoff between the row's two lead
  // workgroups (zero before the first launch); null elsewhere
  uint64_t* key_half;
  const uint16_t* q_idx;     // [B, 64, 128] bf16: the unrotated indexer query (null: none)
  int q_fmt;                 // 0: FP8 b128 -> q_codes [B, 64, 128] + fp32 [B, 64]; 1: MXFP4 -> [B, 64, 64] + e8m0 [B, 64, 4]
  uint8_t* q_codes;
  void* q_scales;
  int64_t B;                 // rows; the workgroups from B on run the prologue
};

// The merged launch splits a group step's key projection (k = latent . wk^T, 128 outputs)
// between the row's emission workgroup (outputs 0..63, then the rest of the key) and its
// window workgroup (outputs 64..127, which it recomputes the pooled latent for): each reads
// half of the 147 KB of key weights.  Handoff record of a row (kKeyHalfWords 64-bit words):
// word 0 the row's epoch (group steps handed over so far), words 1..32 the helper's 64
// outputs as bf16 pairs under the epoch + 1 in the high half, word 33 a flag (nonzero: the
// emission workgroup gave up waiting; it stays set).  Every word is written and read with
// device-scope atomics, so the record needs no fence on any placement of the two.
constexpr int kKeyHalfWords = 40;
constexpr int kKeyHalfSpinLimit = 1 << 20;

constexpr int kQHeads = 64;   // indexer heads
constexpr int kQBlocks = 4;   // query workgroups per row: 16 heads each, 16 threads x 8 channels a head

__device__ __forceinline__ float bf(float v) { return round_to_dtype<MZK_BF16>(v); }

// One RoPE pair (fp32 math, no fused operations, rounded to bf16) -- norm_rope.py:141-145.
__device__ __forceinline__ void rope_pair(float& e, float& o, float c, float s) {
  const float a = e * c - o * s;
  const float b = e * s + o * c;
  e = bf(a);
  o = bf(b);
}

// The indexer query of the step's prologue, in workgroups of its own (their latency
// overlaps the emission's): RoPE of channels 64..127 (owlet1/indexer.py:126-128, the token's
// row of the table), then the query quantizer -- FP8 b128 per head or MXFP4 per 32 channels,
// the operands of the scores launch.  Workgroup B + w: row w / kQBlocks, heads
// 16 (w % kQBlocks) .. +15; thread t: head + t / 16, channels 8 (t % 16) .. +7.
__device__ __forceinline__ void query_prologue(const EmitParams& p, int64_t w, int t) {
  const int64_t b = w / kQBlocks;
  const int64_t pos = p.positions[b];
  if (pos < 0 || pos >= p.tab_rows) return;  // the same rows the emission workgroup skips
  const int h = static_cast<int>(w % kQBlocks) * (kQHeads / kQBlocks) + (t >> 4);
  const int c8 = t & 15;  // channels 8 c8 .. 8 c8 + 7
  const uint4 raw = *reinterpret_cast<const uint4*>(p.q_idx + (b * kQHeads + h) * kDi + 8 * c8);
  // this thread's 4 rope pairs (used for c8 >= 8): pairs 4 (c8 - 8) .. +3
  const uint16_t* trow = p.tab + pos * 2 * kRopePairs;
  const uint2 cr = *reinterpret_cast<const uint2*>(trow + 4 * (c8 & 7));
  const uint2 sr = *reinterpret_cast<const uint2*>(trow + kRopePairs + 4 * (c8 & 7));
  float x[8];
  const uint32_t wq[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    x[2 * k] = __uint_as_float(wq[k] << 16);
    x[2 * k + 1] = __uint_as_float(wq[k] & 0xffff0000u);
  }
  if (c8 >= 8) {
    const uint32_t cw[2] = {cr.x, cr.y}, sw[2] = {sr.x, sr.y};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float c = __uint_as_float((k & 1) ? cw[k >> 1] & 0xffff0000u : cw[k >> 1] << 16);
      const float sn = __uint_as_float((k & 1) ? sw[k >> 1] & 0xffff0000u : sw[k >> 1] << 16);
      rope_pair(x[2 * k], x[2 * k + 1], c, sn);
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = nn_max(amax, fabsf(x[i]));
  const int64_t hrow = b * kQHeads + h;
  if (p.q_fmt == 0) {
    amax = group_max(amax, 16);  // the 16 threads of a head are consecutive lanes
    const float sc = fp8_scale_from_amax(amax);
    // x / sc == x * (1 / sc) exactly: sc is a power of two, in [2^-22, 2^120] for finite input
    const float inv = sc <= 0x1p120f ? pow2_reciprocal(sc) : 1.0f / sc;
    uint32_t wd[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // v_cvt_pk_fp8_f32 is the quantizer's e4m3 encoder for |x| <= 448
      const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(clampf(x[4 * i] * inv, 448.0f),
                                                     clampf(x[4 * i + 1] * inv, 448.0f), 0, false);
      wd[i] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(clampf(x[4 * i + 2] * inv, 448.0f),
                                                                    clampf(x[4 * i + 3] * inv, 448.0f), lo, true));
    }
    *reinterpret_cast<uint2*>(p.q_codes + hrow * kDi + 8 * c8) = uint2{wd[0], wd[1]};
    if (c8 == 0) static_cast<float*>(p.q_scales)[hrow] = sc;
  } else {
    amax = group_max(amax, 4);  // a 32-channel block: 4 consecutive lanes
    const float sc = fp4_scale_from_amax(amax, false);
    // x / sc == x * (1 / sc) exactly: sc is a power of two in [2^-126, 2^127]
    const float inv = sc <= 0x1p126f ? pow2_reciprocal(sc) : 1.0f / sc;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) word |= e2m1_code(clampf(x[j] * inv, 6.0f)) << (4 * j);
    reinterpret_cast<uint32_t*>(p.q_codes + hrow * (kDi / 2))[c8] = word;
    if ((c8 & 3) == 0) static_cast<uint8_t*>(p.q_scales)[hrow * (kDi / 32) + (c8 >> 2)] =
        static_cast<uint8_t>(__float_as_uint(sc) >> 23);
  }
}

// The new token's window entry of the step's prologue, by one wave of a workgroup of its
// own: RMSNorm of the kv projection (owlet1/attention.py:149, norm_rope.py:25-30) in the
// pinned order -- lane l sums channels l, l + 64, ... from 0, then the xor butterfly --, RoPE
// of its rope slice (:150) at the token's row of the table, the FP8-b128 entry (:154) into
// ring slot b * win_batch + pos % win_cap.  Registers and lane exchanges only.
__device__ __forceinline__ void kv_prologue(const EmitParams& p, int64_t b, int lane) {
  const int64_t pos = p.positions[b];
  if (pos < 0 || pos >= p.tab_rows) return;
  constexpr int kKvPer = kD / 64;  // 9: channels lane + 64 i
  uint16_t pkr[kKvPer], pwr[kKvPer];
#pragma unroll
  for (int i = 0; i < kKvPer; ++i) {
    pkr[i] = p.kv_raw[b * kD + lane + 64 * i];
    pwr[i] = p.kv_w[lane + 64 * i];
  }
  const uint16_t* trow = p.tab + pos * 2 * kRopePairs;
  const uint16_t kcr = trow[lane >> 1], ksr = trow[kRopePairs + (lane >> 1)];
  // RMSNorm of the kv projection (owlet1/attention.py:149, norm_rope.py:25-30) in the
  // pinned order -- lane l sums channels l, l + 64, ... from 0, then the xor butterfly --,
  // RoPE of its rope slice (:150), the FP8-b128 window entry (:154)
  float pkv[kKvPer];
#pragma unroll
  for (int i = 0; i < kKvPer; ++i) pkv[i] = bf16_to_f32(pkr[i]);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kKvPer; ++i) ss = ss + pkv[i] * pkv[i];
  ss = ss + lane_xor<32>(ss);
  ss = ss + lane_xor<16>(ss);
  ss = ss + lane_xor<8>(ss);
  ss = ss + lane_xor<4>(ss);
  ss = ss + lane_xor<2>(ss);
  ss = ss + lane_xor<1>(ss);
  const float inv = div_rn(1.0f, sqrt_rn(div_rn(ss, static_cast<float>(kD)) + p.kv_eps));
  float y[kKvPer];
#pragma unroll
  for (int i = 0; i < kKvPer; ++i) y[i] = bf(bf16_to_f32(pwr[i]) * bf(pkv[i] * inv));
  // the rope slice (channels 512 + lane): lane 2j holds the even channel of pair j
  const float partner = lane_xor<1>(y[kKvPer - 1]);
  const bool odd = lane & 1;
  const float e = odd ? partner : y[kKvPer - 1];
  const float o = odd ? y[kKvPer - 1] : partner;
  const float kc_ = bf16_to_f32(kcr), ks_ = bf16_to_f32(ksr);
  const uint16_t rot = f32_to_bf16(odd ? e * ks_ + o * kc_ : e * kc_ - o * ks_);
  uint8_t* went = p.win + (b * p.win_batch + pos % p.win_cap) * kEntryBytes;
  static_assert(kNope / 128 == 4 && kKvPer == 9, "four nope blocks of 128, one rope channel per lane");
  float scs[4], invs[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    scs[k] = fp8_scale_from_amax(wave_max_nonneg(nn_max(fabsf(y[2 * k]), fabsf(y[2 * k + 1]))));
    invs[k] = 1.0f / scs[k];  // exact: a power of two in [2^-22, 2^127]
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // v_cvt_pk_fp8_f32 is the quantizer's e4m3 encoder for |x| <= 448
    const int code = __builtin_amdgcn_cvt_pk_fp8_f32(clampf(y[i] * invs[i >> 1], 448.0f), 0.0f, 0, false);
    went[lane + 64 * i] = static_cast<uint8_t>(code & 0xff);
  }
  if (lane < 4) reinterpret_cast<float*>(went + kNope)[lane] = lane == 0 ? scs[0] : lane == 1 ? scs[1] : lane == 2 ? scs[2] : scs[3];
  reinterpret_cast<uint16_t*>(went + kNope + 4 * (kNope / 128))[lane] = rot;
}

// The token's carry slot (slot pos % ratio of the row's ring, the reference's buffer_kv /
// buffer_gate) for the merged launch, where emit_row<R, true> leaves it: NT threads from
// thread 0, the projections requested with the position.
template <int NT>
__device__ __forceinline__ void carry_slot(const EmitParams& p, int64_t b, int t) {
  static_assert(kD % NT == 0, "whole channels per thread");
  constexpr int kPer = kD / NT;
  const EmitBranch& br = p.br;
  float kin[kPer], gin[kPer];
#pragma unroll
  for (int c = 0; c < kPer; ++c) {
    kin[c] = br.kv[b * kD + t + NT * c];
    gin[c] = br.gate[b * kD + t + NT * c];
  }
  const int64_t pos = p.positions[b];
  if (pos < 0) return;  // an inactive row: nothing to carry
  const int r = br.ratio;
  float* ckv = br.carry_kv + (b * r + pos % r) * static_cast<int64_t>(kD);
  float* cgt = br.carry_gate + (b * r + pos % r) * static_cast<int64_t>(kD);
#pragma unroll
  for (int c = 0; c < kPer; ++c) {
    ckv[t + NT * c] = kin[c];
    cgt[t + NT * c] = gin[c];
  }
}

// R > 0: the ratio is R (the group stays in registers); R == 0: any ratio (br.ratio).
// The carry / group work of row b (all threads of a 256-thread workgroup, uniform control
// flow).  Returns whether the step emitted the row's index key (group g = (pos + 1) / r - 1);
// with `key_out` (16-byte aligned LDS) the key's operand bytes are also left there for the
// caller, after the workgroup's next barrier: FP8 -- 128 codes, then the fp32 scale at byte
// 128; MXFP4 -- 64 bytes of e2m1 pairs, then the 4 e8m0 bytes at byte 64.
// MERGED (the merged emission + scores launch, R > 1): the token's carry slot and the step's
// RoPE tables are written by other workgroups of that launch (carry_slot, the row's first
// scoring workgroup), so a step that completes no group ends as soon as the position is
// known.  ROLE (MERGED): 1 the emission workgroup (key outputs 0..63, the rest from the
// handoff), 2 the window workgroup's half (the pooled latent, key outputs 64..127 to the
// handoff; no entry, no key; returns false).
template <int R, bool MERGED = false, int ROLE = 0>
__device__ __forceinline__ bool emit_row(const EmitParams& p, int64_t b, uint8_t* key_out) {
  static_assert(!MERGED || R > 1, "the merged form keeps the group in registers");
  static_assert(ROLE == 0 || MERGED, "the key split is the merged launch's");
  constexpr int NPS = ROLE ? 2 : 4;         // key-output passes of 8 per wave
  constexpr int OBASE = ROLE == 2 ? 64 : 0;  // this workgroup's first key output
  __shared__ float lat[kD];
  __shared__ float kvec[kDi];
  __shared__ float inv_s[2];
  const int t = threadIdx.x;
  const EmitBranch& br = p.br;
  const float* kvb = br.kv + b * kD;
  const float* gtb = br.gate + b * kD;

  // ---- every load the step needs, issued before any of them is waited on ----------------
  // Loads are unconditional from always-valid addresses (clamped indices, a stand-in
  // pointer when an operand is absent) or, for the large optional operands, sit in a
  // workgroup-uniform branch into uninitialised registers; bf16 values stay raw until their
  // use.  A `cond ? convert(load) : 0` form puts each load with a wait for it into a branch
  // of its own: one memory round trip per load.  The operands that do not depend on the
  // row's position -- the token's projections, the norm weight and (R > 1) the carried
  // slots 0 .. R - 2, which a completing step pools -- are requested with the position, so a
  // group step pays one round trip for them, not two (the carried slots cost 14 KB a row on
  // the steps that do not pool them).
  // this thread's channels: t, t + 256, t + 512 (the last only for t < 64; clamped)
  constexpr int kCh = 3;
  constexpr int kRegR = R > 1 ? R - 1 : 1;  // carried slots held in registers (R > 1)
  float kin[kCh], gin[kCh] = {};
  uint16_t nwr[kCh];
  float ck[kRegR][kCh], cg[kRegR][kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) kin[c] = kvb[min(t + 256 * c, kD - 1)];
  if (R != 1 && (R > 1 || br.ratio > 1)) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) gin[c] = gtb[min(t + 256 * c, kD - 1)];
  }
#pragma unroll
  for (int c = 0; c < kCh; ++c) nwr[c] = br.norm_w[min(t + 256 * c, kD - 1)];
  if constexpr (R > 1) {
    const float* ckv0 = br.carry_kv + b * static_cast<int64_t>(R) * kD;
    const float* cgt0 = br.carry_gate + b * static_cast<int64_t>(R) * kD;
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int d = min(t + 256 * c, kD - 1);
#pragma unroll
      for (int i = 0; i < R - 1; ++i) {
        ck[i][c] = ckv0[i * kD + d];
        cg[i][c] = cgt0[i * kD + d];
      }
    }
  }
  // MERGED: the position through the scalar cache (no vector-memory write in the launch
  // touches it), so it arrives within one round trip instead of behind the operands above
  // (a vector load completes after every load issued before it: 4 us into a config-2 group
  // step, which held back the key weights' requests below)
  typedef const __attribute__((address_space(4))) int64_t* scalar_i64_ptr;
  const int64_t pos = MERGED ? *(scalar_i64_ptr)(p.positions + b) : p.positions[b];
  if (pos < 0) return false;  // an inactive row: nothing to carry or emit
  const int r = R > 0 ? R : br.ratio;
  const int slot = static_cast<int>(pos % r);
  const bool completes = (pos + 1) % r == 0;  // uniform over the workgroup
  const int64_t g = (pos + 1) / r - 1;
  const int64_t gp = g * r;  // the group's position (its first token)
  const bool emit = completes && g < br.cache_cap && gp < p.tab_rows;
  const bool key = emit && br.wk != nullptr;
  float* ckv = br.carry_kv + b * static_cast<int64_t>(r) * kD;
  float* cgt = br.carry_gate + b * static_cast<int64_t>(r) * kD;
  if (MERGED && !emit) return false;  // uniform: the carry slot is another workgroup's
  // ROLE: the row's handoff record and the epoch this step hands over under
  uint64_t* kh = ROLE ? p.key_half + b * kKeyHalfWords : nullptr;
  uint32_t epoch = 0;
  if constexpr (ROLE != 0) {
    if (t == 0) inv_s[1] = __uint_as_float(static_cast<uint32_t>(
                    __hip_atomic_load(kh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + 1u);
  }
  // key weights: lane j of each 8-lane group reads chunks j, j+8, ... of its output's row,
  // so one load instruction covers 8 rows x 128 contiguous bytes; a wave serves 8 outputs
  // per pass, 4 passes (outputs 32 w + 8 pass + lane / 8), or with ROLE 2 passes over the
  // workgroup's half (OBASE + 16 w + 8 pass + lane / 8)
  const int lane = t & 63, wv = t >> 6;
  const int j8 = lane & (kLanesPerOut - 1);
  // key output of pass ps of this lane (8 lanes per output)
  auto out_of = [&](int ps) __attribute__((always_inline)) {
    return OBASE + (ROLE ? 16 : 32) * wv + 8 * ps + (lane >> 3);
  };
  uint4 wreg[NPS][kChunksPerLane];
  auto load_wk = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
      const int o = out_of(ps);
      const uint4* wrow = reinterpret_cast<const uint4*>(br.wk + static_cast<int64_t>(o) * kD);
#pragma unroll
      for (int c = 0; c < kChunksPerLane; ++c) wreg[ps][c] = wrow[j8 + kLanesPerOut * c];
    }
  };
  if constexpr (!MERGED) {
    if (key) load_wk();
  }
  const uint16_t knr = (key ? br.kn_w : br.norm_w)[t & (kDi - 1)];
  // the group's RoPE pair (t & 31): threads 128..159 rotate the latent, 0..31 the key
  const int64_t last_row = p.tab_rows - 1;
  const uint16_t* tg = p.tab + min(max(gp, int64_t{0}), last_row) * 2 * kRopePairs;
  const uint16_t gcr = tg[t & 31], gsr = tg[kRopePairs + (t & 31)];
  // the token's row: the step's tables and the prologue's RoPE
  const uint16_t* trow = p.tab + min(pos, last_row) * 2 * kRopePairs;
  const bool step_tab = p.step_cos && pos < p.tab_rows;  // uniform
  const uint16_t stab = trow[t & 63];
  // MERGED (whose launch always has the key weights, and here a step that emits): the 147 KB
  // of key weights are requested last and outside any branch, so the pooling and the entry
  // wait only for their own operands (loads complete in order, and a load inside a branch
  // would make the waits after it count as if every later load were outstanding: the
  // pooling then waited for the weights, 8.4 us into a config-2 group step)
  if constexpr (MERGED) load_wk();

  // ---- the token into its carry slot; the step's RoPE tables --------------------------
  if constexpr (!MERGED) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int d = t + 256 * c;
      if (d < kD) {
        ckv[slot * kD + d] = kin[c];
        if (r > 1) cgt[slot * kD + d] = gin[c];
      }
    }
    if (step_tab && t < 2 * kRopePairs) {
      if (t < kRopePairs) p.step_cos[b * kRopePairs + t] = stab;
      else p.step_sin[b * kRopePairs + (t - kRopePairs)] = stab;
    }
  }
  if (!emit) return false;  // uniform over the workgroup
  float nw[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) nw[c] = bf16_to_f32(nwr[c]);
  const float gc = bf16_to_f32(gcr), gs = bf16_to_f32(gsr);

  // ---- pool (slot r - 1 is this token) -> bf16 -------------------------------------------
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int d = t + 256 * c;
    if (d >= kD) continue;
    float v;
    if (r == 1) {
      v = kin[c];
    } else if constexpr (R > 1) {
      float m = cg[0][c];
#pragma unroll
      for (int i = 1; i < R; ++i) m = fmaxf(m, i == R - 1 ? gin[c] : cg[i][c]);
      float e[R];
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        e[i] = exp_pinned((i == R - 1 ? gin[c] : cg[i][c]) - m);
        s = s + e[i];
      }
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < R; ++i) acc = acc + (i == R - 1 ? kin[c] : ck[i][c]) * div_rn(e[i], s);
      v = acc;
    } else {
      // the carried slots stream through registers kSB at a time: a batch's loads are all
      // issued before the first is used (clamped to slot r-2; slot r-1 is this token, still
      // in registers), so a pass over r slots costs r / kSB memory round trips, not r; the
      // arithmetic is the pinned order (max, the sum of exps from slot 0, the weighted sum
      // from slot 0)
      constexpr int kSB = 32;
      float m = -__builtin_huge_valf();
      for (int i0 = 0; i0 < r; i0 += kSB) {
        float gv[kSB];
#pragma unroll
        for (int ii = 0; ii < kSB; ++ii) gv[ii] = cgt[min(i0 + ii, r - 2) * kD + d];
#pragma unroll
        for (int ii = 0; ii < kSB; ++ii) {
          const int i = i0 + ii;
          if (i < r) m = fmaxf(m, i == r - 1 ? gin[c] : gv[ii]);
        }
      }
      float s = 0.0f;
      for (int i0 = 0; i0 < r; i0 += kSB) {
        float gv[kSB];
#pragma unroll
        for (int ii = 0; ii < kSB; ++ii) gv[ii] = cgt[min(i0 + ii, r - 2) * kD + d];
#pragma unroll
        for (int ii = 0; ii < kSB; ++ii) {
          const int i = i0 + ii;
          if (i < r) s = s + exp_pinned((i == r - 1 ? gin[c] : gv[ii]) - m);
        }
      }
      float acc = 0.0f;
      for (int i0 = 0; i0 < r; i0 += kSB / 2) {
        float gv[kSB / 2], kv[kSB / 2];
#pragma unroll
        for (int ii = 0; ii < kSB / 2; ++ii) {
          const int i = min(i0 + ii, r - 2);
          gv[ii] = cgt[i * kD + d];
          kv[ii] = ckv[i * kD + d];
        }
#pragma unroll
        for (int ii = 0; ii < kSB / 2; ++ii) {
          const int i = i0 + ii;
          if (i < r) {
            const float e = exp_pinned((i == r - 1 ? gin[c] : gv[ii]) - m);
            acc = acc + (i == r - 1 ? kin[c] : kv[ii]) * div_rn(e, s);
          }
        }
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
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int d = t + 256 * c;
      if (d < kD) lat[d] = bf(nw[c] * bf(lat[d] * inv));
    }
  }
  __syncthreads();
  if constexpr (ROLE != 0) epoch = __float_as_uint(inv_s[1]);  // written before the barriers above

  // ---- the main cache entry: FP8-b128 nope blocks + rotated bf16 rope channels
  uint8_t* ent = br.cache + (b * br.cache_batch + g) * kEntryBytes;
  if (ROLE == 2) {
    // the window workgroup's half: no entry
  } else if (t < kNope / 4) {
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
    rope_pair(e, o, gc, gs);
    uint16_t* rp = reinterpret_cast<uint16_t*>(ent + kNope + 4 * (kNope / 128));
    rp[2 * i] = f32_to_bf16(e);
    rp[2 * i + 1] = f32_to_bf16(o);
  }
  if (!key) return false;

  // ---- the index key: k = bf16(latent . wk^T), pinned 8-lane order
#pragma unroll
  for (int ps = 0; ps < NPS; ++ps) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunksPerLane; ++c) {
      const uint4 w8 = wreg[ps][c];
      const uint32_t ws[4] = {w8.x, w8.y, w8.z, w8.w};
      const int i0 = 8 * (j8 + kLanesPerOut * c);
      // a bf16 x bf16 product is exact in fp32, so the fused multiply-add rounds exactly as
      // the product-then-sum does
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = __builtin_fmaf(lat[i0 + 2 * j], __uint_as_float(ws[j] << 16), acc);
        acc = __builtin_fmaf(lat[i0 + 2 * j + 1], __uint_as_float(ws[j] & 0xffff0000u), acc);
      }
    }
    acc = acc + lane_xor<4>(acc);
    acc = acc + lane_xor<2>(acc);
    acc = acc + lane_xor<1>(acc);
    if (j8 == 0) kvec[out_of(ps)] = bf(acc);
  }
  __syncthreads();
  if constexpr (ROLE == 2) {
    // outputs 64..127 to the handoff: lane l of wave 0 sends outputs 64 + 2l, 65 + 2l
    if (t < 32) {
      const uint32_t pair = static_cast<uint32_t>(f32_to_bf16(kvec[64 + 2 * t])) |
                            (static_cast<uint32_t>(f32_to_bf16(kvec[65 + 2 * t])) << 16);
      __hip_atomic_store(kh + 1 + t, (static_cast<uint64_t>(epoch) << 32) | pair, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    return false;
  }
  if constexpr (ROLE == 1) {
    // outputs 64..127 from the window workgroup: lane l of wave 0 polls its pair's word
    // until it carries this step's epoch (bounded: after kKeyHalfSpinLimit polls the flag
    // is set and the key is written from zeros)
    if (t < 64) {
      uint64_t w = 0;
      bool have = true;
      if (t < 32) {
        w = __hip_atomic_load(kh + 1 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        have = static_cast<uint32_t>(w >> 32) == epoch;
      }
      for (int it = 0; !__all(have) && it < kKeyHalfSpinLimit; ++it) {
        __builtin_amdgcn_s_sleep(1);
        if (!have) {
          w = __hip_atomic_load(kh + 1 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          have = static_cast<uint32_t>(w >> 32) == epoch;
        }
      }
      const bool all = __all(have);
      if (t < 32) {
        const uint32_t pair = all ? static_cast<uint32_t>(w) : 0u;
        kvec[64 + 2 * t] = bf16_to_f32(static_cast<uint16_t>(pair & 0xffffu));
        kvec[65 + 2 * t] = bf16_to_f32(static_cast<uint16_t>(pair >> 16));
      }
      if (t == 0) {
        __hip_atomic_store(kh, static_cast<uint64_t>(epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!all) __hip_atomic_store(kh + 33, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
  }
  if (t < 64) {  // k_norm: lane l sums channels l, l + 64
    float ss = 0.0f;
    ss = ss + kvec[t] * kvec[t];
    ss = ss + kvec[t + 64] * kvec[t + 64];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss = ss + __shfl_xor(ss, m, 64);
    if (t == 0) inv_s[1] = div_rn(1.0f, sqrt_rn(div_rn(ss, static_cast<float>(kDi)) + br.k_eps));
  }
  __syncthreads();
  if (t < kDi) kvec[t] = bf(bf16_to_f32(knr) * bf(kvec[t] * inv_s[1]));
  __syncthreads();
  if (t < kRopePairs) {  // RoPE of channels 64..127
    float e = kvec[kDi - 2 * kRopePairs + 2 * t], o = kvec[kDi - 2 * kRopePairs + 2 * t + 1];
    rope_pair(e, o, gc, gs);
    kvec[kDi - 2 * kRopePairs + 2 * t] = e;
    kvec[kDi - 2 * kRopePairs + 2 * t + 1] = o;
  }
  __syncthreads();
  if (t < kDi / 4) {  // wave 0, lanes 0..31: four channels each
    float v[4] = {kvec[4 * t], kvec[4 * t + 1], kvec[4 * t + 2], kvec[4 * t + 3]};
    float amax = abs_max4(v);
    const int64_t kidx = b * br.key_batch + g;
    if (br.key_fmt == 0) {
      amax = wave_max_group(amax, 32);
      const float sc = fp8_scale_from_amax(amax);
      uint32_t word = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) word |= static_cast<uint32_t>(e4m3_encode(clampf(div_rn(v[i], sc), 448.0f))) << (8 * i);
      reinterpret_cast<uint32_t*>(br.k_codes + kidx * kDi)[t] = word;
      if (t == 0) static_cast<float*>(br.k_scales)[kidx] = sc;
      if (key_out) {
        reinterpret_cast<uint32_t*>(key_out)[t] = word;
        if (t == 0) *reinterpret_cast<float*>(key_out + kDi) = sc;
      }
    } else {
      amax = wave_max_group(amax, 8);
      const float sc = fp4_scale_from_amax(amax, false);
      uint32_t c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = e2m1_code(clampf(div_rn(v[i], sc), 6.0f));
      const uint16_t code = static_cast<uint16_t>(c[0] | (c[1] << 4) | (c[2] << 8) | (c[3] << 12));
      const uint8_t e8 = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
      reinterpret_cast<uint16_t*>(br.k_codes + kidx * (kDi / 2))[t] = code;
      if ((t & 7) == 0) static_cast<uint8_t*>(br.k_scales)[kidx * (kDi / 32) + (t >> 3)] = e8;
      if (key_out) {
        reinterpret_cast<uint16_t*>(key_out)[t] = code;
        if ((t & 7) == 0) key_out[kDi / 2 + (t >> 3)] = e8;
      }
    }
  }
  return true;
}

// Workgroup `blk` of an emission launch (emit_kernel, or the first workgroups of
// emit_pair_kernel): rows first, then the step's prologue workgroups.
template <int R>
__device__ __forceinline__ void emit_body(const EmitParams& p, int64_t blk) {
  const int t = threadIdx.x;
  if (blk >= p.B) {  // uniform: a prologue workgroup
    // per row: kQBlocks query workgroups (with a query), then one for the window entry
    const int nq = p.q_idx ? kQBlocks : 0;
    const int64_t w = blk - p.B;
    const int64_t row = w / (nq + 1), k = w % (nq + 1);
    if (k < nq) query_prologue(p, row * kQBlocks + k, t);
    else if (t < 64) kv_prologue(p, row, t);
    return;
  }
  emit_row<R>(p, blk, nullptr);
}


// ---- a long-ratio branch without an index key (the coarse branch), its group step
// spread over workgroups ------------------------------------------------------------------
// Pooling r carried slots of 576 channels in the pinned order (the running max, the sum of
// exps from slot 0, the weighted sum from slot 0) is an exp, a correctly rounded divide and
// a few more operations per (slot, channel): at r = 128, one workgroup per row spent ~130 us
// on it.  Here kCoarseParts workgroups per row take 64 channels each.  In a part, four
// threads per channel compute the exps and the weighted terms of a quarter of the slots
// each, and one thread per channel adds them up in slot order over LDS, so every sum keeps
// the pinned order and the latent its bits.  Each part writes its pooled channels into the
// token's own carry slot r - 1 (whose inputs it has used), makes them visible device-wide
// and counts itself in on the row's arrival counter; the last part to arrive reads the whole
// latent back, finishes the group (norm, the FP8-b128 entry with its rope channels rotated
// at the group's position) and resets the counter.  Steps that complete no group only write
// their 64 channels of the carry slot.  Launches that overlap on one GPU would share the
// counters: the decode step issues them in stream order.
constexpr int kCoarseParts = kD / 64;      // 9 parts of 64 channels
constexpr int kCoarseMaxRatio = 128;       // slots held in LDS
constexpr int kCoarseMaxRows = 1024;
// zero at load; every group step leaves it zero.  One array per translation unit that
// includes this header: each is used only by that unit's kernels.
__device__ unsigned g_coarse_arrivals[kCoarseMaxRows];

// Workgroup `blk` = row * kCoarseParts + part of a coarse branch (coarse_emit_kernel, the
// workgroups after the fine branch's in emit_pair_kernel, or those of the merged indexer
// launch).
__device__ __forceinline__ void coarse_body(const EmitParams& p, int64_t blk) {
  __shared__ float ev[kCoarseMaxRatio][64];  // a part's gates, then exps, then weighted terms
  __shared__ float pmax[4][64];
  __shared__ float psum[64];
  __shared__ float lat[kD];
  __shared__ float inv_s;
  __shared__ int last;
  const int t = threadIdx.x;
  const int64_t b = blk / kCoarseParts;
  const int part = static_cast<int>(blk % kCoarseParts);
  const EmitBranch& br = p.br;
  const int c = t & 63, k = t >> 6;  // channel of the part, quarter of the slots
  const int d = 64 * part + c;
  // the token's projections are requested with the position (one round trip, not two)
  const float kin = br.kv[b * kD + d], gin = br.gate[b * kD + d];
  const int64_t pos = p.positions[b];
  if (pos < 0) return;  // an inactive row: nothing to carry or emit
  const int r = br.ratio;  // 2 .. kCoarseMaxRatio (host check)
  const int slot = static_cast<int>(pos % r);
  const bool completes = (pos + 1) % r == 0;
  const int64_t g = (pos + 1) / r - 1;
  const int64_t gp = g * r;
  const bool emit = completes && g < br.cache_cap && gp < p.tab_rows;
  float* ckv = br.carry_kv + b * static_cast<int64_t>(r) * kD;
  float* cgt = br.carry_gate + b * static_cast<int64_t>(r) * kD;
  if (k == 0) {
    ckv[slot * kD + d] = kin;
    cgt[slot * kD + d] = gin;
  }
  if (!emit) return;  // uniform over the workgroup

  // the quarter's gates (slot r - 1 is this token, in registers) into LDS, and their max;
  // every load of a pass is issued before the first is used (indices clamped to slot r - 2),
  // so a pass costs one memory round trip
  constexpr int kQ = kCoarseMaxRatio / 4;
  const int q = (r + 3) / 4, i0 = k * q, i1 = min(i0 + q, r);
  float m = -__builtin_huge_valf();
  {
    float gv[kQ];
#pragma unroll
    for (int j = 0; j < kQ; ++j) gv[j] = cgt[min(i0 + j, r - 2) * kD + d];
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      const int i = i0 + j;
      if (i < i1) {
        const float x = i == r - 1 ? gin : gv[j];
        ev[i][c] = x;
        m = fmaxf(m, x);
      }
    }
  }
  pmax[k][c] = m;
  __syncthreads();
  // the max ignores the order of its operands
  m = fmaxf(fmaxf(pmax[0][c], pmax[1][c]), fmaxf(pmax[2][c], pmax[3][c]));
  for (int i = i0; i < i1; ++i) ev[i][c] = exp_pinned(ev[i][c] - m);
  __syncthreads();
  if (k == 0) {  // the sum of exps from slot 0
    float s = 0.0f;
    for (int i = 0; i < r; ++i) s = s + ev[i][c];
    psum[c] = s;
  }
  __syncthreads();
  const float s = psum[c];
  {
    float kvv[kQ];
#pragma unroll
    for (int j = 0; j < kQ; ++j) kvv[j] = ckv[min(i0 + j, r - 2) * kD + d];
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      const int i = i0 + j;
      if (i < i1) ev[i][c] = (i == r - 1 ? kin : kvv[j]) * div_rn(ev[i][c], s);
    }
  }
  __syncthreads();
  if (k == 0) {  // the weighted sum from slot 0, rounded to bf16 (latent.to(dtype))
    float acc = 0.0f;
    for (int i = 0; i < r; ++i) acc = acc + ev[i][c];
    cgt[(r - 1) * kD + d] = bf(acc);
  }
  __threadfence();  // this part's channels are visible device-wide before it counts itself in
  __syncthreads();
  if (t == 0) last = atomicAdd(&g_coarse_arrivals[b], 1u) == kCoarseParts - 1;
  __syncthreads();
  if (!last) return;  // uniform
  __threadfence();  // the other parts' channels
  if (t == 0) g_coarse_arrivals[b] = 0u;
  for (int dd = t; dd < kD; dd += 256) lat[dd] = cgt[(r - 1) * kD + dd];
  __syncthreads();

  // ---- RMSNorm of the latent (wave 0, pinned order), as emit_kernel
  if (t < 64) {
    float ss = 0.0f;
    for (int dd = t; dd < kD; dd += 64) ss = ss + lat[dd] * lat[dd];
#pragma unroll
    for (int mm = 32; mm >= 1; mm >>= 1) ss = ss + __shfl_xor(ss, mm, 64);
    if (t == 0) inv_s = div_rn(1.0f, sqrt_rn(div_rn(ss, static_cast<float>(kD)) + br.eps));
  }
  __syncthreads();
  {
    const float inv = inv_s;
    for (int dd = t; dd < kD; dd += 256) lat[dd] = bf(bf16_to_f32(br.norm_w[dd]) * bf(lat[dd] * inv));
  }
  __syncthreads();
  // ---- the entry: FP8-b128 nope blocks + the rope channels rotated at the group's position
  const int64_t last_row = p.tab_rows - 1;
  const uint16_t* tg = p.tab + min(max(gp, int64_t{0}), last_row) * 2 * kRopePairs;
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
}

// ---- host side ------------------------------------------------------------------------

// The checked parameters of one emission launch (mzk_decode_emit's contract).
int build_emit(const int64_t* positions, int64_t B, const float* kv, const float* gate,
               float* carry_kv, float* carry_gate, int ratio, const void* norm_weight, float eps,
               uint8_t* cache, int64_t cache_batch_entries, int64_t cache_cap, const void* wk,
               const void* k_norm_weight, float k_eps, int key_format, uint8_t* k_codes,
               void* k_scales, int64_t key_batch_entries, const void* rope_table, int64_t table_rows,
               void* step_cos, void* step_sin, const void* kv_proj, const void* kv_weight, float kv_eps,
               uint8_t* win_cache, int64_t win_batch_entries, int win_cap, const void* q_idx,
               int q_format, uint8_t* q_codes, void* q_scales, EmitParams& p) {
  MZK_CHECK_ARG(B >= 0 && B <= 0x7fffffff, "decode_emit: bad B");
  MZK_CHECK_ARG(ratio >= 1 && ratio <= 1024, "decode_emit: ratio %d not in [1, 1024]", ratio);
  if (B == 0) return MZK_OK;  // nothing to launch (the caller checks B too)
  MZK_CHECK_ARG(positions && kv && carry_kv && norm_weight && cache && rope_table && (ratio == 1 || (gate && carry_gate)),
                "decode_emit: null pointer");
  MZK_CHECK_ARG(table_rows >= 1, "decode_emit: empty RoPE table");
  MZK_CHECK_ARG((step_cos == nullptr) == (step_sin == nullptr), "decode_emit: step cos and sin go together");
  MZK_CHECK_ARG(aligned16(cache) && cache_cap >= 0 && cache_batch_entries >= cache_cap,
                "decode_emit: the cache must be 16-byte aligned with cache_batch_entries >= cache_cap");
  p = EmitParams{};
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
  if (kv_proj) {
    MZK_CHECK_ARG(kv_weight && win_cache && win_cap >= 1 && win_batch_entries >= win_cap && aligned16(win_cache),
                  "decode_emit: the kv prologue needs kv_weight and a 16-byte aligned window ring");
    MZK_CHECK_ARG(!q_idx || (q_codes && q_scales && (q_format == 0 || q_format == 1) && aligned16(q_idx) &&
                             aligned16(q_codes)),
                  "decode_emit: the query prologue needs 16-byte aligned q_idx / q_codes, q_scales and q_format 0 / 1");
    MZK_CHECK_ARG(aligned16(rope_table), "decode_emit: the RoPE table must be 16-byte aligned");
    MZK_CHECK_ARG(B <= 0x7fffffff / (2 + kQBlocks), "decode_emit: B too large for the prologue");
    p.kv_raw = static_cast<const uint16_t*>(kv_proj);
    p.kv_w = static_cast<const uint16_t*>(kv_weight);
    p.kv_eps = kv_eps;
    p.win = win_cache;
    p.win_batch = win_batch_entries;
    p.win_cap = win_cap;
    p.q_idx = static_cast<const uint16_t*>(q_idx);
    p.q_fmt = q_format;
    p.q_codes = q_codes;
    p.q_scales = q_scales;
  } else {
    MZK_CHECK_ARG(q_idx == nullptr, "decode_emit: the query prologue comes with the kv prologue");
  }
  p.B = B;
  return MZK_OK;
}


// The coarse kernel's branch: a ratio of 2 .. kCoarseMaxRatio without key, prologue or step tables.
bool coarse_form(const EmitParams& p) {
  return p.br.ratio >= 2 && p.br.ratio <= kCoarseMaxRatio && !p.br.wk && !p.kv_raw && !p.step_cos &&
         p.B <= kCoarseMaxRows;
}

}  // namespace
}  // namespace mzk

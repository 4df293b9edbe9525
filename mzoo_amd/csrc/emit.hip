// Compressed-group emission inside the decode step (the device code: emit_core.h).
//
// One workgroup (256 threads) per batch row, one launch per compressed branch (or both
// branches in one, emit_pair_kernel).  With the step's prologue, further workgroups per row
// (after the B emission workgroups) write the token's window entry (one) and rotate +
// quantize the indexer query (kQBlocks): their latency overlaps the emission's.
#include "emit_core.h"

namespace mzk {
namespace {

template <int R>
__global__ void __launch_bounds__(256) emit_kernel(EmitParams p) {
  emit_body<R>(p, blockIdx.x);
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
__device__ unsigned g_coarse_arrivals[kCoarseMaxRows];  // zero at load; every group step leaves it zero

// Workgroup `blk` of a coarse-branch launch (coarse_emit_kernel, or the workgroups after the
// fine branch's in emit_pair_kernel).
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
  const int64_t pos = p.positions[b];
  if (pos < 0) return;  // an inactive row: nothing to carry or emit
  const int r = br.ratio;  // 2 .. kCoarseMaxRatio (host check)
  const int slot = static_cast<int>(pos % r);
  const bool completes = (pos + 1) % r == 0;
  const int64_t g = (pos + 1) / r - 1;
  const int64_t gp = g * r;
  const bool emit = completes && g < br.cache_cap && gp < p.tab_rows;
  const int c = t & 63, k = t >> 6;  // channel of the part, quarter of the slots
  const int d = 64 * part + c;
  float* ckv = br.carry_kv + b * static_cast<int64_t>(r) * kD;
  float* cgt = br.carry_gate + b * static_cast<int64_t>(r) * kD;
  const float kin = br.kv[b * kD + d], gin = br.gate[b * kD + d];
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

__global__ void __launch_bounds__(256) coarse_emit_kernel(EmitParams p) { coarse_body(p, blockIdx.x); }

// Both branches of a hierarchical step in one launch: workgroups [0, nfine) are the fine
// (ratio-4) branch's emit_kernel<4> launch with its prologue, the rest the coarse branch's
// coarse_emit_kernel launch -- the same work, one launch instead of two.
__global__ void __launch_bounds__(256) emit_pair_kernel(EmitParams pf, EmitParams pc, unsigned nfine) {
  if (blockIdx.x < nfine) emit_body<4>(pf, blockIdx.x);
  else coarse_body(pc, static_cast<int64_t>(blockIdx.x) - nfine);
}

// The workgroups of an emission launch (its rows, and the prologue's per row).
unsigned emit_grid(const EmitParams& p) {
  return static_cast<unsigned>(p.B * (p.kv_raw ? (p.q_idx ? 2 + kQBlocks : 2) : 1));
}

// The coarse kernel's branch: a ratio of 2 .. kCoarseMaxRatio without key, prologue or step tables.
bool coarse_form(const EmitParams& p) {
  return p.br.ratio >= 2 && p.br.ratio <= kCoarseMaxRatio && !p.br.wk && !p.kv_raw && !p.step_cos &&
         p.B <= kCoarseMaxRows;
}

int launch_emit(const EmitParams& p, void* stream) {
  if (p.br.ratio == 4) {
    emit_kernel<4><<<emit_grid(p), 256, 0, as_stream(stream)>>>(p);
  } else if (coarse_form(p)) {
    coarse_emit_kernel<<<static_cast<unsigned>(p.B * kCoarseParts), 256, 0, as_stream(stream)>>>(p);
  } else {
    emit_kernel<0><<<emit_grid(p), 256, 0, as_stream(stream)>>>(p);
  }
  MZK_LAUNCH_CHECK("decode_emit");
  return MZK_OK;
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_decode_emit(const int64_t* positions, int64_t B, const float* kv, const float* gate,
                               float* carry_kv, float* carry_gate, int ratio, const void* norm_weight, float eps,
                               uint8_t* cache, int64_t cache_batch_entries, int64_t cache_cap, const void* wk,
                               const void* k_norm_weight, float k_eps, int key_format, uint8_t* k_codes,
                               void* k_scales, int64_t key_batch_entries, const void* rope_table, int64_t table_rows,
                               void* step_cos, void* step_sin, const void* kv_proj, const void* kv_weight, float kv_eps,
                               uint8_t* win_cache, int64_t win_batch_entries, int win_cap, const void* q_idx,
                               int q_format, uint8_t* q_codes, void* q_scales, void* stream) {
  EmitParams p;
  const int rc = build_emit(positions, B, kv, gate, carry_kv, carry_gate, ratio, norm_weight, eps, cache,
                            cache_batch_entries, cache_cap, wk, k_norm_weight, k_eps, key_format, k_codes, k_scales,
                            key_batch_entries, rope_table, table_rows, step_cos, step_sin, kv_proj, kv_weight, kv_eps,
                            win_cache, win_batch_entries, win_cap, q_idx, q_format, q_codes, q_scales, p);
  if (rc || B == 0) return rc;
  return launch_emit(p, stream);
}

extern "C" int mzk_decode_emit_pair(const int64_t* positions, int64_t B, const float* kv, const float* gate,
                                    float* carry_kv, float* carry_gate, int ratio, const void* norm_weight, float eps,
                                    uint8_t* cache, int64_t cache_batch_entries, int64_t cache_cap, const void* wk,
                                    const void* k_norm_weight, float k_eps, int key_format, uint8_t* k_codes,
                                    void* k_scales, int64_t key_batch_entries, const void* rope_table,
                                    int64_t table_rows, void* step_cos, void* step_sin, const void* kv_proj,
                                    const void* kv_weight, float kv_eps, uint8_t* win_cache, int64_t win_batch_entries,
                                    int win_cap, const void* q_idx, int q_format, uint8_t* q_codes, void* q_scales,
                                    const float* c_kv, const float* c_gate, float* c_carry_kv, float* c_carry_gate,
                                    int c_ratio, const void* c_norm_weight, float c_eps, uint8_t* c_cache,
                                    int64_t c_cache_batch_entries, int64_t c_cache_cap, void* stream) {
  EmitParams pf, pc;
  int rc = build_emit(positions, B, kv, gate, carry_kv, carry_gate, ratio, norm_weight, eps, cache,
                      cache_batch_entries, cache_cap, wk, k_norm_weight, k_eps, key_format, k_codes, k_scales,
                      key_batch_entries, rope_table, table_rows, step_cos, step_sin, kv_proj, kv_weight, kv_eps,
                      win_cache, win_batch_entries, win_cap, q_idx, q_format, q_codes, q_scales, pf);
  if (rc) return rc;
  rc = build_emit(positions, B, c_kv, c_gate, c_carry_kv, c_carry_gate, c_ratio, c_norm_weight, c_eps, c_cache,
                  c_cache_batch_entries, c_cache_cap, nullptr, nullptr, 0.0f, 0, nullptr, nullptr, 0, rope_table,
                  table_rows, nullptr, nullptr, nullptr, nullptr, 0.0f, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, pc);
  if (rc || B == 0) return rc;
  if (pf.br.ratio == 4 && coarse_form(pc)) {
    const unsigned nfine = emit_grid(pf);
    emit_pair_kernel<<<nfine + static_cast<unsigned>(B * kCoarseParts), 256, 0, as_stream(stream)>>>(pf, pc, nfine);
    MZK_LAUNCH_CHECK("decode_emit_pair");
    return MZK_OK;
  }
  rc = launch_emit(pf, stream);
  return rc ? rc : launch_emit(pc, stream);
}

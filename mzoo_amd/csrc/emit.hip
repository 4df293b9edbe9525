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

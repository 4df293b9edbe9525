// Piece 4: per-row top-k selection with a deterministic tie rule (radix select).
//
// Replaces `scores.topk(min(k, G), sorted=False)` + the -inf -> -1 "dummy slot" logic of
// src/mzoo/archs/owlet1/indexer.py:158-165 / layers/attn/golden_ref.py:230-243 /
// layers/attn/indexer/attn.py:67-81.  Contract:
//   * an entry with score -inf is never selected (the reference maps such picks to -1);
//   * among equal scores the LOWER index wins (the reference leaves ties unspecified);
//   * the selected indices are written in ascending index order, then -1 up to k.
//
// Algorithm (one 1024-thread workgroup per row):
//   key(x) = order-preserving uint32 of the fp32 score; -inf -> 0x007fffff.
//   1. count finite entries; if <= k, threshold T = key(-inf) and every finite entry is taken.
//   2. otherwise 4 MSB-first 8-bit digit passes: LDS histogram of the entries matching the
//      digits fixed so far, a suffix scan picks the digit holding the k-th largest key.
//      After the last pass T is the k-th largest key and `need_eq` entries equal to T
//      are still to be taken.
//   3. compaction in index order: take key > T, and the first `need_eq` entries with
//      key == T; two block-wide exclusive scans per 4096-entry chunk give the ranks.
// When the row fits (G <= kLdsKeys) the keys are staged once in LDS; otherwise every pass
// re-reads the row (L2-resident after the first pass).
#include "common.h"

namespace mzk {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsKeys = 16384;            // 64 KiB of keys
constexpr uint32_t kNegInfKey = 0x007fffffu;

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  return v;
}

// Exclusive block scan of one int per thread; returns the exclusive prefix and the total.
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v, lane);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = (lane < kWaves) ? wsum[lane] : 0;
    const int wi = wave_incl_scan(w, lane);
    if (lane < kWaves) wsum[kWaves + lane] = wi - w;  // exclusive wave offsets
    if (lane == kWaves - 1) wsum[2 * kWaves] = wi;
  }
  __syncthreads();
  const int out = wsum[kWaves + wave] + incl - v;
  total = wsum[2 * kWaves];
  __syncthreads();
  return out;
}

template <bool STAGE>
__global__ void __launch_bounds__(kThreads) topk_rows_kernel(const float* __restrict__ scores, int64_t row_stride,
                                                             int G, int k, int32_t* __restrict__ out,
                                                             int64_t out_stride) {
  extern __shared__ uint32_t lds_keys[];
  __shared__ int hist[256];
  __shared__ int wsum[2 * kWaves + 1];
  __shared__ uint32_t sel_digit;
  __shared__ int sel_rem;

  const int64_t row = blockIdx.x;
  const float* src = scores + row * row_stride;
  int32_t* dst = out + row * out_stride;
  const int tid = threadIdx.x;
  auto key_at = [&](int i) -> uint32_t { return STAGE ? lds_keys[i] : order_key(src[i]); };

  // 0. stage + count finite
  int nfin = 0;
  for (int i = tid; i < G; i += kThreads) {
    const uint32_t kk = order_key(src[i]);
    if (STAGE) lds_keys[i] = kk;
    nfin += (kk > kNegInfKey);
  }
  int total_fin;
  block_excl_scan(nfin, wsum, total_fin);

  uint32_t T = kNegInfKey;
  int need_eq = 0;
  if (total_fin > k) {
    uint32_t prefix = 0, mask = 0;
    int rem = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += kThreads) hist[i] = 0;
      __syncthreads();
      for (int i = tid; i < G; i += kThreads) {
        const uint32_t kk = key_at(i);
        if ((kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & 255u], 1);
      }
      __syncthreads();
      if (tid < 64) {
        const int lane = tid;
        int h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = hist[4 * lane + j];
        const int s = h[0] + h[1] + h[2] + h[3];
        // inclusive suffix sum over lanes (lanes above hold larger digits)
        int suf = s;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int o = __shfl_down(suf, off, 64);
          if (lane + off < 64) suf += o;
        }
        int above = suf - s;  // entries in digits of higher lanes
#pragma unroll
        for (int j = 3; j >= 0; --j) {
          if (above < rem && rem <= above + h[j]) {
            sel_digit = static_cast<uint32_t>(4 * lane + j);
            sel_rem = rem - above;
          }
          above += h[j];
        }
      }
      __syncthreads();
      prefix |= sel_digit << shift;
      mask |= 255u << shift;
      rem = sel_rem;
      __syncthreads();
    }
    T = prefix;
    need_eq = rem;
  }

  // 3. index-ordered compaction: 4 consecutive entries per thread per chunk
  int eq_seen = 0, written = 0;
  for (int base = 0; base < G; base += 4 * kThreads) {
    const int i0 = base + 4 * tid;
    uint32_t kk[4];
    int n_eq = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kk[j] = (i0 + j < G) ? key_at(i0 + j) : 0u;
      n_eq += (i0 + j < G) && (kk[j] == T) && (T != kNegInfKey);
    }
    int eq_total;
    const int eq_before = eq_seen + block_excl_scan(n_eq, wsum, eq_total);
    bool take[4];
    int n_take = 0, r = eq_before;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = i0 + j < G;
      bool t = valid && kk[j] > T;
      if (valid && kk[j] == T && T != kNegInfKey) {
        t = r < need_eq;
        ++r;
      }
      take[j] = t;
      n_take += t;
    }
    int take_total;
    int pos = written + block_excl_scan(n_take, wsum, take_total);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (take[j]) dst[pos++] = i0 + j;
    eq_seen += eq_total;
    written += take_total;
  }
  for (int i = written + tid; i < k; i += kThreads) dst[i] = -1;
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_topk_rows(const float* scores, int64_t rows, int64_t cols, int64_t row_stride, int topk,
                             int32_t* out, int64_t out_stride, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && cols >= 0 && topk >= 0, "topk_rows: negative size");
  MZK_CHECK_ARG(cols <= (int64_t(1) << 30) && topk <= (1 << 30), "topk_rows: row too long");
  MZK_CHECK_ARG(row_stride >= cols && out_stride >= topk, "topk_rows: strides smaller than the row");
  if (rows == 0 || topk == 0) return MZK_OK;
  MZK_CHECK_ARG(out != nullptr && (cols == 0 || scores != nullptr), "topk_rows: null pointer");
  MZK_CHECK_ARG(rows <= 0x7fffffff, "topk_rows: too many rows");
  hipStream_t s = as_stream(stream);
  const int G = static_cast<int>(cols);
  if (G <= kLdsKeys)
    topk_rows_kernel<true><<<static_cast<unsigned>(rows), kThreads, static_cast<size_t>(G) * 4, s>>>(
        scores, row_stride, G, topk, out, out_stride);
  else
    topk_rows_kernel<false><<<static_cast<unsigned>(rows), kThreads, 0, s>>>(scores, row_stride, G, topk, out,
                                                                             out_stride);
  MZK_LAUNCH_CHECK("topk_rows");
  return MZK_OK;
}

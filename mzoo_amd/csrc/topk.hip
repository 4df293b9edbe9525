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
// Rows up to 32 * 1024 keys keep them in registers (topk_rows_reg_kernel); longer rows
// re-read the row every pass (L2-resident after the first pass).
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

// hist[bin] += 1 for every active lane.  The first radix pass sees few distinct digits
// (scores share a handful of exponents), where per-lane LDS atomics would serialize on
// the same addresses: two rounds aggregate the lanes of the lowest pending lane's bin with
// a ballot (one atomic per round), the remaining lanes (spread digits) add individually.
__device__ __forceinline__ void hist_add(int* hist, uint32_t bin, bool active) {
  uint64_t pending = __ballot(active);
#pragma unroll
  for (int round = 0; round < 2; ++round) {
    if (pending == 0) return;
    const int leader = __builtin_ctzll(pending);
    const uint32_t lb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bin), leader));
    const bool mine = active && bin == lb;
    const uint64_t same = __ballot(mine);
    if ((threadIdx.x & 63) == leader) atomicAdd(&hist[lb], __popcll(same));
    active = active && !mine;
    pending &= ~same;
  }
  if (active) atomicAdd(&hist[bin], 1);
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
      // wave-uniform trip count, so every lane takes part in the ballots
      for (int i0 = 0; i0 < G; i0 += kThreads) {
        const int i = i0 + tid;
        const uint32_t kk = i < G ? key_at(i) : 0u;
        hist_add(hist, (kk >> shift) & 255u, i < G && (kk & mask) == prefix);
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

// ---- rows of G <= KPT * kThreads, keys held in registers -----------------------------

// Inclusive prefix sum over the 64 lanes with DPP: Kogge-Stone inside each row of 16
// lanes (row_shr 1, 2, 4, 8), then row_bcast:15 adds row r's total to row r+1 (rows 1, 3)
// and row_bcast:31 adds the total of rows 0-1 to rows 2-3.  Lanes a DPP source does not
// reach, and rows the row mask leaves out, add 0.
__device__ __forceinline__ int wave_incl_scan_dpp(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); // row_bcast:31
  return v;
}

// Every bin of the radix histogram has kSub counters, lane l adding to counter l % kSub:
// lanes whose keys share a digit (the leading digits of similar scores) then collide on
// at most 64 / kSub addresses per LDS atomic instead of all 64.
constexpr int kSub = 16;
constexpr int kHist = 256 * kSub;

// Digit selection in two steps.  (1) Every wave folds the sub-counters of its 256 / NW
// bins into bin totals: consecutive lanes read consecutive 16 B (conflict-free), each
// int4 being the four counters 4(l%4).. of one bin, and a quad reduction completes the
// bin.  (2) After a barrier, one wave owns bins 255-4l .. 252-4l in lane l (descending),
// so an inclusive prefix over lanes counts the entries in higher bins; it finds the bin
// holding the rem-th largest key and returns its digit, the rank left inside it, and
// whether the whole bin is taken (rank == count).
struct DigitSel {
  int digit, rem, whole;
};
template <int NW>
__device__ __forceinline__ void reduce_bins(const int* hist, int* tot, int wave, int lane) {
  static_assert(kSub == 16, "one int4 per lane covers a quarter of a bin");
  constexpr int R = 1024 / NW / 64;  // int4 reads per lane (each wave folds 1024/NW int4)
  const int4* h4 = reinterpret_cast<const int4*>(hist) + wave * (1024 / NW);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int4 v = h4[r * 64 + lane];  // bin (wave * 1024/NW + 64 r + lane) / 4
    int c = (v.x + v.y) + (v.z + v.w);
    c += __builtin_amdgcn_update_dpp(0, c, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    c += __builtin_amdgcn_update_dpp(0, c, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    if ((lane & 3) == 0) tot[(wave * (1024 / NW) + r * 64 + lane) >> 2] = c;
  }
}
__device__ __forceinline__ DigitSel select_digit(const int* tot, int rem, int lane) {
  const int4 t4 = reinterpret_cast<const int4*>(tot)[63 - lane];  // bins 252-4l .. 255-4l
  const int h[4] = {t4.w, t4.z, t4.y, t4.x};                      // h[j] = bin 255-4l-j
  const int s = (h[0] + h[1]) + (h[2] + h[3]);
  int above = wave_incl_scan_dpp(s) - s;
  DigitSel res{0, 0, 0};
  bool hit = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (above < rem && rem <= above + h[j]) {
      res.digit = 255 - 4 * lane - j;
      res.rem = rem - above;
      res.whole = (rem - above) == h[j];
      hit = true;
    }
    above += h[j];
  }
  // exactly one lane hits (the counts above the k-th key are < rem <= counts down to it)
  const uint64_t m = __ballot(hit);
  const int src_lane = m ? __builtin_ctzll(m) : 0;
  res.digit = __builtin_amdgcn_readlane(res.digit, src_lane);
  res.rem = __builtin_amdgcn_readlane(res.rem, src_lane);
  res.whole = __builtin_amdgcn_readlane(res.whole, src_lane);
  return res;
}

// Thread t holds keys t*KPT .. t*KPT+KPT-1.  The first digit's histogram is built while
// the finite entries are counted, and a pass stops the search early when the bin of the
// k-th largest key is taken whole (threshold: every key >= the bin's lowest key), which
// for distinct scores usually happens after two or three of the four 8-bit digits.
// Compaction: the output slot of an entry is (#key > T before it) +
// min(#key == T before it, need_eq), so one exclusive scan of the packed pair
// (n_gt << 16 | n_eq) gives every position.
template <int KPT, int NT>
__global__ void __launch_bounds__(NT) topk_rows_reg_kernel(const float* __restrict__ scores, int64_t row_stride,
                                                                 int G, int k, int32_t* __restrict__ out,
                                                                 int64_t out_stride) {
  __shared__ __align__(16) int hist[2][kHist];
  constexpr int NW = NT / 64;
  static_assert(NW % 4 == 0, "wave sums are read as int4");
  __shared__ __align__(16) int wsum[NW];
  __shared__ int sel[2][3];  // digit, rem, whole of the pass using hist[p & 1]
  __shared__ __align__(16) int bin_tot[256];

  const int64_t row = blockIdx.x;
  const float* src = scores + row * row_stride;
  int32_t* dst = out + row * out_stride;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int i0 = tid * KPT;

  float x[KPT];
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0 && i0 + KPT <= G) {
#pragma unroll
    for (int j = 0; j < KPT; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(src + i0 + j);
      x[j] = v.x;
      x[j + 1] = v.y;
      x[j + 2] = v.z;
      x[j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < KPT; ++j) x[j] = (i0 + j < G) ? src[i0 + j] : 0.0f;
  }
  {
    int4* h4 = reinterpret_cast<int4*>(&hist[0][0]);
    for (int i = tid; i < 2 * kHist / 4; i += NT) h4[i] = int4{0, 0, 0, 0};
  }
  __syncthreads();  // histograms cleared (while the scores are in flight)

  uint32_t key[KPT];
  int nfin = 0;  // wave-uniform
  int* h0 = &hist[0][lane % kSub];
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    key[j] = (i0 + j < G) ? order_key(x[j]) : 0u;  // 0 sorts below -inf: never taken
    nfin += __popcll(__ballot(key[j] > kNegInfKey));
    atomicAdd(h0 + (key[j] >> 24) * kSub, 1);
  }
  if (lane == 0) wsum[wave] = nfin;
  __syncthreads();  // first histogram and the finite counts complete
  int total_fin = 0;
  {
    const int4* w4 = reinterpret_cast<const int4*>(wsum);
#pragma unroll
    for (int q = 0; q < NW / 4; ++q) {
      const int4 v = w4[q];
      total_fin += (v.x + v.y) + (v.z + v.w);
    }
  }

  uint32_t T = kNegInfKey;
  int need_eq = 0;
  if (total_fin > k) {
    uint32_t prefix = 0, mask = 0;
    int rem = k;
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      const int cur = pass & 1;
      reduce_bins<NW>(hist[cur], bin_tot, wave, lane);
      if (pass > 0) {
        // the next pass's copy (its last reader, the reduction two passes ago, is done);
        // hist[1] is still clear for the second pass
        int4* h4 = reinterpret_cast<int4*>(&hist[cur ^ 1][0]);
        for (int i = tid; i < kHist / 4; i += NT) h4[i] = int4{0, 0, 0, 0};
      }
      __syncthreads();  // bin totals complete
      if (wave == 0) {
        const DigitSel r = select_digit(bin_tot, rem, lane);
        if (lane == 0) {
          sel[cur][0] = r.digit;
          sel[cur][1] = r.rem;
          sel[cur][2] = r.whole;
        }
      }
      __syncthreads();  // selection published, next copy cleared
      const uint32_t digit = static_cast<uint32_t>(sel[cur][0]);
      rem = sel[cur][1];
      const uint32_t low = prefix | (digit << shift);
      if (sel[cur][2] && low != 0u) {  // bin taken whole: every key >= low
        T = low - 1u;
        need_eq = 0;
        break;
      }
      prefix = low;
      mask |= 255u << shift;
      if (shift == 0) {
        T = prefix;
        need_eq = rem;
        break;
      }
      int* hn = &hist[cur ^ 1][lane % kSub];
#pragma unroll
      for (int j = 0; j < KPT; ++j)
        if ((key[j] & mask) == prefix) atomicAdd(hn + ((key[j] >> (shift - 8)) & 255u) * kSub, 1);
      __syncthreads();  // next histogram complete
    }
  }

  // compaction in index order
  int n_gt = 0, n_eq = 0;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    n_gt += key[j] > T;
    n_eq += (key[j] == T) && (T != kNegInfKey);
  }
  // packed as unsigned: n_gt <= G <= 32768 fills bit 31 at most, n_eq stays below 2^16
  const int packed = (n_gt << 16) | n_eq;
  const int incl = wave_incl_scan_dpp(packed);
  __syncthreads();  // every wave is done reading wsum (finite counts)
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = static_cast<uint32_t>(incl - packed), tot = 0;
  {
    const int4* w4 = reinterpret_cast<const int4*>(wsum);
#pragma unroll
    for (int q = 0; q < NW / 4; ++q) {
      const int4 v = w4[q];
      const int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (4 * q + e < wave) before += static_cast<uint32_t>(w[e]);
        tot += static_cast<uint32_t>(w[e]);
      }
    }
  }
  int gt_before = static_cast<int>(before >> 16), eq_before = static_cast<int>(before & 0xffffu);
  const int written = static_cast<int>(tot >> 16) + min(static_cast<int>(tot & 0xffffu), need_eq);
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    if (key[j] > T) {
      dst[gt_before + min(eq_before, need_eq)] = i0 + j;
      ++gt_before;
    } else if (key[j] == T && T != kNegInfKey) {
      if (eq_before < need_eq) dst[gt_before + eq_before] = i0 + j;
      ++eq_before;
    }
  }
  for (int i = written + tid; i < k; i += NT) dst[i] = -1;
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
  const unsigned nr = static_cast<unsigned>(rows);
  if (G <= 8 * kThreads)
    topk_rows_reg_kernel<8, kThreads><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= 16 * kThreads)
    topk_rows_reg_kernel<16, kThreads><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= 32 * kThreads)
    topk_rows_reg_kernel<32, kThreads><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= kLdsKeys)
    topk_rows_kernel<true><<<nr, kThreads, static_cast<size_t>(G) * 4, s>>>(scores, row_stride, G, topk, out,
                                                                           out_stride);
  else
    topk_rows_kernel<false><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  MZK_LAUNCH_CHECK("topk_rows");
  return MZK_OK;
}

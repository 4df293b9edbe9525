// The row selection of the top-k (piece 4), shared by the top-k kernels (topk.hip) and the
// decode attention kernel that selects its row's entries itself (attention.hip).
//
// One workgroup of NT threads holds a row of up to KPT * NT scores as order keys, KPT per
// thread (thread t: keys KPT t .. KPT t + KPT - 1).  The k-th largest key T and the number
// need_eq of keys equal to T still to take come from three levels of bins, each a histogram
// in LDS over the keys still open: the top 11 bits of the key (sign, exponent and two
// mantissa bits of the score: four bins per octave; finite keys lie in bins >= 4, -inf is key
// 0x007fffff in bin 3, the padding key 0 in bin 0), then bits 20..10 and bits 9..0 of the
// keys in the bin holding the k-th largest.  A level stops the search when that bin is taken
// whole (its keys are all among the k largest), which for distinct scores happens after the
// first or the second.  The three histograms are cleared up front, so a level costs one
// barrier for its histogram and two for its bin search: workgroup barriers, not arithmetic,
// are what a level costs.  The selection (owlet1/indexer.py:158-165 with a deterministic tie
// rule): key > T, and the first need_eq keys equal to T in index order; the output slot of a
// taken key is (#key > T before it) + min(#key == T before it, need_eq), from one scan of the
// packed pair (n_gt << 16 | n_eq).
#pragma once

#include "common.h"

namespace mzk {

// Order-preserving uint32 of an fp32 score (larger score, larger key); -inf -> 0x007fffff.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
constexpr uint32_t kNegInfKey = 0x007fffffu;
// All ones for a position inside the row, else 0: `order_key(x) & key_mask(i, G)` gives the
// padding key 0 (below -inf: never counted or taken) past the row's end, branch-free (a
// conditional expression here compiles to one branch per key).
__device__ __forceinline__ uint32_t key_mask(int i, int G) { return 0u - static_cast<uint32_t>(i < G); }

constexpr int kBinBits = 11;
constexpr int kBins = 1 << kBinBits;           // 2048 first-level bins
constexpr int kLowBits = 32 - kBinBits;        // 21 bits below a first-level bin
constexpr int kSub1 = 4;                       // first-level sub-counters per bin (lane % kSub1)
static_assert(kSub1 % 4 == 0, "a bin's sub-counters are read as whole int4s");

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

// Inclusive scan over the NT threads of one int each (one barrier); `total` is the sum.
// wsum [NT/64] may be written again after the caller's next barrier.
template <int NT>
__device__ __forceinline__ int block_incl_scan(int v, int* wsum, int& total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int incl = wave_incl_scan_dpp(v);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int x = wsum[w];
    before += w < wave ? x : 0;
    tot += x;
  }
  total = tot;
  return incl + before;
}

// The bin holding the rem-th largest entry of an NB-bin histogram: thread t holds the counts
// c[j] of bins NB-1-(BPT*t+j) (descending), so the block scan counts the entries above each
// thread's bins.  Every thread returns the same (bin = rem = count = 0 when rem exceeds the
// total).  Two barriers; sh [3] may be written again after the caller's next barrier.
struct BinHit {
  int bin, rem, count, total;  // the bin, the rank left inside it, its count, the histogram total
};
template <int NT, int NB>
__device__ __forceinline__ BinHit find_bin(const int (&c)[NB / NT], int rem, int* wsum, int* sh) {
  constexpr int BPT = NB / NT;
  const int tid = threadIdx.x;
  if (tid == 0) {
    sh[0] = 0;
    sh[1] = 0;
    sh[2] = 0;
  }
  int s = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) s += c[j];
  int total;
  const int incl = block_incl_scan<NT>(s, wsum, total);
  int above = incl - s;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    if (above < rem && rem <= above + c[j]) {  // exactly one (thread, j) when rem <= total
      sh[0] = NB - 1 - (BPT * tid + j);
      sh[1] = rem - above;
      sh[2] = c[j];
    }
    above += c[j];
  }
  __syncthreads();
  return BinHit{sh[0], sh[1], sh[2], total};
}

// The LDS of one row's selection: hist1 [kBins * kSub1], hist2 [kBins] (bits 20..10 of the
// keys in the first level's bin), hist3 [kBins / 2] (bits 9..0 of the keys in the second
// level's bin), all 16-byte aligned; wsum [NT / 64]; sh0, sh1 [3] each (the bin searches
// alternate between the two).
struct RowSelLds {
  int* hist1;
  int* hist2;
  int* hist3;
  int* wsum;
  int* sh0;
  int* sh1;
};
template <int NT>
constexpr int row_sel_lds_bytes() {
  return (kBins * kSub1 + kBins + kBins / 2 + NT / 64 + 8) * 4;
}

// Clear the three histograms (no barrier: the caller's next barrier publishes it; issue it
// while the scores are in flight).
template <int NT>
__device__ __forceinline__ void row_sel_clear(const RowSelLds& s, int tid) {
  int4* h4 = reinterpret_cast<int4*>(s.hist1);
  for (int i = tid; i < kBins * kSub1 / 4; i += NT) h4[i] = int4{0, 0, 0, 0};
  for (int i = tid; i < kBins / 4; i += NT) reinterpret_cast<int4*>(s.hist2)[i] = int4{0, 0, 0, 0};
  for (int i = tid; i < kBins / 8; i += NT) reinterpret_cast<int4*>(s.hist3)[i] = int4{0, 0, 0, 0};
}

// T and need_eq of the row (T = kNegInfKey, need_eq = 0: at most k finite keys, take them
// all).  `search` (workgroup-uniform) is G > k; when set, the caller has cleared the
// histograms and passed a barrier since.
template <int KPT, int NT>
__device__ __forceinline__ void row_sel_threshold(const uint32_t (&key)[KPT], bool search, int k, const RowSelLds& s,
                                                  uint32_t& T, int& need_eq) {
  constexpr int BPT = kBins / NT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  BinHit h1{0, 0, 0, 0};
  if (search) {
    int* hl = s.hist1 + (lane & (kSub1 - 1));
#pragma unroll
    for (int j = 0; j < KPT; ++j)
      if (key[j] > kNegInfKey) atomicAdd(hl + (key[j] >> kLowBits) * kSub1, 1);
    __syncthreads();
    int c1[BPT];
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int4* hb = reinterpret_cast<const int4*>(s.hist1) + (kBins - 1 - (BPT * tid + j)) * (kSub1 / 4);
      int sum = 0;
#pragma unroll
      for (int q = 0; q < kSub1 / 4; ++q) {
        const int4 v = hb[q];
        sum += (v.x + v.y) + (v.z + v.w);
      }
      c1[j] = sum;
    }
    h1 = find_bin<NT, kBins>(c1, k, s.wsum, s.sh0);
  }
  T = kNegInfKey;
  need_eq = 0;
  if (search && h1.total > k) {
    const uint32_t b1 = static_cast<uint32_t>(h1.bin);  // >= 4
    if (h1.count == h1.rem) {
      T = (b1 << kLowBits) - 1u;
    } else {
#pragma unroll
      for (int j = 0; j < KPT; ++j)
        if ((key[j] >> kLowBits) == b1) atomicAdd(&s.hist2[(key[j] >> 10) & (kBins - 1)], 1);
      __syncthreads();
      int c2[BPT];
#pragma unroll
      for (int j = 0; j < BPT; ++j) c2[j] = s.hist2[kBins - 1 - (BPT * tid + j)];
      const BinHit h2 = find_bin<NT, kBins>(c2, h1.rem, s.wsum, s.sh1);
      const uint32_t p2 = (b1 << kLowBits) | (static_cast<uint32_t>(h2.bin) << 10);
      if (h2.count == h2.rem) {
        T = p2 - 1u;
      } else {
#pragma unroll
        for (int j = 0; j < KPT; ++j)
          if ((key[j] >> 10) == (p2 >> 10)) atomicAdd(&s.hist3[key[j] & 1023u], 1);
        __syncthreads();
        constexpr int B3 = kBins / 2;
        int c3[B3 / NT];
#pragma unroll
        for (int j = 0; j < B3 / NT; ++j) c3[j] = s.hist3[B3 - 1 - ((B3 / NT) * tid + j)];
        const BinHit h3 = find_bin<NT, B3>(c3, h2.rem, s.wsum, s.sh0);
        T = p2 | static_cast<uint32_t>(h3.bin);  // the k-th largest key itself
        need_eq = h3.rem;
      }
    }
  }
}

// The compaction's per-thread share: `sel` the thread's taken keys (bit j: key j), `pos` the
// output slot of its lowest taken key (the next ones follow in order), `written` the row's
// count of taken keys.  One block scan (one barrier).
struct RowTake {
  uint32_t sel;
  int pos, written;
};
template <int KPT, int NT>
__device__ __forceinline__ RowTake row_sel_take(const uint32_t (&key)[KPT], uint32_t T, int need_eq, int* wsum) {
  static_assert(KPT <= 32, "one bit per key of a thread");
  static_assert(KPT * NT <= 32768, "packed counts: at most 2^15 keys per row");
  uint32_t gt_mask = 0u, eq_mask = 0u;
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    gt_mask |= static_cast<uint32_t>(key[j] > T) << j;
    eq_mask |= static_cast<uint32_t>((key[j] == T) && (T != kNegInfKey)) << j;
  }
  const int n_gt = __builtin_popcount(gt_mask), n_eq = __builtin_popcount(eq_mask);
  // packed as unsigned: n_gt <= G <= 32768 fills bit 31 at most, n_eq stays below 2^16
  const int packed = (n_gt << 16) | n_eq;
  int tot_p;
  const int incl = block_incl_scan<NT>(packed, wsum, tot_p);
  const uint32_t before = static_cast<uint32_t>(incl - packed), tot = static_cast<uint32_t>(tot_p);
  const int gt_before = static_cast<int>(before >> 16), eq_before = static_cast<int>(before & 0xffffu);
  RowTake r;
  r.written = static_cast<int>(tot >> 16) + min(static_cast<int>(tot & 0xffffu), need_eq);
  r.sel = gt_mask;
  for (int m = need_eq - eq_before; m > 0 && eq_mask != 0u; --m) {
    const uint32_t low = eq_mask & (0u - eq_mask);  // its lowest-indexed keys equal to T first
    r.sel |= low;
    eq_mask ^= low;
  }
  r.pos = gt_before + min(eq_before, need_eq);
  return r;
}

}  // namespace mzk

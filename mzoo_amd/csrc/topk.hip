// Piece 4: per-row top-k selection with a deterministic tie rule (radix select).
//
// Replaces `scores.topk(min(k, G), sorted=False)` + the -inf -> -1 "dummy slot" logic of
// src/mzoo/archs/owlet1/indexer.py:158-165 / layers/attn/golden_ref.py:230-243 /
// layers/attn/indexer/attn.py:67-81.  Contract:
//   * an entry with score -inf is never selected (the reference maps such picks to -1);
//   * among equal scores the LOWER index wins (the reference leaves ties unspecified);
//   * the selected indices are written in ascending index order, then -1 up to k.
//
// Algorithm:
//   key(x) = order-preserving uint32 of the fp32 score; -inf -> 0x007fffff.
//   1. first-level histogram of the finite keys over their top 11 bits; a block scan finds
//      the bin b1 of the k-th largest key (or: at most k finite keys, take them all);
//   2. the keys of b1 are resolved by re-binning the window of keys still open over its
//      own min .. max (at most two passes for 21 bits) -- T, the k-th largest key, and
//      `need_eq`, the entries equal to T still to be taken;
//   3. compaction in index order: take key > T, and the first `need_eq` entries with
//      key == T.
// Rows up to 32 * 1024 keys keep them in registers (topk_row_kernel, one workgroup per
// row); longer rows without a workspace stream the row through 8-bit digit passes
// (topk_rows_kernel).  mzk_topk_rows_ws splits rows of 32769 .. 64 x 8192 keys over chunk
// workgroups (three launches, see below).
#include "topk_core.h"

namespace mzk {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsKeys = 16384;            // 64 KiB of keys

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


// ---- rows of G <= KPT * NT, one workgroup per row, keys held in registers -------------
//
// The row selection of topk_core.h (three levels of bins, then the compaction in index
// order) over the row's scores, KPT keys per thread.

// MAP: the row is a candidate axis of blocks of kMapBs slots (slot j = key
// cand[row][j / kMapBs] * kMapBs + j % kMapBs, the level-two scores); the index list is
// written as key positions.  A thread's KPT slots are whole blocks, so it loads KPT / kMapBs
// list entries with its scores.
constexpr int kMapBs = 8;
struct SlotMap {
  const int32_t* cand;
  int64_t stride;
  int nb;
};

template <int KPT, int NT, bool MAP = false>
__global__ void __launch_bounds__(NT) topk_row_kernel(const float* __restrict__ scores, int64_t row_stride, int G,
                                                      int k, int32_t* __restrict__ out, int64_t out_stride,
                                                      SlotMap sm = SlotMap{}) {
  constexpr int NW = NT / 64;
  __shared__ __align__(16) int hist1[kBins * kSub1];
  __shared__ __align__(16) int hist2[kBins];
  __shared__ __align__(16) int hist3[kBins / 2];
  __shared__ int wsum[NW];
  __shared__ int sh[2][3];
  const RowSelLds lds{hist1, hist2, hist3, wsum, sh[0], sh[1]};

  const int64_t row = blockIdx.x;
  const float* src = scores + row * row_stride;
  int32_t* dst = out + row * out_stride;
  const int tid = threadIdx.x;
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
  static_assert(!MAP || KPT % kMapBs == 0, "whole candidate blocks per thread");
  int32_t cb[MAP ? KPT / kMapBs : 1];  // MAP: the candidate blocks of this thread's slots
  if constexpr (MAP) {
    const int32_t* crow = sm.cand + row * sm.stride;
#pragma unroll
    for (int m = 0; m < KPT / kMapBs; ++m) cb[m] = crow[min(i0 / kMapBs + m, sm.nb - 1)];
  }
  // G <= k (workgroup-uniform): every finite key is taken, no search
  const bool search = G > k;
  if (search) {
    row_sel_clear<NT>(lds, tid);
    __syncthreads();  // histograms cleared (while the scores are in flight)
  }
  uint32_t key[KPT];
#pragma unroll
  for (int j = 0; j < KPT; ++j) key[j] = order_key(x[j]) & key_mask(i0 + j, G);  // 0 sorts below -inf: never taken
  uint32_t T;
  int need_eq;
  row_sel_threshold<KPT, NT>(key, search, k, lds, T, need_eq);
  const RowTake tk = row_sel_take<KPT, NT>(key, T, need_eq, wsum);
  uint32_t sel = tk.sel;
  int pos = tk.pos;
  // Written in rounds, one taken key per thread (lowest index first), so a wave issues as
  // many store instructions as its busiest thread has taken keys rather than KPT.
  while (__any(sel != 0u)) {
    if (sel != 0u) {
      const int j = __builtin_ctz(sel);
      // the value written: the index, or under MAP the slot's key position (a taken slot has
      // a finite score, which the candidate scorer writes only for slots of a listed block)
      int32_t v = i0 + j;
      if constexpr (MAP) {
        int32_t c = cb[0];
#pragma unroll
        for (int b = 1; b < KPT / kMapBs; ++b)
          if (j / kMapBs == b) c = cb[b];
        v = c >= 0 ? c * kMapBs + j % kMapBs : -1;
      }
      if (pos < k) dst[pos] = v;  // always true when the histograms count the row's keys
      ++pos;
      sel &= sel - 1u;
    }
  }
  for (int i = tk.written + tid; i < k; i += NT) dst[i] = -1;
}

// ---- long rows, few of them: the row split over chunk workgroups ---------------------
//
// A row of G > kMultiMinG keys is cut into chunks of kChunk keys (thread t of a chunk
// holds keys 8t .. 8t+7 in registers).  Three launches, each spread over every (chunk,
// row) workgroup, so no step streams a whole row through one CU:
//   A  histogram of the top kBinBits of the chunk's finite keys;
//   B  every chunk workgroup merges its row's histograms and finds the bin b1 of the k-th
//      largest key (all chunks of a row reach the same b1), counts its keys in the bins
//      above b1 and writes its keys of b1 (a few thousand per row for any spread of
//      scores) to its own candidate region, in index order;
//   C  every chunk workgroup loads its row's candidates into LDS and runs the same 3 x
//      7-bit radix select over their low 21 bits (threshold T, and need_eq keys equal to
//      T taken, lowest indices first), derives its first output slot from the counts of
//      the chunks before it and writes its selected indices in index order.  If b1 holds
//      more than kCandCap keys the selection streams the row instead (slow, but exact).
// Same contract and results as the single-workgroup kernels.
constexpr int kChunk = 8 * kThreads;           // keys per chunk workgroup
constexpr int kCandCap = 12288;                // keys of bin b1 held in LDS
constexpr int kMaxChunks = 64;                 // rows up to 64 x 8192 keys
// shorter rows stay on one workgroup: up to 16384 keys it is twice as fast as the three
// chunk launches, at 32768 even (measured on MI355X in HIP graphs: 8.6 vs 16.2 us at
// 4 x 16384, 16.1 vs 16.8 us at 8 x 32768)
constexpr int64_t kMultiMinG = 32 * kThreads;

// Workspace: hist [rows][nch][kBins] int32 | above [rows][nch] int32 | sel [rows] int4
// (mode, b1, rem, finite total) | cand [rows][nch][kChunk] (key, index): chunk c of a row
// writes its keys of bin b1 to the first hist[row][c][b1] slots of its own region
struct MultiWs {
  int64_t hist, above, sel, cand, total;
};
__host__ __device__ inline int64_t round16(int64_t x) { return (x + 15) / 16 * 16; }
__host__ __device__ inline MultiWs multi_ws(int64_t rows, int64_t nch) {
  MultiWs w;
  w.hist = 0;
  w.above = rows * nch * kBins * 4;
  w.sel = w.above + round16(rows * nch * 4);
  w.cand = w.sel + rows * 16;
  w.total = w.cand + rows * nch * kChunk * 8;
  return w;
}

// The 8 keys of thread t of chunk c (0 beyond G: below -inf, never counted or taken).
__device__ __forceinline__ void load_chunk_keys(const float* __restrict__ src, int G, int base, int t,
                                                uint32_t (&key)[8]) {
  const int i0 = base + 8 * t;
  float x[8];
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0 && i0 + 8 <= G) {
    const float4 a = *reinterpret_cast<const float4*>(src + i0);
    const float4 b = *reinterpret_cast<const float4*>(src + i0 + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (i0 + j < G) ? src[i0 + j] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) key[j] = (i0 + j < G) ? order_key(x[j]) : 0u;
}

__global__ void __launch_bounds__(kThreads) topk_chunk_hist_kernel(const float* __restrict__ scores,
                                                                     int64_t row_stride, int G, int nch,
                                                                     int* __restrict__ hist_out) {
  constexpr int kSubA = 4;  // sub-counters per bin (lane % 4): equal digits spread over 4 addresses
  __shared__ __align__(16) int hist[kBins * kSubA];
  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = scores + static_cast<int64_t>(row) * row_stride;
  const int tid = threadIdx.x;
  uint32_t key[8];
  load_chunk_keys(src, G, c * kChunk, tid, key);
  int4* h4 = reinterpret_cast<int4*>(hist);
  for (int i = tid; i < kBins * kSubA / 4; i += kThreads) h4[i] = int4{0, 0, 0, 0};
  __syncthreads();
  int* hs = hist + (tid & (kSubA - 1));
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (key[j] > kNegInfKey) atomicAdd(hs + (key[j] >> kLowBits) * kSubA, 1);
  __syncthreads();
  // bins 2t, 2t+1: sum their sub-counters, one 8-byte store per thread
  const int4 a = h4[2 * tid], b = h4[2 * tid + 1];
  int* dst = hist_out + (static_cast<int64_t>(row) * nch + c) * kBins;
  *reinterpret_cast<int2*>(dst + 2 * tid) = int2{(a.x + a.y) + (a.z + a.w), (b.x + b.y) + (b.z + b.w)};
}

// Every key of the row, 8 per thread per chunk step (keys beyond G read as 0, which lies
// in no bin a selection looks at); the loads of kScanBatch steps are issued together, one
// memory round trip per batch (a batch inside an aligned row takes one workgroup-uniform
// branch to its vector loads); f(key[8], index of key[0]) runs in wave-uniform control flow.
constexpr int kScanBatch = 4;
template <class F>
__device__ __forceinline__ void for_row_keys(const float* __restrict__ src, int G, F&& f) {
  const int tid = threadIdx.x;
  const bool vec = (reinterpret_cast<uintptr_t>(src) & 15) == 0;
  for (int base = 0; base < G; base += kScanBatch * kChunk) {
    uint32_t key[kScanBatch][8];
    if (vec && base + kScanBatch * kChunk <= G) {
      float4 v[kScanBatch][2];
#pragma unroll
      for (int b = 0; b < kScanBatch; ++b) {
        const float* p = src + base + b * kChunk + 8 * tid;
        v[b][0] = *reinterpret_cast<const float4*>(p);
        v[b][1] = *reinterpret_cast<const float4*>(p + 4);
      }
#pragma unroll
      for (int b = 0; b < kScanBatch; ++b) {
        const float x[8] = {v[b][0].x, v[b][0].y, v[b][0].z, v[b][0].w, v[b][1].x, v[b][1].y, v[b][1].z, v[b][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) key[b][j] = order_key(x[j]);
      }
    } else {
#pragma unroll
      for (int b = 0; b < kScanBatch; ++b) load_chunk_keys(src, G, base + b * kChunk, tid, key[b]);
    }
#pragma unroll
    for (int b = 0; b < kScanBatch; ++b)
      if (base + b * kChunk < G) f(key[b], base + b * kChunk + 8 * tid);
  }
}

// How the row's selection splits at the bin level.  mode 0: at most k finite keys, take
// them all; 1: the keys of bins >= b1 are exactly the k largest; 2: the keys of bins > b1
// plus the rem largest of bin b1 (lowest indices first among equals).
struct RowSel {
  int mode, b1, rem, total;
};

// Merge the row's chunk histograms (thread t: bins 2t, 2t+1; 16 chunks per memory round
// trip) and locate the bin of the k-th largest finite key with one block-wide scan.  Every
// thread returns the same.  wsum [kWaves] and sh [3] are LDS scratch.
__device__ RowSel row_threshold_bin(const int* __restrict__ hrow, int nch, int k, int* wsum, int* sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int t0 = 0, t1 = 0;
  for (int c0 = 0; c0 < nch; c0 += 16) {
    int2 v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {  // branch-free: chunks past the end re-read the last one
      const int cj = c0 + j < nch ? c0 + j : nch - 1;
      v[j] = *reinterpret_cast<const int2*>(hrow + static_cast<int64_t>(cj) * kBins + 2 * tid);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int keep = c0 + j < nch;
      t0 += keep * v[j].x;
      t1 += keep * v[j].y;
    }
  }
  // inclusive prefix of the pair totals over threads (= over bins, ascending)
  const int pair = t0 + t1;
  int incl = wave_incl_scan_dpp(pair);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    total += wsum[w];
    incl += w < wave ? wsum[w] : 0;
  }
  RowSel r{0, 0, 0, total};
  if (total > k) {
    // keys in bins above thread t's pair: total - incl; exactly one (thread, bin) holds
    // the k-th largest key
    const int above_hi = total - incl;  // keys in bins > 2t+1
    const int above_lo = above_hi + t1; // keys in bins > 2t
    if (above_hi < k && k <= above_hi + t1) {
      sh[0] = 2 * tid + 1;
      sh[1] = k - above_hi;
      sh[2] = t1;
    } else if (above_lo < k && k <= above_lo + t0) {
      sh[0] = 2 * tid;
      sh[1] = k - above_lo;
      sh[2] = t0;
    }
    __syncthreads();
    r.b1 = sh[0];
    r.rem = sh[1];
    r.mode = sh[1] == sh[2] ? 1 : 2;
  }
  return r;
}

__global__ void __launch_bounds__(kThreads) topk_chunk_gather_kernel(const float* __restrict__ scores,
                                                                       int64_t row_stride, int G, int k, int nch,
                                                                       const int* __restrict__ hist_in,
                                                                       int* __restrict__ above_out,
                                                                       int4* __restrict__ sel_out,
                                                                       uint2* __restrict__ cand_out) {
  __shared__ int wsum[kWaves];
  __shared__ int red[kWaves];
  __shared__ int msum[kWaves];
  __shared__ int sh[3];
  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = scores + static_cast<int64_t>(row) * row_stride;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t key[8];
  load_chunk_keys(src, G, c * kChunk, tid, key);  // in flight during the histogram merge
  const RowSel rs = row_threshold_bin(hist_in + static_cast<int64_t>(row) * nch * kBins, nch, k, wsum, sh);
  const int b_lo = rs.mode == 0 ? 0 : (rs.mode == 1 ? rs.b1 : rs.b1 + 1);
  // this chunk's finite keys in bins >= b_lo (finite keys sit in bins >= 4)
  int n = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) n += key[j] > kNegInfKey && static_cast<int>(key[j] >> kLowBits) >= b_lo;
  n += __shfl_xor(n, 1, 64);
  n += __shfl_xor(n, 2, 64);
  n += __shfl_xor(n, 4, 64);
  n += __shfl_xor(n, 8, 64);
  n += __shfl_xor(n, 16, 64);
  n += __shfl_xor(n, 32, 64);
  if (lane == 0) red[wave] = n;
  // this chunk's keys of bin b1, in index order, to the chunk's own candidate region
  // (slots from a workgroup scan: no atomics)
  int nm = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) nm += rs.mode == 2 && static_cast<int>(key[j] >> kLowBits) == rs.b1;
  const int mincl = wave_incl_scan_dpp(nm);
  if (lane == 63) msum[wave] = mincl;
  __syncthreads();
  if (rs.mode == 2) {
    int slot = mincl - nm;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) slot += w < wave ? msum[w] : 0;
    uint2* dst = cand_out + (static_cast<int64_t>(row) * nch + c) * kChunk;
    const int i0 = c * kChunk + 8 * tid;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (static_cast<int>(key[j] >> kLowBits) == rs.b1) {
        dst[slot] = uint2{key[j], static_cast<uint32_t>(i0 + j)};
        ++slot;
      }
    }
  }
  if (tid == 0) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += red[w];
    above_out[static_cast<int64_t>(row) * nch + c] = tot;
    if (c == 0) sel_out[row] = int4{rs.mode, rs.b1, rs.rem, rs.total};
  }
}

__global__ void __launch_bounds__(kThreads) topk_chunk_select_write_kernel(
    const float* __restrict__ scores, int64_t row_stride, int G, int k, int nch, const int* __restrict__ hist_in,
    const int* __restrict__ above_in, const int4* __restrict__ sel_in, const uint2* __restrict__ cand_in,
    int32_t* __restrict__ out, int64_t out_stride) {
  __shared__ uint32_t cand_key[kCandCap];
  __shared__ int cand_idx[kCandCap];
  __shared__ int hist7[128];
  __shared__ int chunk_gt[kMaxChunks], chunk_eq[kMaxChunks], chunk_above[kMaxChunks], cand_start[kMaxChunks + 1];
  __shared__ __align__(16) int wsum[kWaves];
  __shared__ int sh_rem, sh_digit, sh_off, sh_take, sh_total;

  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = scores + static_cast<int64_t>(row) * row_stride;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t key[8];
  load_chunk_keys(src, G, c * kChunk, tid, key);
  const int4 rs = sel_in[row];
  const int mode = rs.x, b1 = rs.y;
  // per chunk: keys above b1 and keys in b1 (the candidates, from the chunk histograms)
  int cnt_b1 = 0;
  if (tid < kMaxChunks) {
    const int ct = tid < nch ? tid : nch - 1;
    chunk_gt[tid] = 0;
    chunk_eq[tid] = 0;
    chunk_above[tid] = tid < nch ? above_in[static_cast<int64_t>(row) * nch + ct] : 0;
    cnt_b1 = tid < nch ? hist_in[(static_cast<int64_t>(row) * nch + ct) * kBins + b1] : 0;
  }
  if (wave == 0) {  // candidate start of every chunk (exclusive prefix over the 64 lanes)
    const int ci = wave_incl_scan_dpp(cnt_b1);
    cand_start[lane + 1] = ci;
    if (lane == 0) cand_start[0] = 0;
  }
  __syncthreads();
  const int ncand_all = cand_start[kMaxChunks];
  uint32_t T = kNegInfKey;
  int need_eq = 0;
  if (mode == 1) T = (static_cast<uint32_t>(b1) << kLowBits) - 1u;  // b1 >= 4
  if (mode == 2) {
    const bool in_lds = ncand_all <= kCandCap;
    const int ncand = in_lds ? ncand_all : 0;
    const uint2* cr = cand_in + static_cast<int64_t>(row) * nch * kChunk;
    for (int m = tid; m < ncand; m += kThreads) {
      // chunk holding candidate m: the last start <= m (binary search over the starts)
      int lo = 0, hi = nch - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cand_start[mid] <= m) lo = mid;
        else hi = mid - 1;
      }
      const uint2 v = cr[static_cast<int64_t>(lo) * kChunk + (m - cand_start[lo])];
      cand_key[m] = v.x;
      cand_idx[m] = static_cast<int>(v.y);
    }
    __syncthreads();
    // f(key, index, active) over the keys of bin b1, in wave-uniform control flow
    auto for_cands = [&](auto&& f) {
      if (in_lds) {
        for (int m0 = 0; m0 < ncand; m0 += kThreads) {
          const int m = m0 + tid;
          const bool a = m < ncand;
          f(a ? cand_key[m] : 0u, a ? cand_idx[m] : 0, a);
        }
      } else {
        for_row_keys(src, G, [&](const uint32_t (&kk)[8], int i0) {
#pragma unroll
          for (int j = 0; j < 8; ++j) f(kk[j], i0 + j, static_cast<int>(kk[j] >> kLowBits) == b1);
        });
      }
    };
    uint32_t prefix = static_cast<uint32_t>(b1) << kLowBits, mask = ~((1u << kLowBits) - 1u);
    int rem = rs.z;
    for (int shift = kLowBits - 7; shift >= 0; shift -= 7) {
      if (tid < 128) hist7[tid] = 0;
      __syncthreads();
      for_cands([&](uint32_t kk, int, bool a) { hist_add(hist7, (kk >> shift) & 127u, a && (kk & mask) == prefix); });
      __syncthreads();
      if (wave == 0) {
        const int h0 = hist7[127 - 2 * lane], h1 = hist7[126 - 2 * lane];
        const int hs = h0 + h1;
        const int above = wave_incl_scan_dpp(hs) - hs;
        int d = -1, r = 0;
        if (above < rem && rem <= above + h0) {
          d = 127 - 2 * lane;
          r = rem - above;
        } else if (above + h0 < rem && rem <= above + hs) {
          d = 126 - 2 * lane;
          r = rem - above - h0;
        }
        const uint64_t m = __ballot(d >= 0);
        const int srcl = m ? __builtin_ctzll(m) : 0;
        if (lane == srcl) {
          sh_digit = d < 0 ? 0 : d;
          sh_rem = r;
        }
      }
      __syncthreads();
      prefix |= static_cast<uint32_t>(sh_digit) << shift;
      mask |= 127u << shift;
      rem = sh_rem;
      __syncthreads();  // sh_digit / sh_rem read by every thread before the next pass
    }
    T = prefix;
    need_eq = rem;
    // keys of bin b1 above / equal to T, per chunk
    for_cands([&](uint32_t kk, int i, bool a) {
      const uint32_t cc = static_cast<uint32_t>(i / kChunk);
      hist_add(chunk_gt, cc, a && kk > T);
      hist_add(chunk_eq, cc, a && kk == T);
    });
  }
  __syncthreads();
  // this chunk's first output slot and share of the equal keys (index order), the row total
  if (tid == 0) {
    int off = 0, eq_left = need_eq, my_off = 0, my_take = 0;
    for (int cc = 0; cc < nch; ++cc) {
      const int take = min(eq_left, chunk_eq[cc]);
      if (cc == c) {
        my_off = off;
        my_take = take;
      }
      off += chunk_above[cc] + chunk_gt[cc] + take;
      eq_left -= take;
    }
    sh_off = my_off;
    sh_take = my_take;
    sh_total = off;
  }
  // packed exclusive scan over the chunk (both counts < 2^13 per chunk)
  int n_gt = 0, n_eq = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    n_gt += key[j] > T;
    n_eq += (key[j] == T) && (T != kNegInfKey);
  }
  const int packed = (n_gt << 16) | n_eq;
  const int incl = wave_incl_scan_dpp(packed);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = incl - packed;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) before += w < wave ? wsum[w] : 0;
  int gt_before = before >> 16, eq_before = before & 0xffff;
  const int off = sh_off, eq_take = sh_take;
  int32_t* dst = out + static_cast<int64_t>(row) * out_stride;
  const int i0 = c * kChunk + 8 * tid;
  // slots stay below k by construction; the bound also holds if the scores were changed
  // between the launches
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (key[j] > T) {
      const int slot = off + gt_before + min(eq_before, eq_take);
      if (slot < k) dst[slot] = i0 + j;
      ++gt_before;
    } else if (key[j] == T && T != kNegInfKey) {
      const int slot = off + gt_before + eq_before;
      if (eq_before < eq_take && slot < k) dst[slot] = i0 + j;
      ++eq_before;
    }
  }
  if (c == nch - 1)
    for (int i = sh_total + tid; i < k; i += kThreads) dst[i] = -1;
}

int topk_multi_chunks(int64_t rows, int64_t cols) {
  if (cols <= kMultiMinG || cols > static_cast<int64_t>(kChunk) * kMaxChunks || rows > 65535) return 0;
  return static_cast<int>((cols + kChunk - 1) / kChunk);
}

// ---- two-level candidate selection, level one (select_candidate_blocks) -------------
//
// owlet1/indexer.py:14-40: block maxima of the scores (blocks of block_size positions,
// the tail block padded with -inf), the block holding the query's newest position
// ((compress_len - 1) // block_size) pinned to +inf, the top topk_blocks blocks with a
// score above -inf, expanded back to a per-position mask.  The top-k in between is
// mzk_topk_rows (lowest block index first among equal block scores).

// One thread per (row, block): the block maximum, or +inf for the newest (partial) block.
__global__ void candidate_pool_kernel(const float* __restrict__ logits, int64_t rows, int64_t width,
                                      int64_t row_stride, const int64_t* __restrict__ compress_lens, int block_size,
                                      int64_t nb, float* __restrict__ block_scores) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows * nb) return;
  const int64_t row = t / nb, blk = t - row * nb;
  const float* src = logits + row * row_stride;
  const int64_t p0 = blk * block_size;
  const int64_t p1 = p0 + block_size < width ? p0 + block_size : width;
  float m = -__builtin_huge_valf();
  for (int64_t p = p0; p < p1; ++p) m = fmaxf(m, src[p]);
  const int64_t cl = compress_lens[row];
  const int64_t last = cl > 0 ? (cl - 1) / block_size : -1;  // floor division (cl = 0 pins nothing)
  block_scores[t] = blk == last ? __builtin_huge_valf() : m;
}

// One workgroup per row: the selected blocks into an LDS bitmap, then mask[p] = bit(p / bs).
__global__ void __launch_bounds__(256) candidate_expand_kernel(const int32_t* __restrict__ block_idx, int topk,
                                                                int64_t width, int block_size, int nb,
                                                                uint8_t* __restrict__ mask, int64_t mask_stride) {
  extern __shared__ uint32_t bits[];  // nb bits
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nwords = (nb + 31) / 32;
  for (int i = tid; i < nwords; i += 256) bits[i] = 0u;
  __syncthreads();
  const int32_t* bi = block_idx + row * static_cast<int64_t>(topk);
  for (int i = tid; i < topk; i += 256) {
    const int b = bi[i];
    if (b >= 0 && b < nb) atomicOr(&bits[b >> 5], 1u << (b & 31));
  }
  __syncthreads();
  uint8_t* dst = mask + row * mask_stride;
  for (int64_t p = tid; p < width; p += 256) {
    const int64_t b = p / block_size;
    dst[p] = static_cast<uint8_t>((bits[b >> 5] >> (b & 31)) & 1u);
  }
}

// ---- selection formats ----------------------------------------------------------------

// The additive block bias of owlet1/indexer.py:158-165 from a top-k index list: row r of
// `bias` is 0 at the columns idx[r, :k] names (entries outside [0, G) are empty) and -inf
// elsewhere.  One workgroup per row: fill, barrier, scatter.
__global__ void __launch_bounds__(256) topk_bias_kernel(const int32_t* __restrict__ idx, int k, int64_t idx_stride,
                                                        int64_t G, float* __restrict__ bias, int64_t bias_stride) {
  const int64_t row = blockIdx.x;
  float* brow = bias + row * bias_stride;
  for (int64_t g = threadIdx.x; g < G; g += blockDim.x) brow[g] = -__builtin_huge_valf();
  __syncthreads();
  const int32_t* irow = idx + row * idx_stride;
  for (int j = threadIdx.x; j < k; j += blockDim.x) {
    const int32_t g = irow[j];
    if (g >= 0 && g < G) brow[g] = 0.0f;
  }
}

// The visible columns of an additive attention mask, in ascending order: a column is
// visible where the mask is 0, masked where it is -inf or the dtype's lowest finite value
// (what transformers' eager masks hold); anything else sets bit 0 of flags (a mask this
// conversion cannot represent), more than `cap` visible columns in a row sets bit 1.
// idx [rows, cap] (-1 after the last visible column), counts [rows].  One workgroup per row,
// 256 columns per step: a wave ballot ranks the visible lanes, LDS holds the wave totals.
template <int DT>
__global__ void __launch_bounds__(256) mask_to_indices_kernel(const void* __restrict__ mask, int64_t T,
                                                              int64_t row_stride, int cap, int32_t* __restrict__ idx,
                                                              int32_t* __restrict__ counts, int* __restrict__ flags) {
  __shared__ int wave_cnt[4];
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float lowest = DT == MZK_F32 ? -3.4028234663852886e38f : (DT == MZK_BF16 ? -3.3895313892515355e38f : -65504.0f);
  int32_t* irow = idx + row * static_cast<int64_t>(cap);
  int base = 0;
  bool bad = false;
  for (int64_t t0 = 0; t0 < T; t0 += 256) {
    const int64_t t = t0 + threadIdx.x;
    bool vis = false;
    if (t < T) {
      const float v = load_as_f32<DT>(mask, row * row_stride + t);
      vis = v == 0.0f;
      if (!vis && !(v == -__builtin_huge_valf() || v == lowest)) bad = true;
    }
    const uint64_t bal = __ballot(vis);
    const int rank = __popcll(bal & ((uint64_t{1} << lane) - 1));
    if (lane == 0) wave_cnt[wave] = __popcll(bal);
    __syncthreads();
    int off = base, total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (w < wave) off += wave_cnt[w];
      total += wave_cnt[w];
    }
    if (vis && off + rank < cap) irow[off + rank] = static_cast<int32_t>(t);
    base += total;
    __syncthreads();
  }
  for (int j = base + threadIdx.x; j < cap; j += 256) irow[j] = -1;
  if (threadIdx.x == 0) {
    counts[row] = base;
    if (base > cap) atomicOr(flags, 2);
  }
  if (bad) atomicOr(flags, 1);
}

template <int DT>
void launch_mask_to_indices(const void* mask, int64_t rows, int64_t T, int64_t rs, int cap, int32_t* idx,
                            int32_t* counts, int* flags, hipStream_t s) {
  mask_to_indices_kernel<DT><<<static_cast<unsigned>(rows), 256, 0, s>>>(mask, T, rs, cap, idx, counts, flags);
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
  // short rows take a workgroup sized to them (8 keys per thread), long ones 1024 threads
  if (G <= 8 * 256)
    topk_row_kernel<8, 256><<<nr, 256, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= 8 * 512)
    topk_row_kernel<8, 512><<<nr, 512, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= 8 * kThreads)
    topk_row_kernel<8, kThreads><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= 16 * kThreads)
    topk_row_kernel<16, kThreads><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= 32 * kThreads)
    topk_row_kernel<32, kThreads><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  else if (G <= kLdsKeys)
    topk_rows_kernel<true><<<nr, kThreads, static_cast<size_t>(G) * 4, s>>>(scores, row_stride, G, topk, out,
                                                                           out_stride);
  else
    topk_rows_kernel<false><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride);
  MZK_LAUNCH_CHECK("topk_rows");
  return MZK_OK;
}

extern "C" int mzk_topk_workspace_bytes(int64_t rows, int64_t cols, int64_t* bytes) {
  MZK_CHECK_ARG(rows >= 0 && cols >= 0 && bytes != nullptr, "topk_workspace_bytes: bad arguments");
  const int nch = topk_multi_chunks(rows, cols);
  *bytes = nch ? multi_ws(rows, nch).total : 0;
  return MZK_OK;
}

extern "C" int mzk_topk_rows_ws(const float* scores, int64_t rows, int64_t cols, int64_t row_stride, int topk,
                                int32_t* out, int64_t out_stride, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  const int nch = topk_multi_chunks(rows, cols);
  if (nch == 0 || rows == 0 || topk == 0)
    return mzk_topk_rows(scores, rows, cols, row_stride, topk, out, out_stride, stream);
  MZK_CHECK_ARG(topk > 0 && cols <= (int64_t(1) << 30) && topk <= (1 << 30), "topk_rows: bad sizes");
  MZK_CHECK_ARG(row_stride >= cols && out_stride >= topk, "topk_rows: strides smaller than the row");
  MZK_CHECK_ARG(out != nullptr && scores != nullptr, "topk_rows: null pointer");
  const MultiWs w = multi_ws(rows, nch);
  MZK_CHECK_ARG(workspace != nullptr && workspace_bytes >= w.total && aligned16(workspace),
                "topk_rows: rows of %lld keys need a 16-byte aligned workspace of %lld bytes", (long long)cols,
                (long long)w.total);
  hipStream_t s = as_stream(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int* hist = reinterpret_cast<int*>(ws + w.hist);
  int* above = reinterpret_cast<int*>(ws + w.above);
  int4* sel = reinterpret_cast<int4*>(ws + w.sel);
  uint2* cand = reinterpret_cast<uint2*>(ws + w.cand);
  const int G = static_cast<int>(cols);
  const dim3 grid(static_cast<unsigned>(nch), static_cast<unsigned>(rows));
  topk_chunk_hist_kernel<<<grid, kThreads, 0, s>>>(scores, row_stride, G, nch, hist);
  topk_chunk_gather_kernel<<<grid, kThreads, 0, s>>>(scores, row_stride, G, topk, nch, hist, above, sel, cand);
  topk_chunk_select_write_kernel<<<grid, kThreads, 0, s>>>(scores, row_stride, G, topk, nch, hist, above, sel, cand,
                                                            out, out_stride);
  MZK_LAUNCH_CHECK("topk_rows_ws");
  return MZK_OK;
}

extern "C" int mzk_candidate_topk(const float* scores, int64_t rows, int64_t slots, int64_t row_stride, int topk,
                                  const int32_t* cand_blocks, int64_t cand_stride, int n_blocks, int block_size,
                                  int32_t* out, int64_t out_stride, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && slots >= 0 && topk >= 0 && n_blocks >= 0 && block_size >= 1,
                "candidate_topk: negative size");
  MZK_CHECK_ARG(slots == static_cast<int64_t>(n_blocks) * block_size,
                "candidate_topk: the candidate axis holds n_blocks * block_size slots");
  MZK_CHECK_ARG(slots <= 32 * kThreads, "candidate_topk: at most %d candidate slots (got %lld)", 32 * kThreads,
                (long long)slots);
  MZK_CHECK_ARG(row_stride >= slots && out_stride >= topk && cand_stride >= n_blocks, "candidate_topk: bad strides");
  if (rows == 0 || topk == 0) return MZK_OK;
  if (slots == 0) return mzk_topk_rows(scores, rows, 0, row_stride, topk, out, out_stride, stream);  // all -1
  MZK_CHECK_ARG(rows <= 0x7fffffff, "candidate_topk: too many rows");
  MZK_CHECK_ARG(out != nullptr && (slots == 0 || (scores != nullptr && cand_blocks != nullptr)),
                "candidate_topk: null pointer");
  if (block_size != kMapBs) {  // other block sizes: the top-k, then the position map
    const int rc = mzk_topk_rows(scores, rows, slots, row_stride, topk, out, out_stride, stream);
    if (rc) return rc;
    return mzk_candidate_positions(out, rows, topk, out_stride, cand_blocks, cand_stride, n_blocks, block_size, out,
                                   out_stride, stream);
  }
  hipStream_t s = as_stream(stream);
  const int G = static_cast<int>(slots);
  const unsigned nr = static_cast<unsigned>(rows);
  const SlotMap sm{cand_blocks, cand_stride, n_blocks};
  if (G <= 8 * 256)
    topk_row_kernel<8, 256, true><<<nr, 256, 0, s>>>(scores, row_stride, G, topk, out, out_stride, sm);
  else if (G <= 8 * 512)
    topk_row_kernel<8, 512, true><<<nr, 512, 0, s>>>(scores, row_stride, G, topk, out, out_stride, sm);
  else if (G <= 8 * kThreads)
    topk_row_kernel<8, kThreads, true><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride, sm);
  else if (G <= 16 * kThreads)
    topk_row_kernel<16, kThreads, true><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride, sm);
  else
    topk_row_kernel<32, kThreads, true><<<nr, kThreads, 0, s>>>(scores, row_stride, G, topk, out, out_stride, sm);
  MZK_LAUNCH_CHECK("candidate_topk");
  return MZK_OK;
}

extern "C" int mzk_candidate_blocks_workspace_bytes(int64_t rows, int64_t width, int block_size, int topk_blocks,
                                                    int64_t* bytes) {
  MZK_CHECK_ARG(rows >= 0 && width >= 0 && block_size >= 1 && topk_blocks >= 0 && bytes != nullptr,
                "candidate_blocks_workspace_bytes: bad arguments");
  const int64_t nb = (width + block_size - 1) / block_size;
  int64_t tk = 0;
  MZK_CHECK_ARG(mzk_topk_workspace_bytes(rows, nb, &tk) == MZK_OK, "candidate_blocks_workspace_bytes: bad sizes");
  // block scores [rows, nb] fp32 | block indices [rows, topk_blocks] int32 | top-k workspace
  *bytes = round16(rows * nb * 4) + round16(rows * static_cast<int64_t>(topk_blocks) * 4) + tk;
  return MZK_OK;
}

extern "C" int mzk_candidate_blocks(const float* logits, int64_t rows, int64_t width, int64_t row_stride,
                                    const int64_t* compress_lens, int topk_blocks, int block_size, uint8_t* mask,
                                    int64_t mask_stride, int32_t* block_idx_out, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && width >= 0 && topk_blocks >= 0 && block_size >= 1 && block_size <= (1 << 20),
                "candidate_blocks: bad sizes");
  MZK_CHECK_ARG(row_stride >= width && (mask == nullptr || mask_stride >= width), "candidate_blocks: bad strides");
  if (rows == 0 || width == 0) return MZK_OK;
  const int64_t nb = (width + block_size - 1) / block_size;
  MZK_CHECK_ARG(nb <= (int64_t(1) << 24) && rows <= 0x7fffffff, "candidate_blocks: too many blocks");
  MZK_CHECK_ARG(logits && compress_lens && (mask || block_idx_out), "candidate_blocks: null pointer");
  int64_t need = 0;
  mzk_candidate_blocks_workspace_bytes(rows, width, block_size, topk_blocks, &need);
  MZK_CHECK_ARG(workspace && workspace_bytes >= need && aligned16(workspace),
                "candidate_blocks: needs a 16-byte aligned workspace of %lld bytes", (long long)need);
  hipStream_t s = as_stream(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* bscore = reinterpret_cast<float*>(ws);
  int32_t* bidx = block_idx_out ? block_idx_out : reinterpret_cast<int32_t*>(ws + round16(rows * nb * 4));
  void* tkws = ws + round16(rows * nb * 4) + round16(rows * static_cast<int64_t>(topk_blocks) * 4);
  const int64_t tk_bytes = need - (round16(rows * nb * 4) + round16(rows * static_cast<int64_t>(topk_blocks) * 4));
  const int64_t n = rows * nb;
  candidate_pool_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(logits, rows, width, row_stride,
                                                                                compress_lens, block_size, nb, bscore);
  if (topk_blocks > 0) {
    const int rc = mzk_topk_rows_ws(bscore, rows, nb, nb, topk_blocks, bidx, topk_blocks, tkws, tk_bytes, stream);
    if (rc) return rc;
  }
  if (mask) {
    const size_t lds = static_cast<size_t>((nb + 31) / 32) * 4;
    MZK_CHECK_ARG(lds <= 64 * 1024, "candidate_blocks: %lld blocks exceed the mask kernel's LDS bitmap", (long long)nb);
    candidate_expand_kernel<<<static_cast<unsigned>(rows), 256, lds, s>>>(bidx, topk_blocks, width, block_size,
                                                                           static_cast<int>(nb), mask, mask_stride);
  }
  MZK_LAUNCH_CHECK("candidate_blocks");
  return MZK_OK;
}

extern "C" int mzk_topk_bias(const int32_t* idx, int64_t rows, int topk, int64_t idx_row_stride, int64_t G,
                             float* bias, int64_t bias_row_stride, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && topk >= 0 && G >= 0 && idx_row_stride >= topk && bias_row_stride >= G,
                "topk_bias: bad sizes");
  if (rows == 0 || G == 0) return MZK_OK;
  MZK_CHECK_ARG(bias && (topk == 0 || idx), "topk_bias: null pointer");
  MZK_CHECK_ARG(rows <= 0x7fffffff, "topk_bias: too many rows");
  topk_bias_kernel<<<static_cast<unsigned>(rows), 256, 0, as_stream(stream)>>>(idx, topk, idx_row_stride, G, bias,
                                                                                 bias_row_stride);
  MZK_LAUNCH_CHECK("topk_bias");
  return MZK_OK;
}

extern "C" int mzk_mask_to_indices(const void* mask, int mask_dtype, int64_t rows, int64_t cols, int64_t row_stride,
                                   int cap, int32_t* idx, int32_t* counts, int* flags, void* stream) {
  MZK_CHECK_ARG(rows >= 0 && cols >= 0 && cap >= 0 && row_stride >= cols, "mask_to_indices: bad sizes");
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(mask && idx && counts && flags, "mask_to_indices: null pointer");
  MZK_CHECK_ARG(rows <= 0x7fffffff && cols <= 0x7fffffff, "mask_to_indices: too many rows or columns");
  MZK_DISPATCH_DT(mask_dtype, launch_mask_to_indices, mask, rows, cols, row_stride, cap, idx, counts, flags,
                  as_stream(stream));
  MZK_LAUNCH_CHECK("mask_to_indices");
  return MZK_OK;
}

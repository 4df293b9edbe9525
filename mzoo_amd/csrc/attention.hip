// Piece 5: sparse shared-latent MQA attention (window + dense + top-k gathered sources,
// per-head sink), split over the entry axis with an LSE combine.
//
// Semantics -- one softmax per (row, head) over the concatenation
//     [window entries ; dense compressed entries ; gathered top-k entries] + sink column,
// K == V (the single shared latent head), scale D^-0.5, sink only in the denominator:
//   src/mzoo/archs/owlet1/attention.py:42-71 (eager_attention_forward), :199-214;
//   src/mzoo/layers/attn/golden_ref.py:83-168 (levels window/compressed/sparse);
//   src/mzoo/layers/attn/csa2_attn/fwd.py:70-219 (index < 0 or >= G contributes nothing,
//   lse in natural log including the sink).
// A row is one query token (a decode row, or token t of a prefill), H heads, D channels.
//   window : tokens max(0, pos-W+1) .. pos of the row's batch (ring slot tok % cap, or a
//            linear [B, S] array when cap == 0)
//   dense  : entries 0 .. min(cap, (pos+1)/ratio)-1 of a compressed cache
//   sparse : main[idx[row, s]] for s < topk (idx < 0 or >= G skipped)
// Entry formats: bf16 [D] rows, or the 656 B FP8-b128 latent entry (512 e4m3 + 4 fp32
// scales + 64 bf16 rope), dequantized on load.
//
// Tiling (MI355X): one workgroup = one (row, split, group of <= 64 heads); HG x DS waves,
// HG = head groups of 32 (the MFMA N axis), DS = number of D-parts (2 when D > 256, so a
// wave's q fragments + O^T accumulators fit one SIMD's registers).  Per 32-entry tile:
//   1. the tile (fetched from HBM into registers while the previous tile computed) is
//      dequantized to bf16 into LDS, Kt[entry][d];
//   2. S^T[32 entries x 32 heads] = Kt . Q^T on v_mfma_f32_32x32x16_bf16, each wave over its
//      D-part, partial sums exchanged through LDS (fixed order: part 0 + part 1);
//   3. online softmax in the exp2 domain, lane-local per head (lane l holds head l%32);
//   4. O^T[d x 32 heads] += V^T . P^T on MFMA, each wave owning its D-part of O: P^T stays
//      in the registers the S^T result left it in, and the V^T operand is gathered from
//      Kt columns in the matching entry order.
// The workgroup writes either the final bf16 output + lse (one split) or fp32 partials
// (unnormalized O, running max m, sum l) that mzk combine kernel merges with the sink.
#include <type_traits>

#include <mutex>

#include "common.h"
#include "topk_core.h"

namespace mzk {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));

enum { kFmtBf16 = 0, kFmtFp8 = 1 };

__device__ __forceinline__ __attribute__((address_space(3))) v4s* lds_v4s(const uint8_t* p) {
  return (__attribute__((address_space(3))) v4s*)(p);
}

constexpr int kTile = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnParams {
  const uint16_t* q;  // [rows, H, D] bf16
  int64_t rows;       // B * S
  int64_t S;          // rows per batch: row = b * S + s
  const int64_t* positions;  // [rows] absolute position of each row
  // window source
  const uint8_t* win;
  int64_t win_batch_entries;
  int win_cap;  // ring capacity; 0 = linear (token t at entry t)
  int window;
  // dense source
  const uint8_t* dense;
  int64_t dense_batch_entries;
  int dense_cap;
  int dense_ratio;
  // sparse source
  const uint8_t* main;
  int64_t main_batch_entries;
  int64_t G;
  const int32_t* idx;
  int64_t idx_row_stride;
  int topk;
  // heads / sink
  int H;
  const float* sinks;  // [H] or null
  float scale_log2;    // D^-0.5 * log2(e)
  int nsplit;
  // outputs
  uint16_t* out;  // [rows, H, D] bf16 (nsplit == 1)
  float* lse;     // [B, H, S]       (nsplit == 1)
  uint16_t* part_o;  // [rows, split_stride, D/16, H, 16] bf16: the split's output O / l, by 16-channel group
  float* part_ml;    // [rows, split_stride, H, 2]: the split's running max m (log2 units) and sum l
  int split_stride;  // splits per row in the workspace (nsplit, or more when launches share it)
  int write_final;   // one split writes the final output and lse instead of partials
  // RoPE of the rope slice (channels NOPE .. D-1, FP8 latent rows): null, or cos / sin
  // [rows, (D - NOPE) / 2] bf16 -- q arrives unrotated and is rotated on load, and the
  // final output (nsplit == 1) gets the inverse rotation
  const uint16_t* rope_cos;
  const uint16_t* rope_sin;
  // The split merge inside the launch (null: a merge launch follows): per (row, 64-head
  // group) a record of four words -- the XCC registration (64 bits, 8 per XCC: the group's
  // workgroups that started there), the arrivals, the departures -- zero between launches;
  // merge_err is set when a workgroup gave up waiting for its group.
  uint32_t* merge_rec;
  uint32_t* merge_err;
  int merge_fence;  // every workgroup takes the release / acquire path (a test mode)
  // The sparse list selected in the launch (decode, the SEL kernel instance; idx unused):
  // the top-topk of the row's sel_scores [rows, sel_stride] fp32 over G keys, in the top-k
  // launch's form (ascending picks, then -1), which the row's first workgroup also writes to
  // sel_out [rows, sel_out_stride] int32.
  const float* sel_scores;
  int64_t sel_stride;
  int32_t* sel_out;
  int64_t sel_out_stride;
};

template <int FMT, int D, int NOPE>
struct Layout {
  static constexpr int kEntryBytes = FMT == kFmtFp8 ? NOPE + 4 * (NOPE / 128) + 2 * (D - NOPE) : 2 * D;
  // An entry is fetched as 16-byte pieces: fp8 = NOPE/16 code pieces (16 e4m3 codes each)
  // followed by (D-NOPE)/8 rope pieces (8 bf16 each); bf16 = D/8 pieces of 8 channels.
  static constexpr int kCodePieces = FMT == kFmtFp8 ? NOPE / 16 : 0;
  static constexpr int kPieces = FMT == kFmtFp8 ? NOPE / 16 + (D - NOPE) / 8 : D / 8;
};

// Entry held by register j of lane l in a 32x32 MFMA result: 8*(j/4) + 4*(l/32) + j%4.
__device__ __forceinline__ int c_entry(int j, int lane) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }

// Workgroup barrier that waits only for this wave's LDS operations (not for vector
// memory: the next tile's loads stay in flight across it).  The "memory" clobber keeps
// the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

constexpr int kIdxCap = 4096;       // sparse indices of one split staged in LDS (D <= 256 kernel)
constexpr int kSplitIdxCap = 1024;  // the same for the D-split kernel (its LDS holds three tiles)
constexpr int kAllTabCap = 1024;    // D-split kernel: splits of at most this many entries keep every tile's table

typedef const uint8_t __attribute__((address_space(1)))* gptr_t;  // global (not flat) loads
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ T gload(gptr_t p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

// One fetched 16-byte piece of an entry (held in registers a tile ahead of use).
struct Piece {
  u32x4 v;  // fp8 code piece: 16 codes; rope / bf16 piece: 8 bf16
  float s;  // fp8 code piece: its 128-channel block scale
};

template <int FMT, int D, int NOPE>
__device__ __forceinline__ Piece fetch_piece(gptr_t e, int q) {
  using L = Layout<FMT, D, NOPE>;
  Piece r;
  r.s = 1.0f;
  if constexpr (FMT == kFmtFp8) {
    constexpr int NB = NOPE / 128;
    if (q < L::kCodePieces) {
      r.v = gload<u32x4>(e + 16 * q);
      r.s = gload<float>(e + NOPE + 4 * (q >> 3));
    } else {
      r.v = gload<u32x4>(e + NOPE + 4 * NB + 16 * (q - L::kCodePieces));
    }
  } else {
    r.v = gload<u32x4>(e + 16 * q);
  }
  return r;
}

// Writes piece q of an entry to its bf16 row in LDS: e4m3 codes times the pow2 block scale
// through the hardware conversion (exact in bf16); rope / bf16 pieces as they are.
template <int FMT, int D, int NOPE>
__device__ __forceinline__ void store_piece(uint8_t* krow, const Piece& r, int q) {
  using L = Layout<FMT, D, NOPE>;
  if constexpr (FMT == kFmtFp8) {
    if (q < L::kCodePieces) {
      *reinterpret_cast<uint4*>(krow + 32 * q) = dequant_fp8x8_bf16(uint2{r.v.x, r.v.y}, r.s);
      *reinterpret_cast<uint4*>(krow + 32 * q + 16) = dequant_fp8x8_bf16(uint2{r.v.z, r.v.w}, r.s);
    } else {
      *reinterpret_cast<uint4*>(krow + 2 * NOPE + 16 * (q - L::kCodePieces)) = uint4{r.v.x, r.v.y, r.v.z, r.v.w};
    }
  } else {
    *reinterpret_cast<uint4*>(krow + 16 * q) = uint4{r.v.x, r.v.y, r.v.z, r.v.w};
  }
}

// One (row, split, head group)'s share of the row's virtual entry list
// [window nw | dense nd | sparse ns], the entry tables of its tiles, and the register
// prefetch of a tile.  Shared by both kernels.
template <int FMT, int D, int NOPE, int NT, int NSLOT = 2>
struct RowPlan {
  using L = Layout<FMT, D, NOPE>;
  static constexpr int TPE = NT / kTile;                          // threads per entry
  static constexpr int PPT = (L::kPieces + TPE - 1) / TPE;        // pieces per thread

  int64_t row, b, pos;
  int split, hgrp;
  int nw, nwd, v_begin, v_end, ntiles, sp_begin, win_first;
  int64_t g_lim;
  const uint8_t* win_b;
  const uint8_t* dense_b;
  const uint8_t* main_b;
  const uint8_t** tab_ptr;   // [NSLOT][kTile] in LDS: tile t uses slot t & slot_mask
  uint32_t* tab_mask;        // [NSLOT] in LDS
  uint32_t slot_mask = NSLOT - 1;  // all the split's tables at once (build_all_tables): ~0
  // typed address spaces: a generic pointer would make these FLAT loads, which count
  // against the LDS wait counter too and force every later LDS wait to drain completely
  const __attribute__((address_space(3))) int32_t* sidx;     // this split's sparse indices (the first sidx_cap), in LDS
  const __attribute__((address_space(1))) int32_t* idx_row;  // the row's sparse indices in global memory
  int sidx_cap;

  // Workgroup -> (row, split, head group).  Workgroups are dealt to the 8 XCDs round-robin
  // (workgroup i runs on XCD i % 8).  ROW_XCD (the decode kernel instance) with rows a
  // multiple of 8: every workgroup of row r runs on XCD r % 8: the head groups of a (row, split), which read the same entries, and
  // the splits, which read the same q, share an L2, and so does the merge launch, which maps
  // its workgroups the same way and finds the row's partials there.  Otherwise the head
  // groups of one (row, split) get consecutive slots of one XCD.
  // 32-bit arithmetic: the host keeps the grid below 2^31 workgroups and the list
  // lengths (window + dense_cap + topk) below 2^31.
  __device__ void init(const AttnParams& p, int heads_per_wg) {
    locate(p, heads_per_wg);
    plan(p, p.positions[row]);
  }

  // The workgroup's (row, split, head group); no memory access.  (ROW_XCD is a template
  // argument so that the other kernel instances compile without its branch: their code,
  // the prefill's long tile loops included, stays as it was.)
  template <bool ROW_XCD = false>
  __device__ void locate(const AttnParams& p, int heads_per_wg) {
    const uint32_t nhg = static_cast<uint32_t>((p.H + heads_per_wg - 1) / heads_per_wg);
    const uint32_t units = static_cast<uint32_t>(p.rows) * static_cast<uint32_t>(p.nsplit);
    const uint32_t L0 = blockIdx.x;
    uint32_t unit;
    if (ROW_XCD && (p.rows & 7) == 0) {  // row-per-XCD
      const uint32_t per_row = static_cast<uint32_t>(p.nsplit) * nhg;
      const uint32_t k = L0 >> 3;
      const uint32_t r8 = k / per_row, i = k - r8 * per_row;
      hgrp = static_cast<int>(i % nhg);
      unit = (r8 * 8 + (L0 & 7u)) * static_cast<uint32_t>(p.nsplit) + i / nhg;
    } else if (ROW_XCD && p.merge_rec != nullptr && ((static_cast<uint32_t>(p.rows) * nhg) & 7u) == 0) {
      // (row, head group)-per-XCD, for the in-launch merge of fewer rows: group g = row * nhg
      // + head group runs on XCD g % 8
      const uint32_t k = L0 >> 3;
      const uint32_t g8 = k / static_cast<uint32_t>(p.nsplit);
      const uint32_t grp = g8 * 8 + (L0 & 7u);
      hgrp = static_cast<int>(grp % nhg);
      unit = (grp / nhg) * static_cast<uint32_t>(p.nsplit) + (k - g8 * static_cast<uint32_t>(p.nsplit));
    } else if ((units & 7u) == 0) {
      const uint32_t w = L0 >> 3;
      hgrp = static_cast<int>(w % nhg);
      unit = (w / nhg) * 8 + (L0 & 7u);
    } else {
      hgrp = static_cast<int>(L0 % nhg);
      unit = L0 / nhg;
    }
    uint32_t row32 = unit / static_cast<uint32_t>(p.nsplit);
    split = static_cast<int>(unit - row32 * static_cast<uint32_t>(p.nsplit));
    // with several rows per batch (prefill) a row's entry count grows with its position:
    // the last rows go first, so the longest workgroups do not form the tail
    if (p.S > 1) row32 = static_cast<uint32_t>(p.rows) - 1u - row32;
    row = row32;
    b = row32 / static_cast<uint32_t>(p.S);
  }

  // The row's entry list split, given its absolute position; `ns_used` (-1: topk) is the
  // length of the sparse list to walk.
  __device__ void plan(const AttnParams& p, int64_t row_pos, int ns_used = -1) {
    pos = row_pos < -1 ? -1 : row_pos;  // a negative position sees no window or dense entry
    nw = static_cast<int>(pos + 1 < p.window ? pos + 1 : p.window);
    int nd = 0;
    if (p.dense) {
      const int64_t n = (pos + 1) / p.dense_ratio;
      nd = static_cast<int>(n < p.dense_cap ? n : p.dense_cap);
    }
    const int ns = p.main ? (ns_used >= 0 ? ns_used : p.topk) : 0;
    nwd = nw + nd;
    const int total = nwd + ns;
    int chunk = (total + p.nsplit - 1) / p.nsplit;
    chunk = (chunk + kTile - 1) / kTile * kTile;
    v_begin = split * chunk;
    v_end = v_begin + chunk < total ? v_begin + chunk : total;
    ntiles = v_end > v_begin ? (v_end - v_begin + kTile - 1) / kTile : 0;
    sp_begin = v_begin > nwd ? v_begin - nwd : 0;

    win_b = p.win + b * p.win_batch_entries * L::kEntryBytes;
    dense_b = p.dense ? p.dense + b * p.dense_batch_entries * L::kEntryBytes : nullptr;
    main_b = p.main ? p.main + b * p.main_batch_entries * L::kEntryBytes : nullptr;
    // ring slot of window entry 0 (token pos - nw + 1); entry v sits v slots later
    win_first = static_cast<int>(p.win_cap ? (pos - nw + 1) % p.win_cap : pos - nw + 1);
    g_lim = p.G < 0x7fffffff ? p.G : 0x7fffffff;
  }

  // plan() in two parts, for the selecting kernel: the row's (plan_row, given its position;
  // its divisions run while the scores are in flight) and the split's (plan_split, given the
  // sparse list's valid length once it is selected).  The same results as plan().
  __device__ void plan_row(const AttnParams& p, int64_t row_pos) {
    pos = row_pos < -1 ? -1 : row_pos;
    nw = static_cast<int>(pos + 1 < p.window ? pos + 1 : p.window);
    int nd = 0;
    if (p.dense) {
      const int64_t n = (pos + 1) / p.dense_ratio;
      nd = static_cast<int>(n < p.dense_cap ? n : p.dense_cap);
    }
    nwd = nw + nd;
    win_b = p.win + b * p.win_batch_entries * L::kEntryBytes;
    dense_b = p.dense ? p.dense + b * p.dense_batch_entries * L::kEntryBytes : nullptr;
    main_b = p.main ? p.main + b * p.main_batch_entries * L::kEntryBytes : nullptr;
    win_first = static_cast<int>(p.win_cap ? (pos - nw + 1) % p.win_cap : pos - nw + 1);
    g_lim = p.G < 0x7fffffff ? p.G : 0x7fffffff;
  }
  __device__ void plan_split(const AttnParams& p, int ns_used) {
    const int ns = p.main ? ns_used : 0;
    const int total = nwd + ns;
    int chunk = (total + p.nsplit - 1) / p.nsplit;
    chunk = (chunk + kTile - 1) / kTile * kTile;
    v_begin = split * chunk;
    v_end = v_begin + chunk < total ? v_begin + chunk : total;
    ntiles = v_end > v_begin ? (v_end - v_begin + kTile - 1) / kTile : 0;
    sp_begin = v_begin > nwd ? v_begin - nwd : 0;
  }

  // Stage up to `cap` indices of this split's slice of the sparse list in LDS, so the tile
  // loop reads them from there; positions beyond the cap are read from global memory.
  // The caller synchronises before the slice is read.
  __device__ void stage_indices(const AttnParams& p, int32_t* sidx_lds, int cap, int tid) {
    const int sp_end = v_end > nwd ? v_end - nwd : 0;
    idx_row = p.idx ? (const __attribute__((address_space(1))) int32_t*)(p.idx + row * p.idx_row_stride) : nullptr;
    const int lim = sp_end < sp_begin + cap ? sp_end : sp_begin + cap;
    for (int s = sp_begin + tid; s < lim; s += NT) sidx_lds[s - sp_begin] = idx_row[s];
    sidx = (const __attribute__((address_space(3))) int32_t*)(sidx_lds);
    sidx_cap = cap;
  }

  // Request the row's first 4*NT sparse indices, one 16-byte load per thread, before the
  // row's position (which fixes this split's slice) is known, so the two loads overlap.
  // Returns false (and loads nothing) unless the whole list fits and its row is 16-byte
  // aligned; then stage_indices reads it after the position.
  __device__ bool prefetch_indices(const AttnParams& p, int tid, v4i& pre) {
    idx_row = p.idx ? (const __attribute__((address_space(1))) int32_t*)(p.idx + row * p.idx_row_stride) : nullptr;
    const bool ok = idx_row != nullptr && p.topk > 0 && p.topk <= 4 * NT && (p.topk & 3) == 0 &&
                    (reinterpret_cast<uintptr_t>(idx_row) & 15u) == 0;
    // branch-free: every thread loads from a valid address (the query, 16-byte aligned, when
    // the list is not used), so the compiler's in-order wait counts stay exact
    const int at = 4 * tid < p.topk ? 4 * tid : p.topk - 4;
    const __attribute__((address_space(1))) v4i* src =
        ok ? reinterpret_cast<const __attribute__((address_space(1))) v4i*>(idx_row + at)
           : (const __attribute__((address_space(1))) v4i*)(p.q);
    pre = *src;
    if (!ok || 4 * tid >= p.topk) pre = v4i{-1, -1, -1, -1};
    return ok;
  }

  // stage_indices from the prefetched list (prefetch_indices returned true): the thread
  // holding list positions 4tid..4tid+3 writes those inside the slice.
  __device__ void stage_prefetched(int32_t* sidx_lds, int cap, int tid, const v4i& pre) {
    const int sp_end = v_end > nwd ? v_end - nwd : 0;
    const int lim = sp_end < sp_begin + cap ? sp_end : sp_begin + cap;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = 4 * tid + j;
      if (s >= sp_begin && s < lim) sidx_lds[s - sp_begin] = pre[j];
    }
    sidx = (const __attribute__((address_space(3))) int32_t*)(sidx_lds);
    sidx_cap = cap;
  }

  // With the whole list prefetched (prefetch_indices returned true): the number of its
  // leading valid indices (0 <= g < G) when every valid index precedes every invalid one --
  // the form the top-k launch writes (ascending picks, then -1) -- else topk.  Walking only
  // that prefix skips tiles that would be all masked.  `wred` is 2 * (NT / 64) ints of LDS;
  // two workgroup barriers.
  __device__ int valid_prefix(const AttnParams& p, int tid, const v4i& pre, int* wred) const {
    constexpr int NW = NT / 64;
    const int lane = tid & 63, wave = tid >> 6;
    const int64_t glim = p.G;
    auto valid = [&](int j) { return 4 * tid + j < p.topk && pre[j] >= 0 && pre[j] < glim; };
    int c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) c += valid(j);
    int wc = c;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) wc += __shfl_xor(wc, m, 64);
    if (lane == 0) wred[wave] = wc;
    __syncthreads();
    int n = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) n += wred[w];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) bad |= valid(j) && 4 * tid + j >= n;
    const uint64_t bb = __ballot(bad);
    if (lane == 0) wred[NW + wave] = bb != 0;
    __syncthreads();
    int nb = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) nb += wred[NW + w];
    return nb ? p.topk : n;
  }

  // sparse index of list position v (-1 outside the sparse part of this split)
  __device__ int slot(int v) const {
    if (v < nwd || v >= v_end) return -1;
    const int s = v - nwd - sp_begin;
    if (s < sidx_cap) return sidx[s];
    return idx_row[sp_begin + s];
  }

  // address of entry e of tile t (null if empty); g = its sparse index (slot of the entry)
  __device__ const uint8_t* entry_ptr(const AttnParams& p, int t, int e, int g) const {
    const int v = v_begin + t * kTile + e;
    const uint8_t* ptr = nullptr;
    if (v < v_end) {
      if (v < nw) {
        int slot_w = win_first + v;
        if (p.win_cap && slot_w >= p.win_cap) slot_w -= p.win_cap;
        ptr = win_b + static_cast<int64_t>(slot_w) * L::kEntryBytes;
      } else if (v < nwd) {
        ptr = dense_b + static_cast<int64_t>(v - nw) * L::kEntryBytes;
      } else if (g >= 0 && g < g_lim) {
        ptr = main_b + static_cast<int64_t>(g) * L::kEntryBytes;
      }
    }
    return ptr;
  }

  // entry table of tile t (threads 0..31); g = this thread's prefetched sparse index
  __device__ void build_table(const AttnParams& p, int t, int g, int tid) {
    if (tid < kTile) {
      const uint8_t* ptr = entry_ptr(p, t, tid, g);
      tab_ptr[(t & slot_mask) * kTile + tid] = ptr;
      const uint64_t bal = __ballot(ptr != nullptr);
      if (tid == 0) tab_mask[t & slot_mask] = static_cast<uint32_t>(bal);
    }
  }

  // entry tables of tiles 0..3 at once (after the indices are staged): thread tid < 4*kTile
  // fills entry tid % kTile of tile tid / kTile, two tiles per wave
  __device__ void build_first_tables(const AttnParams& p, int tid) {
    static_assert(NSLOT >= 4 && NT >= 4 * kTile, "four tables in flight");
    if (tid < 4 * kTile) {
      const int t = tid / kTile, e = tid % kTile;
      const uint8_t* ptr = entry_ptr(p, t, e, slot(v_begin + t * kTile + e));
      tab_ptr[t * kTile + e] = ptr;
      const uint64_t bal = __ballot(ptr != nullptr);
      if (e == 0) tab_mask[t] = static_cast<uint32_t>(bal >> (32 * (t & 1)));
    }
  }

  // Tables the D-split tile loop reads: tiles 0..3 (its prologue) and up to three past the
  // last tile (it fetches tile u+3 while at tile u), whose entries are all empty.
  __device__ int table_tiles() const { return ntiles + 3 > 4 ? ntiles + 3 : 4; }

  // Every entry table the tile loop reads (table_tiles()), at once, when they fit `CAP`
  // pointers at `all` (which may overlap the staged sparse indices: each thread reads its
  // indices before a barrier, then writes).  Tile t then uses table t, and the tile loop
  // builds none.  Entry e = tid + NT * r; a wave's ballot covers tiles 2w' and 2w'+1.
  // One workgroup barrier; the caller synchronises before the tables are read.
  template <int CAP>
  __device__ void build_all_tables(const AttnParams& p, int tid, const uint8_t** all, uint32_t* masks) {
    static_assert(CAP % NT == 0 && NT % 64 == 0, "whole waves per round");
    constexpr int R = CAP / NT;
    const int n = table_tiles() * kTile;  // <= CAP (the caller checks)
    int g[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = tid + NT * r;
      g[r] = e < n ? slot(v_begin + e) : -1;
    }
    __syncthreads();  // every staged index is read before the tables overwrite them
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = tid + NT * r;
      const bool in = e < n;
      const uint8_t* ptr = in ? entry_ptr(p, e / kTile, e % kTile, g[r]) : nullptr;
      if (in) all[e] = ptr;
      const uint64_t bal = __ballot(ptr != nullptr);
      const int lane = tid & 63;
      if (in && (lane & 31) == 0) masks[e / kTile] = static_cast<uint32_t>(lane ? bal >> 32 : bal);
    }
    tab_ptr = all;
    tab_mask = masks;
    slot_mask = ~0u;
  }

  // The tile's pieces for this thread: entry tid / TPE, pieces (tid % TPE) + TPE*k, so the
  // TPE threads of an entry read TPE consecutive 16-byte pieces per load instruction.
  // Empty slots load zeros.
  __device__ void fetch(int t, int tid, Piece (&raw)[PPT]) const {
    const gptr_t e = (gptr_t)(tab_ptr[(t & slot_mask) * kTile + tid / TPE]);
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = tid % TPE + TPE * k;
      raw[k].v = u32x4{0u, 0u, 0u, 0u};
      raw[k].s = 1.0f;
      if (e != nullptr && q < L::kPieces) raw[k] = fetch_piece<FMT, D, NOPE>(e, q);
    }
  }

  // Dequantize the fetched pieces into this thread's entry row of a bf16 tile in LDS.
  __device__ void store(uint8_t* kt, int kt_pitch, int tid, const Piece (&raw)[PPT]) const {
    uint8_t* krow = kt + (tid / TPE) * kt_pitch;
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = tid % TPE + TPE * k;
      if (q < L::kPieces) store_piece<FMT, D, NOPE>(krow, raw[k], q);
    }
  }
};

// V^T operand of O^T += V^T . P^T for one 32-channel block and the two 16-entry K-steps,
// read from a bf16 tile with ds_read_b64_tr_b16: inside a 16-lane group, lane i receives
// element i%4 of the 4-element rows the lanes 4k + i/4 (k = 0..3) point at.  Lane j
// therefore points at Kt[e0 + j/4][d0 + 4*(j%4)] and receives Kt[e0 + k][d0 + i] for
// k = 0..3: four consecutive entries of its own channel, two reads per fragment.
// K-step ks covers entries 16ks + {0..3, 8..11} + 4*half (the S^T register order).
template <int KT_PITCH>
__device__ __forceinline__ void pv_block(const uint8_t* tp, const v8bf& pf0, const v8bf& pf1, v16f& acc) {
  const v4s r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp));                  // entries 0-3 (+4h)
  const v4s r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 8 * KT_PITCH));   // entries 8-11
  const v4s r2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 16 * KT_PITCH));  // entries 16-19
  const v4s r3 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 24 * KT_PITCH));  // entries 24-27
  const v8bf a0 = __builtin_bit_cast(v8bf, v8s{r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]});
  const v8bf a1 = __builtin_bit_cast(v8bf, v8s{r2[0], r2[1], r2[2], r2[3], r3[0], r3[1], r3[2], r3[3]});
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, pf0, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, pf1, acc, 0, 0, 0);
}

// Lane offset of the V^T read pattern above inside a tile, for channel block base d_base.
template <int KT_PITCH>
__device__ __forceinline__ int pv_lane_offset(int lane, int d_base) {
  const int grp = lane >> 4;  // 16-lane group: channel half (grp & 1), entry half (grp >> 1)
  const int j = lane & 15;
  const int e0 = 4 * (grp >> 1) + (j >> 2);
  return e0 * KT_PITCH + 2 * (d_base + 16 * (grp & 1) + 4 * (j & 3));
}

// Stores one 32-channel O^T block of a head.  Lane (head, half) holds channels
// 8 g4 + 4 half + [0, 4) of the block as the bf16 pairs w[2 g4], w[2 g4 + 1]; one
// v_permlane32_swap per word pair (the upper half-wave's first operand trades places with
// the lower half-wave's second) leaves each lane 8 consecutive channels per two g4, so
// the two lanes of a head write 32 contiguous bytes per store instead of two 8-byte
// pieces 8 bytes apart.  Both lanes of a head must execute it together.
__device__ __forceinline__ void store_o_block(uint16_t* blk, const uint32_t (&w)[8], int half) {
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(w[4 * pr], w[4 * pr + 2], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(w[4 * pr + 1], w[4 * pr + 3], false, false);
    *reinterpret_cast<uint4*>(blk + 16 * pr + 8 * half) = uint4{s0[0], s1[0], s0[1], s1[1]};
  }
}

// Final bf16 output + lse (one split) or fp32 partials (several) for one lane's head and
// O^T blocks [b_lo, b_lo + nb): acc[db][j] holds O^T[d][head], d = (b_lo+db)*32 + c_entry(j).
template <int D, int NOPE, int NDBM>
__device__ __forceinline__ void write_result(const AttnParams& p, int64_t row, int64_t b, int split, int head, int half,
                                             bool lse_lane, int b_lo, int nb, float m_run, float l_run,
                                             const v16f (&acc)[NDBM]) {
  if (p.write_final) {
    float m_fin = m_run, l_fin = l_run, o_scale;
    if (p.sinks) {
      const float sk = p.sinks[head] * kLog2e;
      const float mm = fmaxf(m_run, sk);
      const float a = m_run == -__builtin_huge_valf() ? 0.0f : exp2f(m_run - mm);
      l_fin = l_run * a + exp2f(sk - mm);
      m_fin = mm;
      o_scale = a / l_fin;
    } else {
      o_scale = 1.0f / l_fin;
    }
    uint16_t* orow = p.out + row * p.H * D + static_cast<uint32_t>(head * D + b_lo * 32);
#pragma unroll
    for (int db = 0; db < NDBM; ++db) {
      if (db < nb) {
        uint32_t w[8];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d0 = db * 32 + 8 * g4 + 4 * half;
          uint32_t w0 = f32_to_bf16(acc[db][4 * g4 + 0] * o_scale) |
                        (static_cast<uint32_t>(f32_to_bf16(acc[db][4 * g4 + 1] * o_scale)) << 16);
          uint32_t w1 = f32_to_bf16(acc[db][4 * g4 + 2] * o_scale) |
                        (static_cast<uint32_t>(f32_to_bf16(acc[db][4 * g4 + 3] * o_scale)) << 16);
          if constexpr (NOPE < D) {
            // the inverse rotation of the bf16 output (owlet1/attention.py:226)
            const int ch = b_lo * 32 + d0;
            if (p.rope_cos && ch >= NOPE) {
              const int64_t ci = row * ((D - NOPE) / 2) + (ch - NOPE) / 2;
              const uint32_t cp = *reinterpret_cast<const uint32_t*>(p.rope_cos + ci);
              const uint32_t sp = *reinterpret_cast<const uint32_t*>(p.rope_sin + ci);
              w0 = rope_pair_bf16(w0, bf16_to_f32(static_cast<uint16_t>(cp & 0xffffu)),
                                  -bf16_to_f32(static_cast<uint16_t>(sp & 0xffffu)));
              w1 = rope_pair_bf16(w1, bf16_to_f32(static_cast<uint16_t>(cp >> 16)),
                                  -bf16_to_f32(static_cast<uint16_t>(sp >> 16)));
            }
          }
          w[2 * g4] = w0;
          w[2 * g4 + 1] = w1;
        }
        store_o_block(orow + db * 32, w, half);
      }
    }
    if (lse_lane) {
      const int64_t s_idx = row % p.S;
      p.lse[(b * p.H + head) * p.S + s_idx] = (m_fin + __log2f(l_fin)) * kLn2;
    }
  } else {
    // the split's own normalized output in bf16 (a split that saw no entry writes zeros), in
    // 16-channel groups with the heads innermost: a store instruction of the two group halves
    // the permlane swap gives a head's two lanes covers 32 heads x 32 bytes, 1 KB contiguous
    const float inv_l = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    uint16_t* pbase = p.part_o + (row * p.split_stride + split) * p.H * static_cast<int64_t>(D);
#pragma unroll
    for (int db = 0; db < NDBM; ++db) {
      if (db < nb) {
        uint32_t w[8];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          w[2 * g4] = pack_bf16x2(acc[db][4 * g4] * inv_l, acc[db][4 * g4 + 1] * inv_l);
          w[2 * g4 + 1] = pack_bf16x2(acc[db][4 * g4 + 2] * inv_l, acc[db][4 * g4 + 3] * inv_l);
        }
        // groups 2 (b_lo + db) and 2 (b_lo + db) + 1 of the head
        uint16_t* grp = pbase + static_cast<uint32_t>((b_lo + db) * p.H * 32 + head * 16);
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const auto s0 = __builtin_amdgcn_permlane32_swap(w[4 * pr], w[4 * pr + 2], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(w[4 * pr + 1], w[4 * pr + 3], false, false);
          *reinterpret_cast<uint4*>(grp + static_cast<uint32_t>(pr * p.H * 16) + 8 * half) = uint4{s0[0], s1[0], s0[1], s1[1]};
        }
      }
    }
    if (lse_lane) {
      float* ml = p.part_ml + (row * p.split_stride + split) * p.H * 2 + static_cast<uint32_t>(head * 2);
      ml[0] = m_run;
      ml[1] = l_run;
    }
  }
}

constexpr float kLazy = 8.0f;  // log2 headroom before the running max must be raised

// ---- the split merge's arithmetic (the merge launch and the in-launch merge share it) ----
// Split s contributes its normalized output O_s with weight l_s exp2(m_s - M) / L, where
// M = max(m_s, sink) and L = sum_s l_s exp2(m_s - M) + exp2(sink - M).  Splits are merged
// kCombineRegSplits at a time into a running (M, L, acc) -- the sink first, as a split of
// weight 1 at sk -- so 8 or fewer splits are a single pass with the global maximum.  A split
// that saw no entry (l = 0) contributes nothing (its output is zeros, its m may be -inf).
constexpr int kCombineRegSplits = 8;

// NP 16-byte pieces (8 channels each) of one (row, head): piece i of split s at
// po + s * sstride + (i / 2) * gstride + 8 * (i % 2) (gstride: the next 16-channel group),
// the split's (m, l) at ml + 2 s H.  The loads of PRE splits are issued before any is used.
template <int NP, int PRE>
__device__ __forceinline__ void merge_pieces(const uint16_t* po, int64_t sstride, int64_t gstride, const float* ml,
                                             int nsplit, int H, float sk, bool has_sink, float (&acc)[8 * NP],
                                             float& M, float& L) {
  static_assert(PRE % kCombineRegSplits == 0, "whole chunks per load batch");
#pragma unroll
  for (int i = 0; i < 8 * NP; ++i) acc[i] = 0.0f;
  M = sk;
  L = has_sink ? 1.0f : 0.0f;
  for (int s0 = 0; s0 < nsplit; s0 += PRE) {
    float2 ms[PRE];
    uint4 v[PRE][NP];
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
      if (s0 + j < nsplit) {
        ms[j] = *reinterpret_cast<const float2*>(ml + 2 * (s0 + j) * H);
#pragma unroll
        for (int i = 0; i < NP; ++i)
          v[j][i] = *reinterpret_cast<const uint4*>(po + static_cast<int64_t>(s0 + j) * sstride + (i >> 1) * gstride +
                                                    8 * (i & 1));
      }
    }
#pragma unroll
    for (int c0 = 0; c0 < PRE; c0 += kCombineRegSplits) {
      if (s0 + c0 < nsplit) {
        float M_new = M;
#pragma unroll
        for (int j = c0; j < c0 + kCombineRegSplits; ++j)
          if (s0 + j < nsplit && ms[j].y > 0.0f) M_new = fmaxf(M_new, ms[j].x);
        if (M_new != M) {  // rescale what is merged so far (nothing yet when M = -inf)
          const float a = M == -__builtin_huge_valf() ? 0.0f : exp2f(M - M_new);
          L = L * a;
#pragma unroll
          for (int i = 0; i < 8 * NP; ++i) acc[i] = acc[i] * a;
          M = M_new;
        }
#pragma unroll
        for (int j = c0; j < c0 + kCombineRegSplits; ++j) {
          if (s0 + j < nsplit) {
            const float wgt = ms[j].y > 0.0f ? ms[j].y * exp2f(ms[j].x - M) : 0.0f;
            L = L + wgt;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
              const uint32_t w[4] = {v[j][i].x, v[j][i].y, v[j][i].z, v[j][i].w};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                acc[8 * i + 2 * e] = acc[8 * i + 2 * e] + bf16_to_f32(static_cast<uint16_t>(w[e] & 0xffffu)) * wgt;
                acc[8 * i + 2 * e + 1] = acc[8 * i + 2 * e + 1] + bf16_to_f32(static_cast<uint16_t>(w[e] >> 16)) * wgt;
              }
            }
          }
        }
      }
    }
  }
}

// The merged pieces in bf16 at dst (NP x 8 contiguous channels), with the inverse RoPE of the
// output (owlet1/attention.py:226) when `rot`: rc / rs [i] hold the cos / sin of piece i's
// four pairs.
template <int NP>
__device__ __forceinline__ void store_merged(uint16_t* dst, const float (&acc)[8 * NP], float L, bool rot,
                                             const uint2 (&rc)[NP], const uint2 (&rs)[NP]) {
  const float inv = 1.0f / L;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    uint32_t o[4] = {pack_bf16x2(acc[8 * i] * inv, acc[8 * i + 1] * inv),
                     pack_bf16x2(acc[8 * i + 2] * inv, acc[8 * i + 3] * inv),
                     pack_bf16x2(acc[8 * i + 4] * inv, acc[8 * i + 5] * inv),
                     pack_bf16x2(acc[8 * i + 6] * inv, acc[8 * i + 7] * inv)};
    if (rot) {
      const uint32_t cw_[2] = {rc[i].x, rc[i].y}, sw_[2] = {rs[i].x, rs[i].y};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t cp = cw_[k >> 1], sp = sw_[k >> 1];
        o[k] = rope_pair_bf16(o[k], bf16_to_f32(static_cast<uint16_t>((k & 1) ? cp >> 16 : cp & 0xffffu)),
                              -bf16_to_f32(static_cast<uint16_t>((k & 1) ? sp >> 16 : sp & 0xffffu)));
      }
    }
    *reinterpret_cast<uint4*>(dst + 8 * i) = uint4{o[0], o[1], o[2], o[3]};
  }
}

// ---- the split merge inside the attention launch ----------------------------------------
// XCC (accelerator die) the calling wave runs on: HW_REG_XCC_ID, bits 3:0.
__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg(20 | (3 << 11)) & 15u; }

constexpr int kMergeSpinLimit = 1 << 20;  // polls of the arrival counter before a workgroup gives up

// Workgroup `split` of a (row, 64-head group) merges heads h0 + split * hs .. + hs - 1
// (hs = 64 / nsplit) with merge_pieces, so its output and lse are bit-identical to the merge
// launch's.  An item is NP pieces (NP / 2 whole 16-channel groups, or one half group at NP
// = 1) of one head; consecutive threads take consecutive heads of the same channels, so they
// read contiguous runs of the partials' [D/16][H][16] layout.
template <int D, int NOPE, int NT, int NP>
__device__ __forceinline__ void merge_slice(const AttnParams& p, int64_t row, int h0, int split, int tid) {
  static_assert(D % (8 * NP) == 0 && NOPE % (8 * NP) == 0, "an item lies wholly inside or outside the rope slice");
  const int hs = 64 / p.nsplit;
  const int hlo = h0 + split * hs;
  constexpr int CPH = D / (8 * NP);  // items per head
  const int items = hs * CPH;
  const float* mlrow = p.part_ml + row * p.split_stride * p.H * 2;
  const uint16_t* porow = p.part_o + row * p.split_stride * p.H * static_cast<int64_t>(D);
  for (int it = tid; it < items; it += NT) {
    int head, ch0;
    if constexpr (NP == 1) {  // (16-channel group, head, half)
      const int g = it / (2 * hs), j = it - g * 2 * hs;
      head = hlo + (j >> 1);
      ch0 = 16 * g + 8 * (j & 1);
    } else {                  // (item chunk, head)
      const int c = it / hs;
      head = hlo + (it - c * hs);
      ch0 = 8 * NP * c;
    }
    if (head >= p.H) continue;
    const uint16_t* po = porow + (ch0 >> 4) * (p.H * 16) + head * 16 + (ch0 & 15);
    const float sk = p.sinks ? p.sinks[head] * kLog2e : -__builtin_huge_valf();
    float acc[8 * NP];
    float M, L;
    merge_pieces<NP, NP == 1 ? 2 * kCombineRegSplits : kCombineRegSplits>(po, static_cast<int64_t>(p.H) * D, static_cast<int64_t>(p.H) * 16,
                                            mlrow + head * 2, p.nsplit, p.H, sk, p.sinks != nullptr, acc, M, L);
    uint2 rc[NP], rs[NP];
    const bool rot = NOPE < D && p.rope_cos != nullptr && ch0 >= NOPE;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      rc[i] = rs[i] = uint2{0u, 0u};
      if (rot) {
        const int64_t ci = row * ((D - NOPE) / 2) + (ch0 - NOPE) / 2 + 4 * i;
        rc[i] = *reinterpret_cast<const uint2*>(p.rope_cos + ci);
        rs[i] = *reinterpret_cast<const uint2*>(p.rope_sin + ci);
      }
    }
    store_merged<NP>(p.out + (row * p.H + head) * static_cast<int64_t>(D) + ch0, acc, L, rot, rc, rs);
    if (ch0 == 0) p.lse[((row / p.S) * p.H + head) * p.S + row % p.S] = (M + __log2f(L)) * kLn2;
  }
}

// The in-launch merge of a (row, 64-head group) whose nsplit workgroups all run at once (the
// host allows it only when the whole grid fits the device, one workgroup per CU).  Each
// workgroup's partial stores reach its XCD's L2 (the vector L1 writes through) before it
// arrives; it then waits until all nsplit have arrived and merges its slice of the heads
// (merge_slice).  With the row-per-XCD mapping every workgroup of the group runs on one XCD,
// so the partials are read from the L2 they were written to; a workgroup that cannot see
// its whole group registered on its own XCC releases its partials to memory (agent-scope
// release: an L2 write-back) before arriving, and one whose group turned out spread
// acquires (an L2 invalidate) before reading -- a group is either wholly on one XCC, where
// every member saw it so or released, or spread, where every member released.  The wait is
// bounded: after kMergeSpinLimit polls a workgroup gives up, sets merge_err and writes
// nothing.  The last workgroup to leave clears the record for the next launch.
template <int D, int NOPE, int NT>
__device__ __forceinline__ void merge_in_launch(const AttnParams& p, int64_t row, int h0, int split, uint32_t* mrec,
                                                int tid) {
  __shared__ int m_go;
  const uint32_t ns = static_cast<uint32_t>(p.nsplit);
  uint64_t* reg = reinterpret_cast<uint64_t*>(mrec);
  // the registration is read while the partial stores drain (one wait covers both)
  uint64_t r = 0;
  if (tid == 0) r = __hip_atomic_load(reg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // this wave's partial stores are done
  __syncthreads();
  if (tid == 0) {
    const uint32_t me = xcc_id();
    // every member registered on this XCC: the group is wholly here (registrations only grow)
    const bool local = !p.merge_fence && ((r >> (8 * me)) & 0xffu) == ns;
    if (!local) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // the write-back done before the arrival
    }
    // the last to arrive knows it from the count it replaces; the others poll
    uint32_t a = __hip_atomic_fetch_add(mrec + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    for (int it = 0; a < ns && it < kMergeSpinLimit; ++it) {
      __builtin_amdgcn_s_sleep(1);
      a = __hip_atomic_load(mrec + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int go = a >= ns;
    if (!local) __hip_atomic_fetch_add(p.merge_err + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // diagnostic
    if (go && !local) {
      // every member has arrived, so every one has registered: the group's final placement
      const uint64_t rf = __hip_atomic_load(reg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (p.merge_fence || ((rf >> (8 * me)) & 0xffu) != ns) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    if (!go) __hip_atomic_fetch_or(p.merge_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    m_go = go;
  }
  __syncthreads();
  if (m_go) {
    // an item = 8 * NP channels of a head; NP chosen so that the slice's items fit one pass
    // of NT threads where it can (nsplit 4, 8, 16: 288 items)
    switch (p.nsplit) {
      case 2:
      case 4: merge_slice<D, NOPE, NT, 4>(p, row, h0, split, tid); break;
      case 8: merge_slice<D, NOPE, NT, 2>(p, row, h0, split, tid); break;
      default: merge_slice<D, NOPE, NT, 1>(p, row, h0, split, tid); break;
    }
  }
  // this workgroup reads the record no more: the last to leave clears it and counts the
  // group's merge in merge_err[1] (a diagnostic: merged groups since the workspace was zeroed)
  if (tid == 0 && __hip_atomic_fetch_add(mrec + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ns - 1) {
    __hip_atomic_store(mrec + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(mrec + 3, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reg, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(p.merge_err + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------------------------------
// D <= 256: one wave per 32 heads over the whole of D.  HG waves per workgroup.
// Per tile: dequantize into Kt, S^T = K.Q^T (two MFMA chains), lane-local online
// softmax, O^T += V^T.P^T with P^T straight from the S^T registers.
// ------------------------------------------------------------------------------------
template <int FMT, int D, int NOPE, int HG>
__global__ void __launch_bounds__(HG * 64) sparse_mqa_kernel(const AttnParams p) {
  constexpr int NT = HG * 64;
  constexpr int KS = D / 16;
  constexpr int NB = D / 32;
  constexpr int KT_PITCH = 2 * D + 16;  // bytes per Kt row (16 B pad spreads LDS banks)
  using RP = RowPlan<FMT, D, NOPE, NT>;
  static_assert(D % 32 == 0, "D must be a multiple of 32");

  __shared__ __align__(16) uint8_t kt[kTile * KT_PITCH];
  __shared__ const uint8_t* tab_ptr[2 * kTile];
  __shared__ uint32_t tab_mask[2];
  __shared__ int32_t sidx[kIdxCap];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int hg = tid >> 6;
  const int half = lane >> 5;
  RP rp;
  rp.tab_ptr = tab_ptr;
  rp.tab_mask = tab_mask;
  rp.init(p, HG * 32);
  rp.stage_indices(p, sidx, kIdxCap, tid);
  __syncthreads();

  const int head = rp.hgrp * (HG * 32) + hg * 32 + (lane & 31);
  const bool head_ok = head < p.H;
  v8bf qf[KS];
  {
    const uint16_t* qrow = p.q + (rp.row * p.H + (head_ok ? head : 0)) * D + half * 8;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      uint4 v = head_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * st) : uint4{0, 0, 0, 0};
      qf[st] = __builtin_bit_cast(v8bf, v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w});
    }
  }
  v16f acc_o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc_o[i] = v16f{};
  float m_run = -__builtin_huge_valf();
  float l_run = 0.0f;

  Piece raw[RP::PPT];
  int g_pref = -1;
  if (rp.ntiles > 0) {
    rp.build_table(p, 0, tid < kTile ? rp.slot(rp.v_begin + tid) : -1, tid);
    rp.build_table(p, 1, tid < kTile ? rp.slot(rp.v_begin + kTile + tid) : -1, tid);
    if (tid < kTile) g_pref = rp.slot(rp.v_begin + 2 * kTile + tid);
    __syncthreads();
    rp.fetch(0, tid, raw);
  }

#pragma unroll 1
  for (int t = 0; t < rp.ntiles; ++t) {
    const uint32_t vmask = tab_mask[t & 1];
    rp.store(kt, KT_PITCH, tid, raw);
    lds_barrier();  // Kt complete; every wave has read tile t's table
    rp.build_table(p, t + 2, g_pref, tid);
    if (tid < kTile) g_pref = rp.slot(rp.v_begin + (t + 3) * kTile + tid);
    if (t + 1 < rp.ntiles) rp.fetch(t + 1, tid, raw);  // in flight across the LDS-only barriers

    v16f s = v16f{}, s1 = v16f{};  // even / odd K-steps, summed in that order
    {
      const uint8_t* krow = kt + (lane & 31) * KT_PITCH + 2 * (half * 8);
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const uint4 kv = *reinterpret_cast<const uint4*>(krow + 32 * st);
        const v8bf ka = __builtin_bit_cast(v8bf, v4i{(int)kv.x, (int)kv.y, (int)kv.z, (int)kv.w});
        if (st & 1) s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[st], s1, 0, 0, 0);
        else s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[st], s, 0, 0, 0);
      }
      s = s + s1;
    }
    // online softmax (exp2 domain), lane-local per head over its 16 entries plus the other
    // half's 16.  The running max is raised only when a head's tile max exceeds it by more
    // than kLazy; the decision is wave-uniform, so most tiles skip the O^T *= alpha pass.
    float tmax = -__builtin_huge_valf();
    if (vmask == 0xffffffffu) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[j] = s[j] * p.scale_log2;
        tmax = fmaxf(tmax, s[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[j] = ((vmask >> c_entry(j, lane)) & 1u) ? s[j] * p.scale_log2 : -__builtin_huge_valf();
        tmax = fmaxf(tmax, s[j]);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const bool raise = tmax > m_run + kLazy;
    if (__any(raise)) {
      const float m_new = raise ? tmax : m_run;
      const float alpha = (m_run == -__builtin_huge_valf()) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run = l_run * alpha;
#pragma unroll
      for (int i = 0; i < NB; ++i) acc_o[i] = acc_o[i] * alpha;
      m_run = m_new;
    }
    // masked entries are -inf and v_exp_f32(-inf) = 0; before any finite entry the
    // reference point is 0 instead of -inf (which would give NaN)
    const float m_use = m_run == -__builtin_huge_valf() ? 0.0f : m_run;
    float psum = 0.0f;
    uint32_t pk[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // v_exp_f32 directly: arguments are <= kLazy, results below 2^-126 may flush to 0
      const float p0 = __builtin_amdgcn_exp2f(s[2 * i] - m_use);
      const float p1 = __builtin_amdgcn_exp2f(s[2 * i + 1] - m_use);
      psum = psum + p0 + p1;
      pk[i] = pack_bf16x2(p0, p1);
    }
    psum = psum + __shfl_xor(psum, 32, 64);
    l_run = l_run + psum;
    const v8bf pf0 = __builtin_bit_cast(v8bf, v4i{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]});
    const v8bf pf1 = __builtin_bit_cast(v8bf, v4i{(int)pk[4], (int)pk[5], (int)pk[6], (int)pk[7]});
    const uint8_t* tr0 = kt + pv_lane_offset<KT_PITCH>(lane, 0);
#pragma unroll
    for (int db = 0; db < NB; ++db) pv_block<KT_PITCH>(tr0 + 64 * db, pf0, pf1, acc_o[db]);
    lds_barrier();  // Kt is free for the next tile
  }

  if (!head_ok) return;
  write_result<D, NOPE, NB>(p, rp.row, rp.b, rp.split, head, half, half == 0, 0, NB, m_run, l_run, acc_o);
}

// ------------------------------------------------------------------------------------
// D > 256 (the 512+64 latent): 64 heads per workgroup, each 32-head group split over 4
// waves by D (8 waves, two per SIMD: one of each group).  A wave holds its D-quarter of q
// (9 K-steps) and at most 5 O^T blocks; the four partial S^T of a head group are summed
// through LDS.  The two groups run half a tile apart (ping-pong), so on every SIMD one
// wave does MFMA work (PV of one tile interleaved with QK of the next, operands read a
// block ahead) while the other does the softmax, its half of the next tile's
// dequantization into LDS, and the tile fetches; the schedule is spelled out at the
// tile loop.  Softmax: the running max is raised lazily to an upper bound of the tile
// max (the sum of the four partial maxima), so exp2(s - m) <= 2^kLazy always holds; the
// online softmax is exact for any reference point as long as no significant term
// underflows, which the pass checks at its end (else an exact pass redoes the split).
// One barrier per half-tile (one more per half-tile in the exact pass, which exchanges
// the true tile max).
// ------------------------------------------------------------------------------------
template <int FMT, int D, int NOPE>
struct SplitSmem {
  static constexpr int HG = 2, DS = 4;
  static constexpr int KT_PITCH = 2 * D + 16;
  static constexpr int KT = kTile * KT_PITCH;             // one bf16 tile
  static constexpr int SX = HG * DS * 4 * 64 * 16;        // [wave][4][64] float4 partial S^T
  static constexpr int PM = HG * 32 * 2 * DS * 4;         // [2][64 heads] float4: partial maxima / row sums
  static constexpr int PB = HG * 2 * 64 * 16;             // [hg][2 K-steps][64] P^T
  static constexpr int PE = HG * 32 * 2 * DS * 4;         // [2][64 heads] float4: true lane maxima
  static constexpr int NKT = 3;                            // bf16 tiles in flight: PV, QK, dequantized
  static constexpr int LDS = NKT * KT + SX + PM + PB + PE;
};

// ALLTAB: the host has checked that every split of the launch keeps all its entry tables
// (its longest possible split does), so the ring of tables and its index reads (which may
// go to global memory, and whose waits would then also drain the tile loads in flight) are
// compiled out.
// SEL (with ALLTAB): the workgroup selects its row's sparse list itself from the indexer
// scores (topk_core.h's row selection, 16 scores per thread: G <= 8192, topk <= 2048, both
// multiples of 4), in the LDS the tiles take later -- every workgroup of the row computes
// the same list, so no workgroup waits for another and the top-k launch goes away.
template <int FMT, int D, int NOPE, bool ALLTAB, bool SEL = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
sparse_mqa_dsplit_kernel(const AttnParams p) {
  using M = SplitSmem<FMT, D, NOPE>;
  constexpr int HG = M::HG, DS = M::DS;
  constexpr int NT = HG * DS * 64;
  constexpr int KT_PITCH = M::KT_PITCH;
  constexpr int QST = D / 16 / DS;            // QK K-steps per wave
  constexpr int NB = D / 32;                  // 32-channel blocks of O
  constexpr int NDBM = (NB + DS - 1) / DS;    // most O blocks one wave owns
  // entry tables in flight: t (its mask), t+1 .. t+3 (fetched), t+4 (built this tile)
  constexpr int NSLOT = 8;
  using RP = RowPlan<FMT, D, NOPE, NT, NSLOT>;
  static_assert((D / 16) % DS == 0 && D % 32 == 0, "D must split into 4 parts of 16-channel steps");

  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* kt0 = smem;                                                   // 3 x [32][KT_PITCH]
  float4* sx = reinterpret_cast<float4*>(smem + M::NKT * M::KT);
  float* pm = reinterpret_cast<float*>(smem + M::NKT * M::KT + M::SX);
  uint4* pb = reinterpret_cast<uint4*>(smem + M::NKT * M::KT + M::SX + M::PM);
  float* pe = reinterpret_cast<float*>(smem + M::NKT * M::KT + M::SX + M::PM + M::PB);
  // one LDS region for the entry tables: the staged sparse indices (first 4 KB) and a ring
  // of NSLOT tables after them, or -- when the split has at most kAllTabCap entries --
  // every table of the split over the whole region (built once, before the passes)
  static_assert(kSplitIdxCap * 4 + NSLOT * kTile * 8 <= kAllTabCap * 8, "ring and indices share the region");
  __shared__ __align__(16) const uint8_t* tabs[kAllTabCap];
  __shared__ uint32_t tab_mask[kAllTabCap / kTile];
  int32_t* sidx = reinterpret_cast<int32_t*>(tabs);
  const uint8_t** tab_ptr = tabs + kSplitIdxCap / 2;
  __shared__ int redo;  // set when the fast pass's running max drifted too far above the truth

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) branches on the group
  const int hg = wave / DS;
  if (tid == 0) redo = 0;  // published by the barrier after the indices are staged
  const int ds = wave % DS;
  const int half = lane >> 5;
  RP rp;
  rp.tab_ptr = tab_ptr;
  rp.tab_mask = tab_mask;
  rp.template locate<ALLTAB>(p, HG * 32);
  // The row's index list (SEL: its scores), its position and this lane's query fragment are
  // requested together: one memory round trip at the start instead of three dependent ones.
  v4i pre;
  bool pre_ok;
  constexpr int SKPT = 16;  // SEL: scores per thread
  static_assert(!SEL || (ALLTAB && SKPT * NT == 8192), "the selecting instance: decode, 8192 scores per row");
  float4 sc4[SEL ? SKPT / 4 : 1];
  if constexpr (SEL) {
    // branch-free: G is a multiple of 4, so a thread's last aligned float4 at or past the
    // row's end is re-read from G - 4 (and its keys are padding below)
    const float* srow = p.sel_scores + rp.row * p.sel_stride;
    const int G4 = static_cast<int>(p.G) - 4;
#pragma unroll
    for (int m = 0; m < SKPT / 4; ++m) {
      const int o = SKPT * tid + 4 * m;
      sc4[m] = *reinterpret_cast<const float4*>(srow + (o <= G4 ? o : G4));
    }
    pre_ok = true;
  } else {
    pre_ok = rp.prefetch_indices(p, tid, pre);
  }
  const int64_t row_pos = p.positions[rp.row];

  const int hl = hg * 32 + (lane & 31);  // head within the workgroup
  const int head = rp.hgrp * (HG * 32) + hl;
  const bool head_ok = head < p.H;
  const int qc0 = ds * QST * 16;  // first QK channel of this wave
  // this lane's slot k = 2 ds + half of its head's eight partial maxima / row sums, in a
  // [2][64 heads] float4 layout: a head's eight values are two conflict-free float4 reads,
  // and a wave's 64 b32 writes fall on 32 distinct banks (2-way; [64 heads][8] was 8-way)
  const int pm_slot = (((2 * ds + half) >> 2) * 64 + hl) * 4 + ((2 * ds + half) & 3);
  v8bf qf[QST];
  {
    // branch-free loads (a missing head reads head 0 and is zeroed); uniform row base plus a
    // 32-bit lane offset (H <= 128) keeps no 64-bit per-lane address alive
    const uint16_t* qbase = p.q + rp.row * p.H * D;
    const uint32_t qoff = static_cast<uint32_t>((head_ok ? head : 0) * D + qc0 + half * 8);
#pragma unroll
    for (int st = 0; st < QST; ++st) {
      v4i v = *reinterpret_cast<const v4i*>(qbase + qoff + 16 * st);
      if (!head_ok) v = v4i{0, 0, 0, 0};
      qf[st] = __builtin_bit_cast(v8bf, v);
    }
  }
  // RoPE of q: the rope slice is the last RST K-steps of the last D-quarter; every lane
  // reads the cos / sin of the 4 pairs those steps give it (of the row's first pairs when
  // no table is given), and the last D-quarter rotates them before its first QK
  constexpr int RST = (D - NOPE) / 16;
  static_assert(RST == 0 || ((D - NOPE) % 16 == 0 && D - NOPE <= D / DS), "rope slice inside the last D-quarter");
  uint2 qrc[RST > 0 ? RST : 1], qrs[RST > 0 ? RST : 1];
  const bool q_rope = RST > 0 && p.rope_cos != nullptr && ds == DS - 1;
  if constexpr (RST > 0) {
    const uint16_t* cb = p.rope_cos ? p.rope_cos : p.q;
    const uint16_t* sb = p.rope_cos ? p.rope_sin : p.q;
    const uint32_t roff = static_cast<uint32_t>(rp.row * ((D - NOPE) / 2)) + 4 * half;
#pragma unroll
    for (int r = 0; r < RST; ++r) {
      qrc[r] = *reinterpret_cast<const uint2*>(cb + roff + 8 * r);
      qrs[r] = *reinterpret_cast<const uint2*>(sb + roff + 8 * r);
    }
  }
  // in-launch merge: the workgroup registers the XCC it runs on with its (row, 64-head
  // group), after its first loads (an atomic without return: no wait covers it)
  uint32_t* mrec = nullptr;
  if constexpr (ALLTAB) {
    if (p.merge_rec != nullptr) {
      const uint32_t nhg = static_cast<uint32_t>((p.H + HG * 32 - 1) / (HG * 32));
      mrec = p.merge_rec + 4 * (static_cast<uint32_t>(rp.row) * nhg + static_cast<uint32_t>(rp.hgrp));
      if (tid == 0)
        __hip_atomic_fetch_add(reinterpret_cast<uint64_t*>(mrec), 1ull << (8 * xcc_id()), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __shared__ int wred[2 * 8];
  if constexpr (SEL) {
    rp.plan_row(p, row_pos);
    // the row's selection in the tile region of LDS (first written by the tile loop, after
    // the barriers below): three histograms and the scan scratch
    int* const h1 = reinterpret_cast<int*>(smem);
    int* const h2 = h1 + kBins * kSub1;
    int* const h3 = h2 + kBins;
    int* const sw = h3 + kBins / 2;
    static_assert((kBins * kSub1 + kBins + kBins / 2 + 16) * 4 <= M::NKT * M::KT, "selection LDS");
    const RowSelLds lds{h1, h2, h3, sw, sw + 8, sw + 12};
    const int G = static_cast<int>(p.G), k = p.topk;
    const bool search = G > k;
    if (search) {
      row_sel_clear<NT>(lds, tid);
      __syncthreads();
    }
    const int i0 = SKPT * tid;
    uint32_t key[SKPT];
#pragma unroll
    for (int m = 0; m < SKPT / 4; ++m) {
      const float v[4] = {sc4[m].x, sc4[m].y, sc4[m].z, sc4[m].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) key[4 * m + c] = order_key(v[c]) & key_mask(i0 + 4 * m + c, G);
    }

    uint32_t T;
    int need_eq;
    row_sel_threshold<SKPT, NT>(key, search, k, lds, T, need_eq);
    const RowTake tk = row_sel_take<SKPT, NT>(key, T, need_eq, sw);
    // the list is in the top-k launch's form (ascending picks, then -1) by construction, so
    // the split is planned over its `written` valid entries directly, and every thread puts
    // its picks of this split's slice straight into the staged indices (a slice holds at most
    // kAllTabCap - 96 < kSplitIdxCap entries); the row's first workgroup also writes the list
    rp.plan_split(p, tk.written);
    const int sp_end = rp.v_end > rp.nwd ? rp.v_end - rp.nwd : 0;
    const bool first = p.sel_out != nullptr && rp.split == 0 && rp.hgrp == 0;
    int32_t* const orow = first ? p.sel_out + rp.row * p.sel_out_stride : nullptr;
    // a thread's picks take list positions pos .. pos + popcount - 1, ascending with the
    // thread, so only the threads around this split's slice (and in the row's first
    // workgroup, every thread) walk them
    uint32_t sel = tk.sel;
    if (first || (tk.pos < sp_end && tk.pos + __builtin_popcount(sel) > rp.sp_begin)) {
      for (int at = tk.pos; sel != 0u; ++at) {
        const int g = i0 + __builtin_ctz(sel);
        if (at >= rp.sp_begin && at < sp_end) sidx[at - rp.sp_begin] = g;
        if (first && at < k) orow[at] = g;
        sel &= sel - 1u;
      }
    }
    if (first)
      for (int i = tk.written + tid; i < k; i += NT) orow[i] = -1;
    rp.sidx = (const __attribute__((address_space(3))) int32_t*)(sidx);
    rp.sidx_cap = kSplitIdxCap;
    rp.idx_row = nullptr;  // never read: the slice fits the staged indices
  } else {
    rp.plan(p, row_pos, pre_ok ? rp.valid_prefix(p, tid, pre, wred) : -1);
    if (pre_ok) rp.stage_prefetched(sidx, kSplitIdxCap, tid, pre);
    else rp.stage_indices(p, sidx, kSplitIdxCap, tid);
  }
  __syncthreads();
  // Splits of at most kAllTabCap entries (every decode configuration) get all their entry
  // tables here, so the tile loop builds none (a table build costs the building wave an
  // LDS round trip and the pointer arithmetic on the critical half-step); longer splits
  // (long prefill rows) build them in a ring as the loop goes.
  const bool tables_fit = rp.table_tiles() * kTile <= kAllTabCap;
  const bool all_tables = ALLTAB || tables_fit;
  if (ALLTAB && !tables_fit) rp.ntiles = 0;  // excluded by the host's check: never read past the tables
  if (all_tables) rp.template build_all_tables<kAllTabCap>(p, tid, tabs, tab_mask);
  const int b_lo = ds * NB / DS;
  const int nb_mine = (ds + 1) * NB / DS - b_lo;
  const int pv_off = pv_lane_offset<KT_PITCH>(lane, b_lo * 32);
  // S^T partial over this wave's D-quarter of the tile in `kt`; K fragments are read
  // three K-steps ahead of their MFMA (a rolling window keeps register pressure low)
  auto qk = [&](const uint8_t* kt) __attribute__((always_inline)) -> v16f {
    constexpr int AH = 3;
    const uint8_t* krow = kt + (lane & 31) * KT_PITCH + 2 * (qc0 + half * 8);
    uint4 kv[AH];
#pragma unroll
    for (int i = 0; i < AH; ++i) kv[i] = *reinterpret_cast<const uint4*>(krow + 32 * i);
    v16f s = v16f{};
#pragma unroll
    for (int st = 0; st < QST; ++st) {
      const uint4 cur = kv[st % AH];
      if (st + AH < QST) kv[st % AH] = *reinterpret_cast<const uint4*>(krow + 32 * (st + AH));
      const v8bf kf = __builtin_bit_cast(v8bf, v4i{(int)cur.x, (int)cur.y, (int)cur.z, (int)cur.w});
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s, 0, 0, 0);
    }
    return s;
  };
  // the partial ([wave][j/4][lane] float4: consecutive lanes at consecutive 16 B,
  // conflict-free) and its per-head maximum over this lane's 16 entries go to LDS
  auto publish = [&](const v16f& s) __attribute__((always_inline)) {
    float mx = s[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) mx = fmaxf(mx, s[j]);
    pm[pm_slot] = mx;
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4)
      sx[(wave * 4 + j4) * 64 + lane] = float4{s[4 * j4], s[4 * j4 + 1], s[4 * j4 + 2], s[4 * j4 + 3]};
  };

  // One pass over the split.  The fast pass raises the running max to the partial-maxima
  // bound, which may exceed the true maximum; it tracks each head's true maximum on the
  // side and gives up (returns false, writes nothing) if the final running max lies more
  // than kBoundSlack above it.  Below that every entry that v_exp_f32 flushes to zero
  // (argument < -126) weighs less than 2^-62 of the largest entry, so the result is exact
  // to fp32 resolution.  The exact pass (only run after a fast pass gave up) exchanges
  // the true tile max through LDS with one more barrier per tile.
  constexpr float kBoundSlack = 64.0f;
  auto pass = [&](auto exact_tag) -> bool {
    constexpr bool kExact = decltype(exact_tag)::value;
    v16f acc_o[NDBM];
#pragma unroll
    for (int i = 0; i < NDBM; ++i) acc_o[i] = v16f{};
    float m_run = -__builtin_huge_valf();  // identical in the 8 lanes x waves of a head
    float l_run = 0.0f;                    // this lane's share of the head's row sum
    float m_seen = -__builtin_huge_valf(); // true max of this lane's (unmasked) entries

    // Ping-pong schedule.  The two head groups run half a tile apart, so on every SIMD
    // (which holds one wave of each group) one wave does MFMA work while the other does
    // the softmax and the tile traffic.  Half-step 2u (even) and 2u+1 (odd), each opened by
    // a workgroup barrier:
    //   even(u): group 0 softmax(u) -> P^T(u); stores its half (entries 16..31) of tile u+1,
    //            fetches its half of tile u+3, builds the entry table of tile u+4;
    //            group 1 PV(u-1) + QK(u) -> publishes S^T(u).
    //   odd(u):  group 0 PV(u) + QK(u+1) -> publishes S^T(u+1);
    //            group 1 softmax(u) -> P^T(u); stores its half (entries 0..15) of tile
    //            u+2, fetches its half of tile u+4.
    // Tile u lives in LDS tile u%3: it is read by QK at half-steps 2u-1 and 2u and by PV
    // at 2u+1 and 2u+2, and its halves are written at 2u-3 (group 1) and 2u-2 (group 0),
    // when the tile that used the buffer before (u-3) is no longer read.  A group's raw
    // register set holds its half of two tiles in flight (even tiles in one set, odd in
    // the other), so a load has two tiles' time to arrive.  Group g dequantizes / fetches
    // as thread tid ^ 256, which maps group 0 to entries 16..31 and group 1 to 0..15.
    Piece raw[RP::PPT];
    int g_pref = -1;
    const int ptid = tid ^ 256;
    auto ktile = [&](int u) __attribute__((always_inline)) -> uint8_t* { return kt0 + (u % 3) * M::KT; };

    // softmax of tile u for this wave's heads: S^T partials -> running max / sum -> P^T
    // The softmax runs at a raised wave priority: on its SIMD the other group's wave is in
    // its MFMA half-step, whose issue slots the softmax's dependent LDS reads and exps then
    // win (the MFMA chain waits on its own operand reads most of the time).  Measured: 72.4
    // -> 71.6 us per config-2 step; the priority over the whole traffic half-step (stores
    // and gathers too), or on the MFMA half-step instead, was no better or slower.
    auto softmax = [&](int u) __attribute__((always_inline)) {
      __builtin_amdgcn_s_setprio(1);
      const uint32_t vmask = tab_mask[u & rp.slot_mask];
      // entries 8ds..8ds+7 of tile u for this lane's head
      float4 a = sx[((hg * DS) * 4 + ds) * 64 + lane];
#pragma unroll
      for (int part = 1; part < DS; ++part) {
        const float4 c = sx[((hg * DS + part) * 4 + ds) * 64 + lane];
        a.x = a.x + c.x;
        a.y = a.y + c.y;
        a.z = a.z + c.z;
        a.w = a.w + c.w;
      }
      float v4[4] = {a.x * p.scale_log2, a.y * p.scale_log2, a.z * p.scale_log2, a.w * p.scale_log2};
      if (vmask != 0xffffffffu) {
        const uint32_t bits = vmask >> (8 * ds + 4 * half);  // entries 8ds + 4half + i
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!((bits >> i) & 1u)) v4[i] = -__builtin_huge_valf();
      }
      const float lane_max = fmaxf(fmaxf(v4[0], v4[1]), fmaxf(v4[2], v4[3]));
      float bound;
      if constexpr (kExact) {
        // the head's true tile max: its 8 lanes' maxima through LDS (the other group
        // passes the matching barrier at the start of its MFMA half-step)
        pe[pm_slot] = lane_max;
        lds_barrier();
        const float4 t0 = reinterpret_cast<const float4*>(pe)[hl];
        const float4 t1 = reinterpret_cast<const float4*>(pe)[64 + hl];
        bound = fmaxf(fmaxf(fmaxf(t0.x, t0.y), fmaxf(t0.z, t0.w)), fmaxf(fmaxf(t1.x, t1.y), fmaxf(t1.z, t1.w)));
      } else {
        m_seen = fmaxf(m_seen, lane_max);
        const float4 t0 = reinterpret_cast<const float4*>(pm)[hl];
        const float4 t1 = reinterpret_cast<const float4*>(pm)[64 + hl];
        bound = (((fmaxf(t0.x, t0.y) + fmaxf(t0.z, t0.w)) + fmaxf(t1.x, t1.y)) + fmaxf(t1.z, t1.w)) * p.scale_log2;
      }
      const bool raise = bound > m_run + kLazy;
      if (__any(raise)) {  // identical in every wave of the head group
        const float m_new = raise ? bound : m_run;
        const float alpha = (m_run == -__builtin_huge_valf()) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run = l_run * alpha;
#pragma unroll
        for (int i = 0; i < NDBM; ++i) acc_o[i] = acc_o[i] * alpha;
        m_run = m_new;
      }
      // the exact pass may see a head with no finite entry yet (m_run = -inf): then every
      // entry is -inf and the reference point 0 gives exp2(-inf) = 0 instead of NaN
      const float m_use = (kExact && m_run == -__builtin_huge_valf()) ? 0.0f : m_run;
      const float p0 = __builtin_amdgcn_exp2f(v4[0] - m_use);
      const float p1 = __builtin_amdgcn_exp2f(v4[1] - m_use);
      const float p2 = __builtin_amdgcn_exp2f(v4[2] - m_use);
      const float p3 = __builtin_amdgcn_exp2f(v4[3] - m_use);
      l_run = l_run + ((p0 + p1) + (p2 + p3));
      // PV K-step ks = ds/2 takes registers 8ks..8ks+7 = D-parts 2ks (slots 0-3), 2ks+1 (4-7)
      uint2* dst = reinterpret_cast<uint2*>(pb + (hg * 2 + (ds >> 1)) * 64 + lane) + (ds & 1);
      *dst = uint2{pack_bf16x2(p0, p1), pack_bf16x2(p2, p3)};
      __builtin_amdgcn_s_setprio(0);
    };
    // O^T += V^T.P^T of tile `u` (if pv) and the S^T partial of tile u+1 (if qk), in one
    // block so the two MFMA streams interleave.  Near the end QK runs on a stale buffer;
    // its partial is published but never read.
    auto mfma_step = [&](int u, bool pv, bool qk_next) __attribute__((always_inline)) {
      if constexpr (kExact) lds_barrier();  // pairs with the exact softmax's barrier
      // Software pipeline for a lone MFMA wave: every operand is read from LDS a step
      // ahead of the MFMA that consumes it (V^T one 32-channel block ahead, K two K-steps
      // ahead), and scheduling fences keep the compiler from collapsing the pipeline.
      const uint8_t* kt_q = ktile(u + 1) + (lane & 31) * KT_PITCH + 2 * (qc0 + half * 8);
      constexpr int NB_MIN = NB / DS;  // O^T blocks every wave owns (the last one may own one more)
      uint4 kv[QST];
      v16f s_acc = v16f{};
      // one QK K-step; K fragments are read two steps ahead (compile-time indices only)
      auto qk_step = [&](int st) __attribute__((always_inline)) {
        if (st + 2 < QST) kv[st + 2] = *reinterpret_cast<const uint4*>(kt_q + 32 * (st + 2));
        s_acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(v8bf, v4i{(int)kv[st].x, (int)kv[st].y, (int)kv[st].z, (int)kv[st].w}), qf[st], s_acc,
            0, 0, 0);
      };
      if (qk_next) {
        kv[0] = *reinterpret_cast<const uint4*>(kt_q);
        if (QST > 1) kv[1] = *reinterpret_cast<const uint4*>(kt_q + 32);
      }
      if (pv) {
        const uint4 w0 = pb[(hg * 2 + 0) * 64 + lane];
        const uint4 w1 = pb[(hg * 2 + 1) * 64 + lane];
        const v8bf pf0 = __builtin_bit_cast(v8bf, v4i{(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w});
        const v8bf pf1 = __builtin_bit_cast(v8bf, v4i{(int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w});
        const uint8_t* tr0 = ktile(u) + pv_off;
        // V^T operands double-buffered by block parity, so block db+1's reads are in flight
        // while block db's MFMAs run
        v4s rv[2][4];
        auto read_v = [&](int db) __attribute__((always_inline)) {
          const uint8_t* tp = tr0 + 64 * db;
          v4s (&r)[4] = rv[db & 1];
          r[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp));
          r[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 8 * KT_PITCH));
          r[2] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 16 * KT_PITCH));
          r[3] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 24 * KT_PITCH));
        };
        // PV of block db; with_qk interleaves K-steps 2db and 2db+1 of QK (compile time)
        auto pv_mfma = [&](int db, bool more, bool with_qk) __attribute__((always_inline)) {
          if (more) read_v(db + 1);
          const v4s (&r)[4] = rv[db & 1];
          const v8bf a0 = __builtin_bit_cast(v8bf, v8s{r[0][0], r[0][1], r[0][2], r[0][3], r[1][0], r[1][1], r[1][2], r[1][3]});
          const v8bf a1 = __builtin_bit_cast(v8bf, v8s{r[2][0], r[2][1], r[2][2], r[2][3], r[3][0], r[3][1], r[3][2], r[3][3]});
          acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, pf0, acc_o[db], 0, 0, 0);
          if (with_qk && qk_next && 2 * db < QST) qk_step(2 * db);
          acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, pf1, acc_o[db], 0, 0, 0);
          if (with_qk && qk_next && 2 * db + 1 < QST) qk_step(2 * db + 1);
          __builtin_amdgcn_sched_barrier(0);
        };
        read_v(0);
#pragma unroll
        for (int db = 0; db < NB_MIN; ++db) pv_mfma(db, db + 1 < NB_MIN || nb_mine > NB_MIN, true);
        static_assert(2 * NB_MIN <= QST, "every interleaved K-step index must exist");
#pragma unroll
        for (int st = 2 * NB_MIN; st < QST; ++st)
          if (qk_next) qk_step(st);
        if (nb_mine > NB_MIN) {  // the wave's extra block: the K-steps above are all issued
#pragma unroll
          for (int db = NB_MIN; db < NDBM; ++db) pv_mfma(db, false, false);
        }
      } else if (qk_next) {
#pragma unroll
        for (int st = 0; st < QST; ++st) qk_step(st);
      }
      if (qk_next) publish(s_acc);
    };
    // group 0: even(u) softmax + traffic, odd(u) PV(u) + QK(u+1)
    auto group0_pair = [&](int u, Piece (&r0)[RP::PPT]) {
      lds_barrier();
      softmax(u);
      rp.store(ktile(u + 1), KT_PITCH, ptid, r0);
      // the index of tile u+5 is read before the fetch is issued: the wait on that read
      // (the compiler's counters are in order) then covers no fetch load
      const int g_next = !all_tables && tid < kTile ? rp.slot(rp.v_begin + (u + 5) * kTile + tid) : -1;
      rp.fetch(u + 2, ptid, r0);
      if (!all_tables) rp.build_table(p, u + 4, g_pref, tid);
      g_pref = g_next;
      lds_barrier();
      mfma_step(u, true, true);
    };
    // group 1: even(u) PV(u-1) + QK(u), odd(u) softmax + traffic
    auto group1_pair = [&](int u, Piece (&r1)[RP::PPT]) {
      lds_barrier();
      mfma_step(u - 1, true, true);
      lds_barrier();
      softmax(u);
      rp.store(ktile(u + 2), KT_PITCH, ptid, r1);
      rp.fetch(u + 3, ptid, r1);
    };
    if (rp.ntiles > 0) {
      if (!all_tables) {
        rp.build_first_tables(p, tid);
        if (tid < kTile) g_pref = rp.slot(rp.v_begin + 4 * kTile + tid);
      }
      __syncthreads();
      rp.fetch(0, ptid, raw);
      if constexpr (!kExact && RST > 0) {
        // q's rope steps are rotated while tile 0's gathers are in flight (q and the tables
        // were requested before them, so the wait covers no gather)
        if (q_rope) {
#pragma unroll
          for (int r = 0; r < RST; ++r) {
            v4i v = __builtin_bit_cast(v4i, qf[QST - RST + r]);
            const uint32_t cw_[2] = {qrc[r].x, qrc[r].y}, sw_[2] = {qrs[r].x, qrs[r].y};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const uint32_t cp = cw_[k >> 1], sp = sw_[k >> 1];
              v[k] = static_cast<int>(rope_pair_bf16(static_cast<uint32_t>(v[k]),
                                                     bf16_to_f32(static_cast<uint16_t>((k & 1) ? cp >> 16 : cp & 0xffffu)),
                                                     bf16_to_f32(static_cast<uint16_t>((k & 1) ? sp >> 16 : sp & 0xffffu))));
            }
            qf[QST - RST + r] = __builtin_bit_cast(v8bf, v);
          }
        }
      }
      rp.store(ktile(0), KT_PITCH, ptid, raw);
      rp.fetch(1, ptid, raw);
      if (hg == 1) {  // group 1 also writes its half of tile 1 and holds tile 2
        rp.store(ktile(1), KT_PITCH, ptid, raw);
        rp.fetch(2, ptid, raw);
      }
      lds_barrier();  // tile 0 and half of tile 1 complete
      if (hg == 0) publish(qk(ktile(0)));
    }
    // group 0 dequantizes tile u+1 from set (u+1)&1, group 1 tile u+2 from set u&1
    // the loops execute the same barriers in the same order (two per tile, three in the
    // exact pass)
    if (hg == 0) {
#pragma unroll 1
      for (int u = 0; u < rp.ntiles; ++u) group0_pair(u, raw);
    } else if (rp.ntiles > 0) {
      // u = 0: no PV yet, QK(0) only
      lds_barrier();
      mfma_step(-1, false, true);
      lds_barrier();
      softmax(0);
      rp.store(ktile(2), KT_PITCH, ptid, raw);
      rp.fetch(3, ptid, raw);
#pragma unroll 1
      for (int u = 1; u < rp.ntiles; ++u) group1_pair(u, raw);
    }
    if (rp.ntiles > 0) {
      lds_barrier();  // even(nt): the last P^T of group 1 complete
      if (hg == 1) mfma_step(rp.ntiles - 1, true, false);
      else if constexpr (kExact) lds_barrier();
    }

    // row sum: each lane holds the share of its entries (all scaled to the same running
    // max); the 8 shares of a head are reduced in a fixed order
    __syncthreads();  // every wave is done reading pm and pe
    pm[pm_slot] = l_run;
    if (!kExact) pe[pm_slot] = m_seen;
    __syncthreads();
    {
      const float4 t0 = reinterpret_cast<const float4*>(pm)[hl];
      const float4 t1 = reinterpret_cast<const float4*>(pm)[64 + hl];
      l_run = (((t0.x + t0.y) + (t0.z + t0.w)) + ((t1.x + t1.y) + (t1.z + t1.w)));
    }
    if constexpr (!kExact) {
      const float4 t0 = reinterpret_cast<const float4*>(pe)[hl];
      const float4 t1 = reinterpret_cast<const float4*>(pe)[64 + hl];
      const float m_true =
          fmaxf(fmaxf(fmaxf(t0.x, t0.y), fmaxf(t0.z, t0.w)), fmaxf(fmaxf(t1.x, t1.y), fmaxf(t1.z, t1.w)));
      // a head with no unmasked entry (m_true = -inf) contributes nothing and is exact
      if (head_ok && m_true > -__builtin_huge_valf() && m_run - m_true > kBoundSlack) redo = 1;
      __syncthreads();
      if (redo) return false;  // uniform: every wave reads the flag after the same barrier
    }
    if (head_ok)
      write_result<D, NOPE, NDBM>(p, rp.row, rp.b, rp.split, head, half, ds == 0 && half == 0, b_lo, nb_mine, m_run, l_run,
                            acc_o);
    return true;
  };

  if (!pass(std::false_type{})) pass(std::true_type{});
  if constexpr (ALLTAB) {
    if (mrec != nullptr) merge_in_launch<D, NOPE, NT>(p, rp.row, rp.hgrp * HG * 32, rp.split, mrec, tid);
  }
}

// positions[i] += 1 for the rows of a call whose last launch does not merge splits.
__global__ void __launch_bounds__(256) advance_kernel(int64_t* __restrict__ positions, int64_t rows) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < rows) positions[i] += 1;
}

// The merge launch: the split partials merged with the sink (merge_pieces).  One thread per
// 8 * NP channels of a (row, head), NP 16-byte pieces of every split in flight per memory
// round trip.  A wave takes 16 heads x 4 runs of 8 * NP channels (lane % 16 the head, lane /
// 16 the run): it reads 16 heads x 16 NP bytes contiguous per run from the partials'
// 16-channel groups and writes 4 x 16 NP contiguous bytes of each head's output row.
template <int D, int NP>
__global__ void __launch_bounds__(256) combine_kernel(const uint16_t* __restrict__ part_o,
                                                      const float* __restrict__ part_ml, int nsplit, int H, int64_t S,
                                                      int64_t rows, const float* __restrict__ sinks,
                                                      uint16_t* __restrict__ out, float* __restrict__ lse,
                                                      const uint16_t* __restrict__ rope_cos,
                                                      const uint16_t* __restrict__ rope_sin, int rope_dim,
                                                      int64_t* __restrict__ advance) {
  static_assert(D % 16 == 0 && (NP == 1 || NP == 2), "16-channel groups, one or two pieces per thread");
  // a decode step's position advance: this launch reads no position and the attention launch
  // before it has read them all; thread i of the grid (at least `rows` threads) owns row i
  if (advance != nullptr) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < rows) advance[i] += 1;
  }
  constexpr int CPW = 4 * 8 * NP;             // channels per wave
  constexpr int NWB = (D + CPW - 1) / CPW;    // waves per 16 heads of a row
  const int nhb = (H + 15) / 16;
  // a row's workgroups on XCD row % 8, where the attention launch left its partials
  // (rows a multiple of 8, whole workgroups per row)
  const int64_t wg_per_row = (static_cast<int64_t>(NWB) * nhb + 3) / 4;
  int64_t bid = blockIdx.x;
  if ((rows & 7) == 0 && (static_cast<int64_t>(NWB) * nhb) % 4 == 0) {
    const int64_t k = bid >> 3, x = bid & 7;
    bid = ((k / wg_per_row) * 8 + x) * wg_per_row + k % wg_per_row;
  }
  const int64_t t = bid * 256 + threadIdx.x;
  const int lane = static_cast<int>(t & 63);
  const int64_t wv = t >> 6;
  const int wb = static_cast<int>(wv % NWB);
  const int hb = static_cast<int>((wv / NWB) % nhb);
  const int64_t row = wv / (static_cast<int64_t>(NWB) * nhb);
  const int head = hb * 16 + (lane & 15);
  const int ch0 = wb * CPW + (lane >> 4) * 8 * NP;  // this thread's first channel
  if (row >= rows || head >= H || ch0 >= D) return;
  const int64_t rh = row * H + head;
  const float* ml = part_ml + (row * nsplit * H + head) * 2;  // split s at + 2 s H
  // split s's channel ch0 of this head: group ch0 / 16, heads innermost
  const uint16_t* po = part_o + row * nsplit * H * static_cast<int64_t>(D) + (ch0 >> 4) * (H * 16) + head * 16 + (ch0 & 15);
  const float sk = sinks ? sinks[head] * kLog2e : -__builtin_huge_valf();
  // the inverse RoPE of the merged bf16 output (owlet1/attention.py:226): cos / sin of this
  // thread's pairs when its channels lie in the trailing rope_dim
  const int rope_ch = ch0 - (D - rope_dim);
  const bool rot = rope_cos != nullptr && rope_ch >= 0;
  uint2 rc[NP], rs[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) rc[i] = rs[i] = uint2{0u, 0u};
  if (rot) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      rc[i] = *reinterpret_cast<const uint2*>(rope_cos + row * (rope_dim / 2) + rope_ch / 2 + 4 * i);
      rs[i] = *reinterpret_cast<const uint2*>(rope_sin + row * (rope_dim / 2) + rope_ch / 2 + 4 * i);
    }
  }
  float acc[8 * NP];
  float M, L;
  merge_pieces<NP, kCombineRegSplits>(po, static_cast<int64_t>(H) * D, static_cast<int64_t>(H) * 16, ml, nsplit, H, sk,
                                      sinks != nullptr, acc, M, L);
  store_merged<NP>(out + rh * static_cast<int64_t>(D) + ch0, acc, L, rot, rc, rs);
  if (ch0 == 0) lse[((row / S) * H + head) * S + row % S] = (M + __log2f(L)) * kLn2;
}

template <typename K>
int launch_kernel(K kern, size_t dyn_lds, int threads, int heads_per_wg, const AttnParams& p, int64_t rows, hipStream_t s) {
  const int64_t nhg = (p.H + heads_per_wg - 1) / heads_per_wg;
  const int64_t nblocks = rows * p.nsplit * nhg;
  if (nblocks > 0x7fffffff) {
    set_last_error("sparse_mqa: %lld workgroups exceed the grid limit", (long long)nblocks);
    return MZK_EINVAL;
  }
  kern<<<dim3(static_cast<unsigned>(nblocks)), threads, dyn_lds, s>>>(p);
  return MZK_OK;
}

// Whether the longest split any workgroup of a D-split launch can plan (RowPlan::plan with
// every source full) keeps all its entry tables (RowPlan::table_tiles): the decode kernel
// instances (ALLTAB), which the in-launch merge and the in-launch selection need.
bool dsplit_all_tables(int window, const void* dense, int dense_cap, const void* main_kv, int topk, int nsplit) {
  const int64_t total_max = static_cast<int64_t>(window) + (dense ? dense_cap : 0) + (main_kv ? topk : 0);
  const int64_t chunk_max = ((total_max + nsplit - 1) / nsplit + kTile - 1) / kTile * kTile;
  const int64_t tables_max = chunk_max / kTile + 3 > 4 ? chunk_max / kTile + 3 : 4;
  return tables_max * kTile <= kAllTabCap;
}

// `merged` is set when the launch merges its splits itself (p.merge_rec given and the
// launch takes the kernel instance that carries the merge).
template <int FMT, int D, int NOPE>
int dispatch_heads(const AttnParams& p_in, int64_t rows, hipStream_t s, bool* merged) {
  AttnParams p = p_in;
  *merged = false;
  if (p.H > 128) {
    set_last_error("sparse_mqa: at most 128 heads (got %d)", p.H);
    return MZK_EUNSUPPORTED;
  }
  if constexpr (D > 256) {
    // 64 heads per workgroup, each 32-head group split by D over 4 waves
    using M = SplitSmem<FMT, D, NOPE>;
    static_assert(M::LDS + 8 * kAllTabCap + 4 * (kAllTabCap / kTile) + 128 <= 160 * 1024, "LDS budget");
    auto kern_all = sparse_mqa_dsplit_kernel<FMT, D, NOPE, true>;
    auto kern_ring = sparse_mqa_dsplit_kernel<FMT, D, NOPE, false>;
    auto kern_sel = sparse_mqa_dsplit_kernel<FMT, D, NOPE, true, true>;
    // the dynamic-LDS limit is a per-device function attribute: set once per device
    static std::atomic<bool> attr_set[kMaxDevices] = {};  // setting it twice is harmless
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
      set_last_error("sparse_mqa: no usable current device");
      return MZK_ELAUNCH;
    }
    if (!attr_set[dev].load(std::memory_order_acquire)) {
      for (const void* k : {reinterpret_cast<const void*>(kern_all), reinterpret_cast<const void*>(kern_ring),
                            reinterpret_cast<const void*>(kern_sel)}) {
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, M::LDS) != hipSuccess) {
          set_last_error("sparse_mqa: cannot raise the kernel's LDS limit to %d bytes", M::LDS);
          return MZK_ELAUNCH;
        }
      }
      attr_set[dev].store(true, std::memory_order_release);
    }
    const bool all_tables = dsplit_all_tables(p.window, p.dense, p.dense_cap, p.main, p.topk, p.nsplit);
    if (!all_tables) p.merge_rec = nullptr;  // only the decode instance carries the in-launch merge
    if (p.sel_scores != nullptr) {  // the host checked the selecting instance's limits
      if (!all_tables) {
        set_last_error("sparse_mqa_select: the splits exceed the decode kernel's entry tables");
        return MZK_EUNSUPPORTED;
      }
      *merged = p.merge_rec != nullptr;
      return launch_kernel(kern_sel, M::LDS, 512, 64, p, rows, s);
    }
    *merged = p.merge_rec != nullptr;
    return launch_kernel(all_tables ? kern_all : kern_ring, M::LDS, 512, 64, p, rows, s);
  } else {
    if (p.H <= 32) return launch_kernel(sparse_mqa_kernel<FMT, D, NOPE, 1>, 0, 64, 32, p, rows, s);
    return launch_kernel(sparse_mqa_kernel<FMT, D, NOPE, 2>, 0, 128, 64, p, rows, s);
  }
}

int dispatch(int fmt, int D, int nope, const AttnParams& p, int64_t rows, hipStream_t s, bool* merged) {
  if (fmt == kFmtFp8) {
    if (D == 576 && nope == 512) return dispatch_heads<kFmtFp8, 576, 512>(p, rows, s, merged);
    if (D == 160 && nope == 128) return dispatch_heads<kFmtFp8, 160, 128>(p, rows, s, merged);
    set_last_error("sparse_mqa fp8: unsupported latent %d+%d (have 512+64, 128+32)", nope, D - nope);
    return MZK_EUNSUPPORTED;
  }
  switch (D) {
    case 64: return dispatch_heads<kFmtBf16, 64, 64>(p, rows, s, merged);
    case 96: return dispatch_heads<kFmtBf16, 96, 96>(p, rows, s, merged);
    case 128: return dispatch_heads<kFmtBf16, 128, 128>(p, rows, s, merged);
    case 160: return dispatch_heads<kFmtBf16, 160, 160>(p, rows, s, merged);
    case 256: return dispatch_heads<kFmtBf16, 256, 256>(p, rows, s, merged);
    case 576: return dispatch_heads<kFmtBf16, 576, 576>(p, rows, s, merged);
    default:
      set_last_error("sparse_mqa bf16: unsupported head dim %d (have 64, 96, 128, 160, 256, 576)", D);
      return MZK_EUNSUPPORTED;
  }
}

template <int D>
void launch_combine(const uint16_t* po, const float* pml, int nsplit, int H, int64_t S, const float* sinks,
                    uint16_t* out, float* lse, int64_t rows, const uint16_t* rope_cos, const uint16_t* rope_sin,
                    int rope_dim, int64_t* advance, hipStream_t s) {
  // two 16-byte pieces per thread for a few splits, where a thread's channels cannot straddle
  // the rope slice (config 2, 4 splits: 7.4 vs 7.9 us); with more splits, whose chunk of 8
  // then holds 16 pieces in flight per thread, one is faster (configs 4 / 5, 16 / 32 splits:
  // 7.9 vs 8.4 and 9.2 vs 11.2 us)
  const int64_t nhb = (H + 15) / 16;
  auto threads = [&](int np) { return rows * nhb * ((D + 32 * np - 1) / (32 * np)) * 64; };
  if (nsplit <= 4 && (rope_cos == nullptr || (D - rope_dim) % 16 == 0)) {
    const int64_t n = threads(2);
    combine_kernel<D, 2><<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(po, pml, nsplit, H, S, rows, sinks,
                                                                                out, lse, rope_cos, rope_sin, rope_dim,
                                                                                advance);
  } else {
    const int64_t n = threads(1);
    combine_kernel<D, 1><<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(po, pml, nsplit, H, S, rows, sinks,
                                                                                out, lse, rope_cos, rope_sin, rope_dim,
                                                                                advance);
  }
}

}  // namespace
}  // namespace mzk

using namespace mzk;

namespace {
int combine_impl(const float* workspace, int64_t B, int64_t S, int H, int D, int nsplit, const float* sinks,
                 const void* rope_cos, const void* rope_sin, int rope_dim, void* out, float* lse, int64_t* advance,
                 void* stream);

// Where the split merge runs: 0: the merge launch (the default); 1: inside the attention
// launch where it applies; 2: inside, every workgroup on the release / acquire path (a test
// mode: the path a group spread over several XCDs takes).  The in-launch merge is exact but
// not faster on MI355X: its tail (the arrival, then each split's reads of its siblings'
// partials) costs what the merge launch does at 4 splits, and more at 16 and 32, where the
// splits of a group finish several microseconds apart.
std::atomic<int> g_merge_mode{0};

int64_t align16_bytes(int64_t x) { return (x + 15) & ~static_cast<int64_t>(15); }

// The in-launch merge's records (16 bytes per (row, 64-head group)) and its error word.
int64_t merge_rec_bytes(int64_t rows, int H) { return rows * ((H + 63) / 64) * 16 + 16; }

// Compute units of the current device (cached per device), or 0 if unknown.
int device_cus() {
  static std::atomic<int> cus[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 0) n = 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// split_total < 0: a whole call (partials of nsplit splits then the merge, or the final
// output directly with one split); split_total >= 1: partials only, of splits split_base ..
// split_base + nsplit - 1 of a workspace holding split_total splits per row.
int sparse_mqa_impl(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope, const int64_t* positions,
                    const void* win, int64_t win_batch_entries, int win_cap, int window, const void* dense,
                    int64_t dense_batch_entries, int dense_cap, int dense_ratio, const void* main_kv,
                    int64_t main_batch_entries, int64_t G, const int32_t* idx, int64_t idx_row_stride, int topk,
                    const float* sinks, int nsplit, float* workspace, int64_t workspace_bytes, void* out, float* lse,
                    const void* rope_cos, const void* rope_sin, int rope_dim, int split_base, int split_total,
                    void* stream, int64_t* advance = nullptr, const float* sel_scores = nullptr,
                    int64_t sel_stride = 0, int32_t* sel_out = nullptr, int64_t sel_out_stride = 0) {
  const bool part_only = split_total >= 1;
  MZK_CHECK_ARG(B >= 0 && S >= 0 && H >= 1 && D > 0, "sparse_mqa: bad sizes");
  if (rope_cos || rope_sin) {
    MZK_CHECK_ARG(rope_cos && rope_sin, "sparse_mqa_rope: cos and sin go together");
    MZK_CHECK_ARG(fmt == 1 && D == 576 && nope == 512 && rope_dim == 64,
                  "sparse_mqa_rope: the fused RoPE needs FP8 latent rows of 512 + 64 with rope_dim 64 "
                  "(got fmt %d, D %d, nope %d, rope_dim %d)", fmt, D, nope, rope_dim);
    MZK_CHECK_ARG(aligned16(rope_cos) && aligned16(rope_sin), "sparse_mqa_rope: cos and sin must be 16-byte aligned");
  }
  MZK_CHECK_ARG(fmt == 0 || fmt == 1, "sparse_mqa: fmt must be 0 (bf16) or 1 (fp8-b128)");
  MZK_CHECK_ARG(nsplit >= 1 && nsplit <= 65535, "sparse_mqa: nsplit must be in [1, 65535]");
  if (part_only) {
    MZK_CHECK_ARG(window == 0 || win != nullptr, "sparse_mqa_part: a window of %d entries needs its cache", window);
    MZK_CHECK_ARG(window >= 0, "sparse_mqa_part: negative window");
    MZK_CHECK_ARG(split_base >= 0 && split_base + static_cast<int64_t>(nsplit) <= split_total,
                  "sparse_mqa_part: splits %d .. %d exceed the workspace's %d", split_base, split_base + nsplit - 1,
                  split_total);
    MZK_CHECK_ARG(out == nullptr && lse == nullptr, "sparse_mqa_part: writes partials only");
  } else {
    MZK_CHECK_ARG(window >= 0 && (window == 0 || win != nullptr), "sparse_mqa: a window of %d entries needs its cache",
                  window);
    MZK_CHECK_ARG(window >= 1 || dense != nullptr || main_kv != nullptr,
                  "sparse_mqa: no source (window, dense or sparse) given");
  }
  MZK_CHECK_ARG(win_cap == 0 || win_cap >= window, "sparse_mqa: ring capacity smaller than the window");
  MZK_CHECK_ARG(!dense || (dense_ratio >= 1 && dense_cap >= 0), "sparse_mqa: dense source needs ratio >= 1");
  MZK_CHECK_ARG(!main_kv || ((idx || sel_scores) && topk >= 0 && G >= 0 && idx_row_stride >= topk &&
                              main_batch_entries >= G),
                "sparse_mqa: sparse source needs idx [rows, >= topk] and main_batch_entries >= G");
  const int64_t rows = B * S;
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(q && positions && (part_only || nsplit > 1 || (out && lse)), "sparse_mqa: null pointer");
  MZK_CHECK_ARG((out == nullptr) == (lse == nullptr), "sparse_mqa: out and lse go together");
  MZK_CHECK_ARG(rows <= 0x7fffffff, "sparse_mqa: too many rows");
  {
    const int64_t total_max = static_cast<int64_t>(window) + (dense ? dense_cap : 0) + (main_kv ? topk : 0);
    MZK_CHECK_ARG(total_max < 0x7fffffff, "sparse_mqa: window + dense_cap + topk must stay below 2^31");
    const int64_t chunk = ((total_max + nsplit - 1) / nsplit + 31) / 32 * 32;
    MZK_CHECK_ARG(chunk <= kIdxCap, "sparse_mqa: %lld entries per split exceed %d; use nsplit >= %lld",
                  (long long)chunk, kIdxCap, (long long)((total_max + kIdxCap - 33) / (kIdxCap - 32)));
  }
  const int stride = part_only ? split_total : nsplit;
  if (part_only || nsplit > 1) {
    const int64_t need = rows * stride * static_cast<int64_t>(H) * (2 * D + 8);
    MZK_CHECK_ARG(workspace && workspace_bytes >= need, "sparse_mqa: workspace needs %lld bytes", (long long)need);
  }
  MZK_CHECK_ARG(aligned16(q) && aligned16(win) && aligned16(dense) && aligned16(main_kv) && aligned16(workspace) &&
                    aligned16(out),
                "sparse_mqa: q, caches, workspace and out must be 16-byte aligned");
  AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.rows = rows;
  p.S = S;
  p.positions = positions;
  p.win = static_cast<const uint8_t*>(win);
  p.win_batch_entries = win_batch_entries;
  p.win_cap = win_cap;
  p.window = window;
  p.dense = static_cast<const uint8_t*>(dense);
  p.dense_batch_entries = dense_batch_entries;
  p.dense_cap = dense_cap;
  p.dense_ratio = dense_ratio < 1 ? 1 : dense_ratio;
  p.main = static_cast<const uint8_t*>(main_kv);
  p.main_batch_entries = main_batch_entries;
  p.G = G;
  p.idx = idx;
  p.idx_row_stride = idx_row_stride;
  p.topk = main_kv ? topk : 0;
  p.H = H;
  p.sinks = sinks;
  p.scale_log2 = (1.0f / __builtin_sqrtf(static_cast<float>(D))) * kLog2e;
  p.nsplit = nsplit;
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.split_stride = stride;
  p.write_final = !part_only && nsplit == 1;
  if (workspace) {
    uint16_t* po = reinterpret_cast<uint16_t*>(workspace);
    float* pml = reinterpret_cast<float*>(po + rows * stride * static_cast<int64_t>(H) * D);
    const int base = part_only ? split_base : 0;
    p.part_o = po + static_cast<int64_t>(base) * H * D;
    p.part_ml = pml + static_cast<int64_t>(base) * H * 2;
  }
  p.rope_cos = static_cast<const uint16_t*>(rope_cos);
  p.rope_sin = static_cast<const uint16_t*>(rope_sin);
  p.sel_scores = sel_scores;
  p.sel_stride = sel_stride;
  p.sel_out = sel_out;
  p.sel_out_stride = sel_out_stride;
  if (sel_scores) p.idx = nullptr;
  // The split merge inside the attention launch: a full call of the D-split kernel with
  // nsplit dividing 64, rows or rows * (64-head groups) a multiple of 8 (the mappings that put
  // a group's splits on one XCD), a workspace that holds the merge records, and a grid of at
  // most one workgroup per CU (every workgroup of a group must run at once; one fills a CU's
  // LDS).
  const int merge_mode = g_merge_mode.load(std::memory_order_relaxed);
  const int64_t nhg64 = (H + 63) / 64;
  if (merge_mode != 0 && !part_only && nsplit > 1 && out != nullptr && D > 256 && 64 % nsplit == 0 &&
      ((rows & 7) == 0 || ((rows * nhg64) & 7) == 0)) {
    const int64_t nhg = nhg64;
    const int64_t off = align16_bytes(rows * stride * static_cast<int64_t>(H) * (2 * D + 8));
    const int cus = device_cus();
    if (workspace_bytes >= off + merge_rec_bytes(rows, H) && cus > 0 && rows * nsplit * nhg <= cus) {
      p.merge_rec = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(workspace) + off);
      p.merge_err = p.merge_rec + 4 * rows * nhg;
      p.merge_fence = merge_mode == 2;
    }
  }
  hipStream_t s = as_stream(stream);
  bool merged = false;
  int rc = dispatch(fmt, D, nope, p, rows, s, &merged);
  if (rc) return rc;
  MZK_LAUNCH_CHECK("sparse_mqa");
  if (!part_only && nsplit > 1 && out != nullptr && !merged)
    return combine_impl(workspace, B, S, H, D, nsplit, sinks, rope_cos, rope_sin, rope_dim, out, lse, advance, stream);
  if (advance != nullptr) {  // no merge launch follows: one of its own
    advance_kernel<<<static_cast<unsigned>((rows + 255) / 256), 256, 0, s>>>(advance, rows);
    MZK_LAUNCH_CHECK("sparse_mqa_advance");
  }
  return MZK_OK;
}

int combine_impl(const float* workspace, int64_t B, int64_t S, int H, int D, int nsplit, const float* sinks,
                 const void* rope_cos, const void* rope_sin, int rope_dim, void* out, float* lse, int64_t* advance,
                 void* stream) {
  MZK_CHECK_ARG(B >= 0 && S >= 0 && H >= 1 && nsplit >= 1, "sparse_mqa_combine: bad sizes");
  if (rope_cos || rope_sin) {
    MZK_CHECK_ARG(rope_cos && rope_sin, "sparse_mqa_combine_rope: cos and sin go together");
    MZK_CHECK_ARG(rope_dim >= 8 && rope_dim <= D && rope_dim % 8 == 0,
                  "sparse_mqa_combine_rope: rope_dim must be a multiple of 8 in [8, D] (got %d)", rope_dim);
    MZK_CHECK_ARG(aligned16(rope_cos) && aligned16(rope_sin),
                  "sparse_mqa_combine_rope: cos and sin must be 16-byte aligned");
  }
  const int64_t rows = B * S;
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(workspace && out && lse, "sparse_mqa_combine: null pointer");
  MZK_CHECK_ARG(aligned16(workspace) && aligned16(out), "sparse_mqa_combine: workspace and out must be 16-byte aligned");
  const uint16_t* po = reinterpret_cast<const uint16_t*>(workspace);
  const float* pml = reinterpret_cast<const float*>(po + rows * nsplit * static_cast<int64_t>(H) * D);
  uint16_t* o = static_cast<uint16_t*>(out);
  const uint16_t* rc_ = static_cast<const uint16_t*>(rope_cos);
  const uint16_t* rs_ = static_cast<const uint16_t*>(rope_sin);
  hipStream_t s = as_stream(stream);
  switch (D) {
    case 64: launch_combine<64>(po, pml, nsplit, H, S, sinks, o, lse, rows, rc_, rs_, rope_dim, advance, s); break;
    case 96: launch_combine<96>(po, pml, nsplit, H, S, sinks, o, lse, rows, rc_, rs_, rope_dim, advance, s); break;
    case 128: launch_combine<128>(po, pml, nsplit, H, S, sinks, o, lse, rows, rc_, rs_, rope_dim, advance, s); break;
    case 160: launch_combine<160>(po, pml, nsplit, H, S, sinks, o, lse, rows, rc_, rs_, rope_dim, advance, s); break;
    case 256: launch_combine<256>(po, pml, nsplit, H, S, sinks, o, lse, rows, rc_, rs_, rope_dim, advance, s); break;
    case 576: launch_combine<576>(po, pml, nsplit, H, S, sinks, o, lse, rows, rc_, rs_, rope_dim, advance, s); break;
    default: set_last_error("sparse_mqa_combine: unsupported head dim %d", D); return MZK_EUNSUPPORTED;
  }
  MZK_LAUNCH_CHECK("sparse_mqa_combine");
  return MZK_OK;
}
}  // namespace

extern "C" int mzk_sparse_mqa(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                              const int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                              int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                              int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                              const int32_t* idx, int64_t idx_row_stride, int topk, const float* sinks, int nsplit,
                              float* workspace, int64_t workspace_bytes, void* out, float* lse, void* stream) {
  return sparse_mqa_impl(q, B, S, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                         dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, idx,
                         idx_row_stride, topk, sinks, nsplit, workspace, workspace_bytes, out, lse, nullptr, nullptr, 0,
                         0, -1, stream);
}

extern "C" int mzk_sparse_mqa_rope(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                                   const int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                                   int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                                   int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                                   const int32_t* idx, int64_t idx_row_stride, int topk, const float* sinks,
                                   int nsplit, float* workspace, int64_t workspace_bytes, void* out, float* lse,
                                   const void* rope_cos, const void* rope_sin, int rope_dim, void* stream) {
  MZK_CHECK_ARG(rope_cos && rope_sin, "sparse_mqa_rope: cos and sin are required");
  return sparse_mqa_impl(q, B, S, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                         dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, idx,
                         idx_row_stride, topk, sinks, nsplit, workspace, workspace_bytes, out, lse, rope_cos, rope_sin,
                         rope_dim, 0, -1, stream);
}

extern "C" int mzk_sparse_mqa_advance(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                                      int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                                      int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                                      int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                                      const int32_t* idx, int64_t idx_row_stride, int topk, const float* sinks,
                                      int nsplit, float* workspace, int64_t workspace_bytes, void* out, float* lse,
                                      const void* rope_cos, const void* rope_sin, int rope_dim, void* stream) {
  MZK_CHECK_ARG(S == 1, "sparse_mqa_advance: one query per row (a decode step), got S = %lld", (long long)S);
  MZK_CHECK_ARG(out != nullptr && lse != nullptr, "sparse_mqa_advance: out and lse are required");
  return sparse_mqa_impl(q, B, S, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                         dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, idx,
                         idx_row_stride, topk, sinks, nsplit, workspace, workspace_bytes, out, lse, rope_cos, rope_sin,
                         rope_dim, 0, -1, stream, positions);
}

extern "C" int mzk_sparse_mqa_select(const void* q, int64_t B, int H, int D, int fmt, int nope, int64_t* positions,
                                     int advance, const void* win, int64_t win_batch_entries, int win_cap, int window,
                                     const void* dense, int64_t dense_batch_entries, int dense_cap, int dense_ratio,
                                     const void* main_kv, int64_t main_batch_entries, int64_t G, const float* scores,
                                     int64_t score_stride, int topk, int32_t* idx_out, int64_t idx_out_stride,
                                     const float* sinks, int nsplit, float* workspace, int64_t workspace_bytes,
                                     void* out, float* lse, const void* rope_cos, const void* rope_sin, int rope_dim,
                                     void* stream) {
  MZK_CHECK_ARG(B >= 0 && G >= 0 && topk >= 0, "sparse_mqa_select: negative size");
  MZK_CHECK_ARG(idx_out != nullptr && scores != nullptr && main_kv != nullptr,
                "sparse_mqa_select: needs scores, the main cache and idx_out");
  MZK_CHECK_ARG((out != nullptr && lse != nullptr) || (out == nullptr && lse == nullptr && nsplit > 1 && !advance),
                "sparse_mqa_select: out and lse, or neither (split partials only: nsplit > 1, no advance)");
  MZK_CHECK_ARG(score_stride >= G && idx_out_stride >= topk, "sparse_mqa_select: strides smaller than the row");
  if (B == 0) return MZK_OK;
  // the selecting kernel instance: the FP8 latent decode kernel, 16 scores per thread of its
  // 512, whole float4 / int4 groups
  const bool in_launch = fmt == 1 && D == 576 && nope == 512 && G >= 4 && G <= 8192 && G % 4 == 0 &&
                         score_stride % 4 == 0 && aligned16(scores) && topk >= 4 && topk <= 2048 && topk % 4 == 0 &&
                         idx_out_stride % 4 == 0 && aligned16(idx_out) && nsplit >= 1 && nsplit <= 65535 &&
                         window >= 0 && dense_cap >= 0 &&
                         dsplit_all_tables(window, dense, dense_cap, main_kv, topk, nsplit);
  int64_t* adv = advance ? positions : nullptr;
  if (!in_launch) {  // the top-k launch, then the attention over its list
    int rc = mzk_topk_rows(scores, B, G, score_stride, topk, idx_out, idx_out_stride, stream);
    if (rc) return rc;
    return sparse_mqa_impl(q, B, 1, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                           dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, idx_out,
                           idx_out_stride, topk, sinks, nsplit, workspace, workspace_bytes, out, lse, rope_cos,
                           rope_sin, rope_dim, 0, -1, stream, adv);
  }
  return sparse_mqa_impl(q, B, 1, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                         dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, nullptr, topk,
                         topk, sinks, nsplit, workspace, workspace_bytes, out, lse, rope_cos, rope_sin, rope_dim, 0, -1,
                         stream, adv, scores, score_stride, idx_out, idx_out_stride);
}

extern "C" int mzk_sparse_mqa_part(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                                   const int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                                   int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                                   int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                                   const int32_t* idx, int64_t idx_row_stride, int topk, int nsplit, int split_base,
                                   int split_total, float* workspace, int64_t workspace_bytes, const void* rope_cos,
                                   const void* rope_sin, int rope_dim, void* stream) {
  MZK_CHECK_ARG(split_total >= 1, "sparse_mqa_part: split_total must be >= 1");
  return sparse_mqa_impl(q, B, S, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                         dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, idx,
                         idx_row_stride, topk, nullptr, nsplit, workspace, workspace_bytes, nullptr, nullptr, rope_cos,
                         rope_sin, rope_dim, split_base, split_total, stream);
}

// ---- the allocation-free form -------------------------------------------------------
// The split partials live in a file-scope device array instead of a caller's workspace.
// In host code `scratch` is only a stand-in symbol: its device address (one per GPU) comes
// from hipGetSymbolAddress, taken once per device on that device's first call and kept.
namespace {
constexpr int64_t kScratchBytes = MZK_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// The calling thread's current device's copy of `scratch` (nullptr + error text on failure).
void* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_last_error("sparse_mqa_noalloc: no current HIP device (or device id >= %d)", kScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_last_error("sparse_mqa_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int mzk_sparse_mqa_noalloc(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                                      const int64_t* positions, const void* win, int64_t win_batch_entries,
                                      int win_cap, int window, const void* dense, int64_t dense_batch_entries,
                                      int dense_cap, int dense_ratio, const void* main_kv, int64_t main_batch_entries,
                                      int64_t G, const int32_t* idx, int64_t idx_row_stride, int topk,
                                      const float* sinks, int nsplit, void* out, float* lse, const void* rope_cos,
                                      const void* rope_sin, int rope_dim, void* stream) {
  MZK_CHECK_ARG(B >= 0 && S >= 0 && H >= 1 && D > 0 && nsplit >= 1, "sparse_mqa_noalloc: bad sizes");
  MZK_CHECK_ARG(B == 0 || S <= 0x7fffffff / B, "sparse_mqa_noalloc: too many rows");
  // the partials stay in the private scratch array: only the merged output is observable
  MZK_CHECK_ARG(out != nullptr && lse != nullptr, "sparse_mqa_noalloc: out and lse are required");
  const int64_t need = nsplit > 1 ? B * S * nsplit * static_cast<int64_t>(H) * (2 * D + 8) : 0;
  MZK_CHECK_ARG(need <= kScratchBytes,
                "sparse_mqa_noalloc: %lld rows x %d splits x %d heads need %lld bytes of split partials, above the "
                "%lld-byte scratch; use fewer splits or rows, or mzk_sparse_mqa with a workspace",
                (long long)(B * S), nsplit, H, (long long)need, (long long)kScratchBytes);
  float* ws = nullptr;
  if (need > 0 && B * S > 0) {
    ws = static_cast<float*>(device_scratch());
    if (!ws) return MZK_ELAUNCH;
  }
  return sparse_mqa_impl(q, B, S, H, D, fmt, nope, positions, win, win_batch_entries, win_cap, window, dense,
                         dense_batch_entries, dense_cap, dense_ratio, main_kv, main_batch_entries, G, idx,
                         idx_row_stride, topk, sinks, nsplit, ws, need, out, lse, rope_cos, rope_sin, rope_dim, 0, -1,
                         stream);
}

extern "C" int mzk_sparse_mqa_workspace_bytes(int64_t rows, int H, int D, int nsplit, int64_t* bytes) {
  MZK_CHECK_ARG(bytes != nullptr, "sparse_mqa_workspace_bytes: null output");
  MZK_CHECK_ARG(rows >= 0 && H >= 1 && D > 0 && nsplit >= 1, "sparse_mqa_workspace_bytes: bad sizes");
  *bytes = nsplit > 1 ? align16_bytes(rows * nsplit * static_cast<int64_t>(H) * (2 * D + 8)) + merge_rec_bytes(rows, H)
                      : 0;
  return MZK_OK;
}

extern "C" int mzk_sparse_mqa_set_merge(int mode) {
  MZK_CHECK_ARG(mode >= 0 && mode <= 2, "sparse_mqa_set_merge: mode must be 0, 1 or 2 (got %d)", mode);
  g_merge_mode.store(mode, std::memory_order_relaxed);
  return MZK_OK;
}

extern "C" int mzk_sparse_mqa_combine(const float* workspace, int64_t B, int64_t S, int H, int D, int nsplit,
                                      const float* sinks, void* out, float* lse, void* stream) {
  return combine_impl(workspace, B, S, H, D, nsplit, sinks, nullptr, nullptr, 0, out, lse, nullptr, stream);
}

extern "C" int mzk_sparse_mqa_combine_rope(const float* workspace, int64_t B, int64_t S, int H, int D, int nsplit,
                                           const float* sinks, const void* rope_cos, const void* rope_sin,
                                           int rope_dim, void* out, float* lse, void* stream) {
  MZK_CHECK_ARG(rope_cos && rope_sin, "sparse_mqa_combine_rope: cos and sin are required");
  return combine_impl(workspace, B, S, H, D, nsplit, sinks, rope_cos, rope_sin, rope_dim, out, lse, nullptr, stream);
}

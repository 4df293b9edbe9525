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
#include "common.h"

namespace mzk {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
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
  float* part_o;  // [rows, nsplit, H, D]
  float* part_ml; // [rows, nsplit, H, 2]
};

template <int FMT, int D, int NOPE>
struct Layout {
  static constexpr int kEntryBytes = FMT == kFmtFp8 ? NOPE + 4 * (NOPE / 128) + 2 * (D - NOPE) : 2 * D;
  static constexpr int kChunks = D / 8;  // 8-channel chunks per entry
};

// Entry held by register j of lane l in a 32x32 MFMA result: 8*(j/4) + 4*(l/32) + j%4.
__device__ __forceinline__ int c_entry(int j, int lane) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }

// Workgroup barrier that waits only for this wave's LDS operations (not for vector
// memory: the tile DMA stays in flight across it).  The "memory" clobber keeps the
// compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

constexpr int kIdxCap = 4096;  // sparse indices of one split staged in LDS

typedef const uint8_t __attribute__((address_space(1)))* gptr_t;  // global (not flat) loads
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ T gload(gptr_t p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

// Raw bytes of one 8-channel chunk of an entry, fetched from HBM a tile ahead of use.
struct RawChunk {
  uint4 v;   // bf16: 8 channels; fp8 nope: .x/.y = 8 codes; fp8 rope: 8 bf16
  float s;   // fp8 nope: the chunk's 128-channel block scale
};

template <int FMT, int D, int NOPE>
__device__ __forceinline__ RawChunk fetch_chunk(gptr_t e, int c) {
  RawChunk r;
  r.s = 1.0f;
  if constexpr (FMT == kFmtBf16) {
    const u32x4 v = gload<u32x4>(e + 16 * c);
    r.v = uint4{v.x, v.y, v.z, v.w};
  } else {
    constexpr int NB = NOPE / 128;
    if (c < NOPE / 8) {
      const u32x2 raw = gload<u32x2>(e + 8 * c);
      r.v = uint4{raw.x, raw.y, 0u, 0u};
      r.s = gload<float>(e + NOPE + 4 * (c >> 4));
    } else {
      const u32x4 v = gload<u32x4>(e + NOPE + 4 * NB + 16 * (c - NOPE / 8));
      r.v = uint4{v.x, v.y, v.z, v.w};
    }
  }
  return r;
}

// 8 bf16 (as 4 dwords) of a fetched chunk: e4m3 codes times the pow2 block scale through
// the hardware conversion (exact in bf16), rope / bf16 chunks as they are.
template <int FMT, int NOPE>
__device__ __forceinline__ uint4 decode_chunk(const RawChunk& r, int c) {
  if constexpr (FMT == kFmtBf16) {
    return r.v;
  } else {
    if (c >= NOPE / 8) return r.v;
    return dequant_fp8x8_bf16(uint2{r.v.x, r.v.y}, r.s);
  }
}

template <int FMT, int D, int NOPE, int HG, int DS>
struct Smem {
  static constexpr int KT = kTile * (2 * D + 16);
  static constexpr int SX = DS > 1 ? HG * DS * 16 * 64 * 4 : 0;
  static constexpr int LDS = KT + SX;
};

template <int FMT, int D, int NOPE, int HG, int DS>
__global__ void __launch_bounds__(HG * DS * 64) sparse_mqa_kernel(const AttnParams p) {
  using L = Layout<FMT, D, NOPE>;
  using M = Smem<FMT, D, NOPE, HG, DS>;
  constexpr int NT = HG * DS * 64;
  constexpr int DPART = D / DS;           // channels per D-part
  constexpr int QSTEPS = DPART / 16;      // QK MFMA steps per wave
  constexpr int NDB = DPART / 32;         // 32-channel blocks of O per wave
  constexpr int KT_PITCH = 2 * D + 16;    // bytes per Kt row (16 B pad spreads LDS banks)
  constexpr int NTAB = 2;                 // entry tables: current and next tile
  constexpr int TPE = NT / kTile;         // threads per entry in the load/dequant phase
  constexpr int CPT = (L::kChunks + TPE - 1) / TPE;  // chunks per thread
  static_assert(DPART % 32 == 0, "D-part must be a multiple of 32 channels");

  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* kt = smem;                                           // [32][KT_PITCH] bf16 tile
  float* sx = reinterpret_cast<float*>(kt + M::KT);             // [waves][16][64] partial S
  __shared__ const uint8_t* tab_ptr[NTAB][kTile];
  __shared__ uint32_t tab_mask[NTAB];
  __shared__ int32_t sidx[kIdxCap];  // this split's sparse indices

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hg = wave / DS;
  const int ds = wave % DS;
  const int half = lane >> 5;
  const int64_t row = blockIdx.y;
  const int split = blockIdx.x;
  const int64_t b = row / p.S;
  const int64_t pos = p.positions[row];

  // ---- the row's virtual entry list and this split's share of it
  const int64_t nw = pos + 1 < p.window ? pos + 1 : p.window;
  int64_t nd = 0;
  if (p.dense) {
    nd = (pos + 1) / p.dense_ratio;
    if (nd > p.dense_cap) nd = p.dense_cap;
  }
  const int64_t ns = p.main ? p.topk : 0;
  const int64_t total = nw + nd + ns;
  int64_t chunk = (total + p.nsplit - 1) / p.nsplit;
  chunk = (chunk + kTile - 1) / kTile * kTile;
  const int64_t v_begin = split * chunk;
  const int64_t v_end = v_begin + chunk < total ? v_begin + chunk : total;
  const int ntiles = v_end > v_begin ? static_cast<int>((v_end - v_begin + kTile - 1) / kTile) : 0;

  const uint8_t* win_b = p.win + b * p.win_batch_entries * L::kEntryBytes;
  const uint8_t* dense_b = p.dense ? p.dense + b * p.dense_batch_entries * L::kEntryBytes : nullptr;
  const uint8_t* main_b = p.main ? p.main + b * p.main_batch_entries * L::kEntryBytes : nullptr;
  const int32_t* idx_row = p.idx ? p.idx + row * p.idx_row_stride : nullptr;

  // this split's slice of the sparse index list, staged in LDS once (the host guarantees
  // it fits kIdxCap), so the tile loop issues no vector-memory reads besides the tile DMA
  const int64_t sp_begin = v_begin > nw + nd ? v_begin - nw - nd : 0;
  const int64_t sp_end = v_end > nw + nd ? v_end - nw - nd : 0;
  for (int64_t s = sp_begin + tid; s < sp_end; s += NT) sidx[s - sp_begin] = idx_row[s];
  __syncthreads();  // the slice is read by other threads below
  auto load_slot = [&](int64_t v) -> int64_t {
    return (v >= nw + nd && v < v_end) ? static_cast<int64_t>(sidx[v - nw - nd - sp_begin]) : -1;
  };
  // entry table of tile `t` (threads 0..31); `g` = this thread's prefetched sparse index
  auto build_table = [&](int t, int64_t g) {
    if (tid < kTile) {
      const int64_t v = v_begin + static_cast<int64_t>(t) * kTile + tid;
      const uint8_t* ptr = nullptr;
      if (v < v_end) {
        if (v < nw) {
          const int64_t tok = pos - nw + 1 + v;
          ptr = win_b + (p.win_cap ? tok % p.win_cap : tok) * L::kEntryBytes;
        } else if (v < nw + nd) {
          ptr = dense_b + (v - nw) * L::kEntryBytes;
        } else if (g >= 0 && g < p.G) {
          ptr = main_b + g * L::kEntryBytes;
        }
      }
      tab_ptr[t % NTAB][tid] = ptr;
      const uint64_t bal = __ballot(ptr != nullptr);
      if (tid == 0) tab_mask[t % NTAB] = static_cast<uint32_t>(bal);
    }
  };
  // load phase: thread owns entry tid / TPE, 8-channel chunks (tid % TPE) + TPE*k; the
  // next tile's chunks are fetched into registers while the current tile computes
  const int my_entry = tid / TPE;
  const int my_c0 = tid % TPE;
  RawChunk raw[CPT];
  auto fetch_tile = [&](int t) {
    const gptr_t e = (gptr_t)(tab_ptr[t % NTAB][my_entry]);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = my_c0 + TPE * k;
      raw[k].v = uint4{0u, 0u, 0u, 0u};
      raw[k].s = 1.0f;
      if (e != nullptr && c < L::kChunks) raw[k] = fetch_chunk<FMT, D, NOPE>(e, c);
    }
  };

  // ---- q fragments (B operand of S^T = K Q^T): head, channels of this wave's D-part
  const int head = blockIdx.z * (HG * 32) + hg * 32 + (lane & 31);
  const bool head_ok = head < p.H;
  v8bf qf[QSTEPS];
  {
    const uint16_t* qrow = p.q + (row * p.H + (head_ok ? head : 0)) * D + ds * DPART + half * 8;
#pragma unroll
    for (int st = 0; st < QSTEPS; ++st) {
      uint4 v = head_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * st) : uint4{0, 0, 0, 0};
      qf[st] = __builtin_bit_cast(v8bf, v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w});
    }
  }

  v16f acc_o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc_o[i] = v16f{};
  float m_run = -__builtin_huge_valf();
  float l_run = 0.0f;

  int64_t g_pref = -1;  // prefetched sparse index for table t+2 (threads 0..31)
  if (ntiles > 0) {
    build_table(0, tid < kTile ? load_slot(v_begin + tid) : -1);
    build_table(1, tid < kTile ? load_slot(v_begin + kTile + tid) : -1);
    if (tid < kTile) g_pref = load_slot(v_begin + 2 * kTile + tid);
    __syncthreads();
    fetch_tile(0);
  }

#pragma unroll 1
  for (int t = 0; t < ntiles; ++t) {
    const int tb = t % NTAB;
    // 1. dequantize the fetched tile into Kt (empty slots are zero); the table of tile
    //    t+2 replaces tile t's (no longer read: the softmax below uses its mask copy)
    const uint32_t vmask = tab_mask[tb];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = my_c0 + TPE * k;
      if (c < L::kChunks)
        *reinterpret_cast<uint4*>(kt + my_entry * KT_PITCH + 16 * c) = decode_chunk<FMT, NOPE>(raw[k], c);
    }
    lds_barrier();  // Kt complete; every wave has read tile t's table
    build_table(t + 2, g_pref);
    if (tid < kTile) g_pref = load_slot(v_begin + static_cast<int64_t>(t + 3) * kTile + tid);
    // 2. the next tile's HBM reads overlap this tile's MFMA work (stays in flight across
    //    the LDS-only barriers below)
    if (t + 1 < ntiles) fetch_tile(t + 1);

    // 3. S^T partial over this wave's D-part
    v16f s = v16f{};
    {
      const uint8_t* krow = kt + (lane & 31) * KT_PITCH + 2 * (ds * DPART + half * 8);
      if constexpr (DS == 1) {
        v16f s1 = v16f{};  // two independent chains (even / odd K-steps), summed in that order
#pragma unroll
        for (int st = 0; st < QSTEPS; ++st) {
          const uint4 kv = *reinterpret_cast<const uint4*>(krow + 32 * st);
          const v8bf ka = __builtin_bit_cast(v8bf, v4i{(int)kv.x, (int)kv.y, (int)kv.z, (int)kv.w});
          if (st & 1) s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[st], s1, 0, 0, 0);
          else s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[st], s, 0, 0, 0);
        }
        s = s + s1;
      } else {
#pragma unroll
        for (int st = 0; st < QSTEPS; ++st) {
          const uint4 kv = *reinterpret_cast<const uint4*>(krow + 32 * st);
          const v8bf ka = __builtin_bit_cast(v8bf, v4i{(int)kv.x, (int)kv.y, (int)kv.z, (int)kv.w});
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[st], s, 0, 0, 0);
        }
        // partial S of each D-part through LDS ([wave][j][lane], conflict-free), summed in
        // D-part order by every wave of the head group
#pragma unroll
        for (int j = 0; j < 16; ++j) sx[(wave * 16 + j) * 64 + lane] = s[j];
        lds_barrier();
#pragma unroll
        for (int j = 0; j < 16; ++j) s[j] = sx[((hg * DS) * 16 + j) * 64 + lane];
#pragma unroll
        for (int part = 1; part < DS; ++part) {
#pragma unroll
          for (int j = 0; j < 16; ++j) s[j] = s[j] + sx[((hg * DS + part) * 16 + j) * 64 + lane];
        }
      }
    }

    // 4. online softmax (exp2 domain), lane-local per head.  The running max is only
    // raised when a head's tile max exceeds it by more than kLazy (log2 units): until then
    // exp2(s - m) <= 2^kLazy stays exact enough in fp32/bf16 and O needs no rescale.  The
    // decision is wave-uniform, so most tiles skip the O^T *= alpha pass.
    float tmax = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      s[j] = ((vmask >> c_entry(j, lane)) & 1u) ? s[j] * p.scale_log2 : -__builtin_huge_valf();
      tmax = fmaxf(tmax, s[j]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    constexpr float kLazy = 8.0f;
    const bool raise = tmax > m_run + kLazy;
    if (__any(raise)) {
      const float m_new = raise ? tmax : m_run;
      const float alpha = (m_run == -__builtin_huge_valf()) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run = l_run * alpha;
#pragma unroll
      for (int i = 0; i < NDB; ++i) acc_o[i] = acc_o[i] * alpha;
      m_run = m_new;
    }
    float psum = 0.0f;
    uint32_t pk[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // v_exp_f32 directly: arguments are <= kLazy, results below 2^-126 may flush to 0
      const float p0 = s[2 * i] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(s[2 * i] - m_run);
      const float p1 = s[2 * i + 1] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(s[2 * i + 1] - m_run);
      psum = psum + p0 + p1;
      pk[i] = pack_bf16x2(p0, p1);
    }
    psum = psum + __shfl_xor(psum, 32, 64);
    l_run = l_run + psum;

    // 5. O^T += V^T . P^T.  P^T is the S^T result in registers: PV step ks consumes
    // registers 8ks..8ks+7 = entries 16ks + {0..3, 8..11} + 4*half.  The matching V^T
    // operand (32 channels x 8 entries) comes from Kt with ds_read_b64_tr_b16: inside a
    // 16-lane group, lane i receives element i%4 of the 4-element rows the lanes
    // 4k + i/4 (k = 0..3) point at.  Lane j therefore points at
    // Kt[e0 + j/4][d0 + 4*(j%4)] and receives Kt[e0 + k][d0 + i] for k = 0..3:
    // four consecutive entries of its own channel, two reads per fragment.
    const v8bf pf0 = __builtin_bit_cast(v8bf, v4i{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]});
    const v8bf pf1 = __builtin_bit_cast(v8bf, v4i{(int)pk[4], (int)pk[5], (int)pk[6], (int)pk[7]});
    {
      const int grp = lane >> 4;  // 16-lane group: channel half (grp & 1), entry half (grp >> 1)
      const int j = lane & 15;
      const int e0 = 4 * (grp >> 1) + (j >> 2);
      const int dcol = ds * DPART + 16 * (grp & 1) + 4 * (j & 3);
      const uint8_t* tr0 = kt + e0 * KT_PITCH + 2 * dcol;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint8_t* tp = tr0 + 64 * db;
        const v4s r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp));                     // entries 0-3 (+4h)
        const v4s r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 8 * KT_PITCH));      // entries 8-11
        const v4s r2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 16 * KT_PITCH));     // entries 16-19
        const v4s r3 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4s(tp + 24 * KT_PITCH));     // entries 24-27
        const v8bf a0 = __builtin_bit_cast(v8bf, v8s{r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]});
        const v8bf a1 = __builtin_bit_cast(v8bf, v8s{r2[0], r2[1], r2[2], r2[3], r3[0], r3[1], r3[2], r3[3]});
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, pf0, acc_o[db], 0, 0, 0);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, pf1, acc_o[db], 0, 0, 0);
      }
    }
    lds_barrier();  // Kt and the S exchange buffer are free for the next tile
  }

  // ---- epilogue.  acc_o[db][j] holds O^T[d][head], d = ds*DPART + db*32 + c_entry(j, lane)
  if (!head_ok) return;
  if (p.out != nullptr && p.nsplit == 1) {
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
    uint16_t* orow = p.out + (row * p.H + head) * D + ds * DPART;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = db * 32 + 8 * g4 + 4 * half;
        const uint32_t w0 = f32_to_bf16(acc_o[db][4 * g4 + 0] * o_scale) |
                            (static_cast<uint32_t>(f32_to_bf16(acc_o[db][4 * g4 + 1] * o_scale)) << 16);
        const uint32_t w1 = f32_to_bf16(acc_o[db][4 * g4 + 2] * o_scale) |
                            (static_cast<uint32_t>(f32_to_bf16(acc_o[db][4 * g4 + 3] * o_scale)) << 16);
        *reinterpret_cast<uint2*>(orow + d0) = uint2{w0, w1};
      }
    }
    if (ds == 0 && half == 0) {
      const int64_t s_idx = row % p.S;
      p.lse[(b * p.H + head) * p.S + s_idx] = (m_fin + __log2f(l_fin)) * kLn2;
    }
  } else {
    float* prow = p.part_o + ((row * p.nsplit + split) * p.H + head) * static_cast<int64_t>(D) + ds * DPART;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = db * 32 + 8 * g4 + 4 * half;
        *reinterpret_cast<float4*>(prow + d0) =
            float4{acc_o[db][4 * g4], acc_o[db][4 * g4 + 1], acc_o[db][4 * g4 + 2], acc_o[db][4 * g4 + 3]};
      }
    }
    if (ds == 0 && half == 0) {
      float* ml = p.part_ml + ((row * p.nsplit + split) * p.H + head) * 2;
      ml[0] = m_run;
      ml[1] = l_run;
    }
  }
}

// Merge the split partials of one (row, head) with the sink: one workgroup per (row, head).
template <int D>
__global__ void __launch_bounds__(64) combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                     int nsplit, int H, int64_t S, const float* __restrict__ sinks,
                                                     uint16_t* __restrict__ out, float* __restrict__ lse) {
  const int64_t row = blockIdx.x;
  const int head = blockIdx.y;
  const int lane = threadIdx.x;
  float M = -__builtin_huge_valf();
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, part_ml[((row * nsplit + s) * H + head) * 2]);
  const float sk = sinks ? sinks[head] * kLog2e : -__builtin_huge_valf();
  M = fmaxf(M, sk);
  float L = sinks ? exp2f(sk - M) : 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float m = part_ml[((row * nsplit + s) * H + head) * 2];
    const float l = part_ml[((row * nsplit + s) * H + head) * 2 + 1];
    if (m != -__builtin_huge_valf()) L = L + l * exp2f(m - M);
  }
  const float inv = 1.0f / L;
  for (int d = 4 * lane; d < D; d += 4 * 64) {
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < nsplit; ++s) {
      const float m = part_ml[((row * nsplit + s) * H + head) * 2];
      if (m == -__builtin_huge_valf()) continue;
      const float wgt = exp2f(m - M);
      const float4 o = *reinterpret_cast<const float4*>(part_o + ((row * nsplit + s) * H + head) * static_cast<int64_t>(D) + d);
      acc.x = acc.x + o.x * wgt;
      acc.y = acc.y + o.y * wgt;
      acc.z = acc.z + o.z * wgt;
      acc.w = acc.w + o.w * wgt;
    }
    const uint32_t w0 = f32_to_bf16(acc.x * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.y * inv)) << 16);
    const uint32_t w1 = f32_to_bf16(acc.z * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.w * inv)) << 16);
    *reinterpret_cast<uint2*>(out + (row * H + head) * static_cast<int64_t>(D) + d) = uint2{w0, w1};
  }
  if (lane == 0) {
    const int64_t b = row / S, s_idx = row % S;
    lse[(b * H + head) * S + s_idx] = (M + __log2f(L)) * kLn2;
  }
}

template <int FMT, int D, int NOPE, int HG, int DS>
int launch_attn(const AttnParams& p, int64_t rows, hipStream_t s) {
  constexpr int NT = HG * DS * 64;
  constexpr size_t lds = Smem<FMT, D, NOPE, HG, DS>::LDS;
  static_assert(lds <= 150 * 1024, "LDS budget");
  auto kern = sparse_mqa_kernel<FMT, D, NOPE, HG, DS>;
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                        static_cast<int>(lds));
    attr_set = true;
  }
  // heads beyond HG*32 go to further workgroups along z (each re-reads the KV tiles)
  dim3 grid(static_cast<unsigned>(p.nsplit), static_cast<unsigned>(rows), static_cast<unsigned>((p.H + HG * 32 - 1) / (HG * 32)));
  kern<<<grid, NT, lds, s>>>(p);
  return MZK_OK;
}

template <int FMT, int D, int NOPE>
int dispatch_heads(const AttnParams& p, int64_t rows, hipStream_t s) {
  // D > 256: two waves per 32 heads, each owning half of D (keeps q + O^T within 256 VGPRs)
  constexpr int DS = D > 256 ? 2 : 1;
  // at most 64 heads per workgroup: q fragments + O^T accumulators of 64 heads x D fill the
  // register file of one CU at one wave per SIMD; more heads use several workgroups.
  if (p.H <= 32) return launch_attn<FMT, D, NOPE, 1, DS>(p, rows, s);
  if (p.H <= 128) return launch_attn<FMT, D, NOPE, 2, DS>(p, rows, s);
  set_last_error("sparse_mqa: at most 128 heads (got %d)", p.H);
  return MZK_EUNSUPPORTED;
}

int dispatch(int fmt, int D, int nope, const AttnParams& p, int64_t rows, hipStream_t s) {
  if (fmt == kFmtFp8) {
    if (D == 576 && nope == 512) return dispatch_heads<kFmtFp8, 576, 512>(p, rows, s);
    if (D == 160 && nope == 128) return dispatch_heads<kFmtFp8, 160, 128>(p, rows, s);
    set_last_error("sparse_mqa fp8: unsupported latent %d+%d (have 512+64, 128+32)", nope, D - nope);
    return MZK_EUNSUPPORTED;
  }
  switch (D) {
    case 64: return dispatch_heads<kFmtBf16, 64, 64>(p, rows, s);
    case 96: return dispatch_heads<kFmtBf16, 96, 96>(p, rows, s);
    case 128: return dispatch_heads<kFmtBf16, 128, 128>(p, rows, s);
    case 160: return dispatch_heads<kFmtBf16, 160, 160>(p, rows, s);
    case 256: return dispatch_heads<kFmtBf16, 256, 256>(p, rows, s);
    case 576: return dispatch_heads<kFmtBf16, 576, 576>(p, rows, s);
    default:
      set_last_error("sparse_mqa bf16: unsupported head dim %d (have 64, 96, 128, 160, 256, 576)", D);
      return MZK_EUNSUPPORTED;
  }
}

template <int D>
void launch_combine(const float* po, const float* pml, int nsplit, int H, int64_t S, const float* sinks, uint16_t* out,
                    float* lse, int64_t rows, hipStream_t s) {
  combine_kernel<D><<<dim3(static_cast<unsigned>(rows), static_cast<unsigned>(H)), 64, 0, s>>>(po, pml, nsplit, H, S,
                                                                                               sinks, out, lse);
}

}  // namespace
}  // namespace mzk

using namespace mzk;

extern "C" int mzk_sparse_mqa(const void* q, int64_t B, int64_t S, int H, int D, int fmt, int nope,
                              const int64_t* positions, const void* win, int64_t win_batch_entries, int win_cap,
                              int window, const void* dense, int64_t dense_batch_entries, int dense_cap,
                              int dense_ratio, const void* main_kv, int64_t main_batch_entries, int64_t G,
                              const int32_t* idx, int64_t idx_row_stride, int topk, const float* sinks, int nsplit,
                              float* workspace, int64_t workspace_bytes, void* out, float* lse, void* stream) {
  MZK_CHECK_ARG(B >= 0 && S >= 0 && H >= 1 && D > 0, "sparse_mqa: bad sizes");
  MZK_CHECK_ARG(fmt == 0 || fmt == 1, "sparse_mqa: fmt must be 0 (bf16) or 1 (fp8-b128)");
  MZK_CHECK_ARG(nsplit >= 1 && nsplit <= 65535, "sparse_mqa: nsplit must be in [1, 65535]");
  MZK_CHECK_ARG(window >= 1 && win != nullptr, "sparse_mqa: a window source (window >= 1) is required");
  MZK_CHECK_ARG(win_cap == 0 || win_cap >= window, "sparse_mqa: ring capacity smaller than the window");
  MZK_CHECK_ARG(!dense || (dense_ratio >= 1 && dense_cap >= 0), "sparse_mqa: dense source needs ratio >= 1");
  MZK_CHECK_ARG(!main_kv || (idx && topk >= 0 && G >= 0 && idx_row_stride >= topk && main_batch_entries >= G),
                "sparse_mqa: sparse source needs idx [rows, >= topk] and main_batch_entries >= G");
  const int64_t rows = B * S;
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(q && positions && (nsplit > 1 || (out && lse)), "sparse_mqa: null pointer");
  MZK_CHECK_ARG((out == nullptr) == (lse == nullptr), "sparse_mqa: out and lse go together");
  MZK_CHECK_ARG(rows <= 0x7fffffff, "sparse_mqa: too many rows");
  {
    const int64_t total_max = static_cast<int64_t>(window) + (dense ? dense_cap : 0) + (main_kv ? topk : 0);
    const int64_t chunk = ((total_max + nsplit - 1) / nsplit + 31) / 32 * 32;
    MZK_CHECK_ARG(chunk <= kIdxCap, "sparse_mqa: %lld entries per split exceed %d; use nsplit >= %lld",
                  (long long)chunk, kIdxCap, (long long)((total_max + kIdxCap - 33) / (kIdxCap - 32)));
  }
  if (nsplit > 1) {
    const int64_t need = rows * nsplit * static_cast<int64_t>(H) * (D + 2) * 4;
    MZK_CHECK_ARG(workspace && workspace_bytes >= need, "sparse_mqa: workspace needs %lld bytes", (long long)need);
  }
  AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
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
  p.part_o = workspace;
  p.part_ml = workspace ? workspace + rows * nsplit * static_cast<int64_t>(H) * D : nullptr;
  hipStream_t s = as_stream(stream);
  int rc = dispatch(fmt, D, nope, p, rows, s);
  if (rc) return rc;
  MZK_LAUNCH_CHECK("sparse_mqa");
  if (nsplit > 1 && out != nullptr) return mzk_sparse_mqa_combine(workspace, B, S, H, D, nsplit, sinks, out, lse, stream);
  return MZK_OK;
}

extern "C" int mzk_sparse_mqa_combine(const float* workspace, int64_t B, int64_t S, int H, int D, int nsplit,
                                      const float* sinks, void* out, float* lse, void* stream) {
  MZK_CHECK_ARG(B >= 0 && S >= 0 && H >= 1 && nsplit >= 1, "sparse_mqa_combine: bad sizes");
  const int64_t rows = B * S;
  if (rows == 0) return MZK_OK;
  MZK_CHECK_ARG(workspace && out && lse, "sparse_mqa_combine: null pointer");
  const float* po = workspace;
  const float* pml = workspace + rows * nsplit * static_cast<int64_t>(H) * D;
  uint16_t* o = static_cast<uint16_t*>(out);
  hipStream_t s = as_stream(stream);
  switch (D) {
    case 64: launch_combine<64>(po, pml, nsplit, H, S, sinks, o, lse, rows, s); break;
    case 96: launch_combine<96>(po, pml, nsplit, H, S, sinks, o, lse, rows, s); break;
    case 128: launch_combine<128>(po, pml, nsplit, H, S, sinks, o, lse, rows, s); break;
    case 160: launch_combine<160>(po, pml, nsplit, H, S, sinks, o, lse, rows, s); break;
    case 256: launch_combine<256>(po, pml, nsplit, H, S, sinks, o, lse, rows, s); break;
    case 576: launch_combine<576>(po, pml, nsplit, H, S, sinks, o, lse, rows, s); break;
    default: set_last_error("sparse_mqa_combine: unsupported head dim %d", D); return MZK_EUNSUPPORTED;
  }
  MZK_LAUNCH_CHECK("sparse_mqa_combine");
  return MZK_OK;
}

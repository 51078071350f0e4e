// Product-key sub-key scoring, per-half top-k and cartesian top-k, gfx950.
//
// For every (token t, head h):
//   s_c[i] = score(q[t, h, c*half:(c+1)*half], keys[(2h+c)*n + i, :])   c = 0, 1; i < n
//            score = dot product, or idw: -log(1e-3 + max(|q|^2 + |k|^2 - 2<q,k>, 0))
//   (v_c, i_c) = top-knn of s_c, sorted best first
//   cand[a, b] = v_0[a] + v_1[b],  id = i_0[a] * n + i_1[b]
//   (scores, ids) = top-knn of cand, sorted best first
// Reference: HashingMemory.get_indices (pkm/memory.py:250-289) and
// FastWeightProductKeyMemory.get_indices / compute_qk_scores (fwpkm/fwpkm.py:853-934).
// Rounding follows the reference's tensors: sub-scores are stored in the
// input dtype (a bf16 einsum output), the cartesian sums are rounded to it
// again (bf16 + bf16 in ATen), and top-k selects on the rounded values.
// Equal values are ordered by the smaller index (sub-key index, then flat
// a*knn + b), an order the reference's topk leaves unspecified.
//
// Selection works on unique keys: (order-preserving bits of the rounded value
// << index bits) | (inverted index), so "larger key" is "better", ties
// included, and a rank is a count of larger keys.
//
// One workgroup (8 waves) owns TM tokens of one head; per half:
//   A. The half of the TM queries is staged in LDS. Each wave streams its own
//      1/8 of the key tiles from L2 (16-byte loads two k-steps ahead, keys
//      read once per workgroup) and computes [TM x 16] score tiles on MFMA
//      (16x16x32 bf16 / 16x16x4 f32); the epilogue writes the order keys of
//      the rounded scores into the LDS score tile [TM][n], each row laid out
//      so that the columns g, g + G, g + 2G, ... (one threshold group) are
//      adjacent (a 16-byte chunk for n >= 1024).
//   B. Each row is selected by a group of LPR = 512 / TM lanes, all rows at
//      once: T0 = the knn-th largest chunk maximum (a bit search with DPP
//      group sums) is a lower bound of the knn-th largest score, since knn
//      disjoint chunks each hold a score >= T0; the scores >= T0 (about 1.1
//      knn of them on random data) are compacted with a group prefix sum and
//      ranked by counting. More candidates than the row's buffer holds (e.g.
//      many equal scores) leave the row to an exact bit search by its wave.
//   C. (after the second half) per token and lane group, the cartesian
//      candidates are the pairs (a+1)(b+1) <= knn, every other pair being
//      preceded, in (value, flat index) order, by at least knn of them. The
//      knn-th pair value is found by a bit search between the bound given by
//      the pairs (a, 0) and (0, b) and the best pair, and the pairs reaching
//      it are ranked. With bf16 scores (32-bit keys) the two lists are stored
//      as the low and high words of the index output and C runs as its own
//      kernel at full occupancy; with float32 scores it follows B in LDS.
// Workgroups map head-fastest onto the grid, so with 8 heads each XCD (and its
// L2) serves one head's keys.
#include <atomic>
#include <type_traits>
#include <utility>

#include "pkm_common.h"

namespace pkm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxN = 2048;       // n_keys limit
constexpr int kCandCap = 128;     // candidates ranked per row before the exact fallback
constexpr int kMaxLds = 160 * 1024;

// ---------------------------------------------------------------------------
// Order keys: monotone maps of the stored score bits to unsigned integers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t okey16(uint32_t b) { return b ^ ((b & 0x8000u) ? 0xFFFFu : 0x8000u); }
__device__ __forceinline__ uint32_t okey16_inv(uint32_t k) { return k ^ ((k & 0x8000u) ? 0x8000u : 0xFFFFu); }
// okey16 of both halves of a word: the sign of each half (arithmetic shift)
// selects its mask 0xFFFF or 0x8000
typedef short i16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t okey16x2(uint32_t b) {
  const uint32_t sgn = __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2_t, b) >> (short)15);
  return b ^ ((sgn & 0x7FFF7FFFu) | 0x80008000u);
}
__device__ __forceinline__ uint32_t okey32(uint32_t b) {
  return b ^ ((b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}
__device__ __forceinline__ uint32_t okey32_inv(uint32_t k) {
  return k ^ ((k & 0x80000000u) ? 0x80000000u : 0xFFFFFFFFu);
}

// Per score type: score-tile element (an order key), unique selection key,
// MFMA step.
template <typename TIN>
struct Sel;

template <>
struct Sel<bf16_t> {
  typedef uint16_t Store;  // order key of the bf16 score
  typedef uint32_t Key;    // (order key << 16) | (0xFFFF - index)
  static constexpr int KSTEP = 32;  // k per 16-byte fragment: one 16x16x32 MFMA
  static __device__ __forceinline__ uint32_t okey_of(float v) { return okey16(f32_to_bf16_bits(v + 0.0f)); }
  static __device__ __forceinline__ Key make(uint32_t ok, uint32_t idx) { return (ok << 16) | (0xFFFFu - idx); }
  static __device__ __forceinline__ uint32_t key_okey(Key k) { return k >> 16; }
  static __device__ __forceinline__ uint32_t key_idx(Key k) { return 0xFFFFu - (k & 0xFFFFu); }
  static __device__ __forceinline__ float value(uint32_t ok) { return bf16_to_f32(okey16_inv(ok)); }
  static __device__ __forceinline__ void put(bf16_t* p, int64_t i, uint32_t ok) { p[i].x = (uint16_t)okey16_inv(ok); }
    static __device__ __forceinline__ void mma(const uint4& a, const uint4& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                0, 0, 0);
  }
  static __device__ __forceinline__ float sumsq(const uint4& a) {
    float f[8];
    VecTraits<bf16_t>::unpack(a, f);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = __builtin_fmaf(f[e], f[e], s);
    return s;
  }
};

template <>
struct Sel<float> {
  typedef uint32_t Store;  // order key of the float32 score
  typedef uint64_t Key;    // (order key << 32) | (0xFFFFFFFF - index)
  static constexpr int KSTEP = 16;  // k per 16-byte fragment: four 16x16x4 MFMAs
  static __device__ __forceinline__ uint32_t okey_of(float v) { return okey32(__float_as_uint(v + 0.0f)); }
  static __device__ __forceinline__ Key make(uint32_t ok, uint32_t idx) {
    return ((uint64_t)ok << 32) | (uint64_t)(0xFFFFFFFFu - idx);
  }
  static __device__ __forceinline__ uint32_t key_okey(Key k) { return (uint32_t)(k >> 32); }
  static __device__ __forceinline__ uint32_t key_idx(Key k) { return 0xFFFFFFFFu - (uint32_t)k; }
  static __device__ __forceinline__ float value(uint32_t ok) { return __uint_as_float(okey32_inv(ok)); }
  static __device__ __forceinline__ void put(float* p, int64_t i, uint32_t ok) { p[i] = __uint_as_float(okey32_inv(ok)); }
  // The 16 k values of a fragment pair: lane group g holds k = 4g + s in
  // step s, for A and B alike (a permutation of the summation order).
  static __device__ __forceinline__ void mma(const uint4& a, const uint4& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float sumsq(const uint4& a) {
    float s = __uint_as_float(a.x) * __uint_as_float(a.x);
    s = __builtin_fmaf(__uint_as_float(a.y), __uint_as_float(a.y), s);
    s = __builtin_fmaf(__uint_as_float(a.z), __uint_as_float(a.z), s);
    return __builtin_fmaf(__uint_as_float(a.w), __uint_as_float(a.w), s);
  }
};

// ---------------------------------------------------------------------------
// Wave-level selection on unique keys (larger = better).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lanes_below_count(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Appends the keys of the lanes with `cand` to scr[total...] (positions
// >= cap are dropped, total still counts them).
template <typename Key>
__device__ __forceinline__ void wave_append(bool cand, Key key, Key* scr, uint32_t& total) {
  const uint64_t m = __ballot(cand);
  if (m) {
    const uint32_t pos = total + lanes_below_count(m);
    if (cand && pos < (uint32_t)kCandCap) scr[pos] = key;
    total += (uint32_t)__popcll(m);
  }
}

// Best-first top-knn of the total (knn <= total <= kCandCap) unique keys in
// scr, by counting for each key the keys above it. Returns lane j's rank-j
// key (lanes >= knn: 0); scr is reused as the output list.
template <typename Key>
__device__ __forceinline__ Key rank_select(Key* scr, uint32_t total, int knn) {
  const int lane = threadIdx.x & 63;
  const Key k0 = lane < (int)total ? scr[lane] : (Key)0;
  const Key k1 = lane + 64 < (int)total ? scr[lane + 64] : (Key)0;
  uint32_t r0 = 0, r1 = 0;
  constexpr int PER16 = 16 / (int)sizeof(Key);
  const uint32_t full = total & ~(uint32_t)(PER16 - 1);
  if (total <= 64u) {
    for (uint32_t j = 0; j < full; j += PER16) {
      const uint4 q = *(const uint4*)(scr + j);
      const Key* kq = (const Key*)&q;
#pragma unroll
      for (int i = 0; i < PER16; ++i) r0 += kq[i] > k0 ? 1u : 0u;
    }
    for (uint32_t j = full; j < total; ++j) r0 += scr[j] > k0 ? 1u : 0u;
  } else {
    for (uint32_t j = 0; j < full; j += PER16) {
      const uint4 q = *(const uint4*)(scr + j);
      const Key* kq = (const Key*)&q;
#pragma unroll
      for (int i = 0; i < PER16; ++i) {
        r0 += kq[i] > k0 ? 1u : 0u;
        r1 += kq[i] > k1 ? 1u : 0u;
      }
    }
    for (uint32_t j = full; j < total; ++j) {
      r0 += scr[j] > k0 ? 1u : 0u;
      r1 += scr[j] > k1 ? 1u : 0u;
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < (int)total && r0 < (uint32_t)knn) scr[r0] = k0;
  if (lane + 64 < (int)total && r1 < (uint32_t)knn) scr[r1] = k1;
  __builtin_amdgcn_wave_barrier();
  const Key out = lane < knn ? scr[lane] : (Key)0;
  __builtin_amdgcn_wave_barrier();
  return out;
}

// Exact best-first top-knn of the nonzero keys produced by key_at(slot) for
// slot < nslots (at least knn of them): bit-by-bit threshold search with wave
// ballots, then compaction and ranking. The path for inputs whose cheap
// thresholds leave more than kCandCap candidates (e.g. many equal scores).
template <typename Key, typename F>
__device__ __attribute__((noinline)) Key exact_topk(F key_at, int nslots, int knn, Key* scr) {
  constexpr int BITS = 8 * (int)sizeof(Key);
  const int lane = threadIdx.x & 63;
  const int nv = (nslots + 63) / 64;
  Key T = 0;
  for (int bit = BITS - 1; bit >= 0; --bit) {
    const Key trial = T | ((Key)1 << bit);
    uint32_t c = 0;
    for (int v = 0; v < nv; ++v) {
      const int slot = 64 * v + lane;
      const Key k = slot < nslots ? key_at(slot) : (Key)0;
      c += (uint32_t)__popcll(__ballot(k >= trial));
    }
    if (c >= (uint32_t)knn) {
      T = trial;
      if (c == (uint32_t)knn) break;  // {keys >= T} is exactly the top-knn
    }
  }
  uint32_t total = 0;
  for (int v = 0; v < nv; ++v) {
    const int slot = 64 * v + lane;
    const Key k = slot < nslots ? key_at(slot) : (Key)0;
    wave_append(k >= T && k != 0, k, scr, total);
  }
  __builtin_amdgcn_wave_barrier();
  return rank_select(scr, total, knn);
}

// ---------------------------------------------------------------------------
// Score-tile layout. A row holds the n order keys of one (token, half); the
// scores of the columns c = j * G + g (j < slots) form group g and sit next
// to each other, at positions g * slots + ((j + rho) mod slots), where
// slots = min(8, n / 128) (a power of two, at least 1), G = n / slots, and
// rho = 2 * ((row >> 2) & 3) mod slots spreads the four rows an MFMA
// epilogue store writes at once over different LDS banks.
// ---------------------------------------------------------------------------
struct TileMap {
  int slots, lslots, G;
};
__host__ __device__ inline TileMap tile_map(int n) {
  TileMap m;
  m.lslots = 0;
  while (m.lslots < 3 && (128 << m.lslots) <= n) ++m.lslots;
  if (n < 128) m.lslots = 0;
  m.slots = 1 << m.lslots;
  m.G = n >> m.lslots;
  return m;
}
__device__ __forceinline__ int tile_rho(const TileMap& m, int row) { return (2 * ((row >> 2) & 3)) & (m.slots - 1); }
__device__ __forceinline__ int tile_pos(const TileMap& m, int row, int col) {
  const int j = col / m.G, g = col - j * m.G;
  return g * m.slots + ((j + tile_rho(m, row)) & (m.slots - 1));
}
__device__ __forceinline__ int tile_col(const TileMap& m, int row, int pos) {
  const int g = pos >> m.lslots, q = pos & (m.slots - 1);
  return ((q - tile_rho(m, row)) & (m.slots - 1)) * m.G + g;
}

// exact_topk over one row of the score tile, for rows whose cheap threshold
// leaves more than kCandCap candidates (e.g. many equal scores): the row's keys
// are built once, position by position (the column of a position needs no
// division), and held in registers (NV per lane, n <= 64 NV) through the
// threshold search.
template <typename SLT, int NV>
__device__ __attribute__((noinline)) typename SLT::Key exact_topk_row(const typename SLT::Store* Srow, TileMap M,
                                                                      int row, int n, int knn,
                                                                      typename SLT::Key* scr) {
  typedef typename SLT::Key Key;
  constexpr int BITS = 8 * (int)sizeof(Key);
  const int lane = threadIdx.x & 63;
  Key kr[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int p = 64 * v + lane;
    kr[v] = p < n ? SLT::make(Srow[p], (uint32_t)tile_col(M, row, p)) : (Key)0;
  }
  Key T = 0;
  for (int bit = BITS - 1; bit >= 0; --bit) {
    const Key trial = T | ((Key)1 << bit);
    uint32_t c = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) c += (uint32_t)__popcll(__ballot(kr[v] >= trial));
    if (c >= (uint32_t)knn) {
      T = trial;
      if (c == (uint32_t)knn) break;  // {keys >= T} is exactly the top-knn
    }
  }
  uint32_t total = 0;
#pragma unroll
  for (int v = 0; v < NV; ++v) wave_append(kr[v] >= T && kr[v] != 0, kr[v], scr, total);
  __builtin_amdgcn_wave_barrier();
  return rank_select(scr, total, knn);
}

// ---------------------------------------------------------------------------
// LDS layout (host and device agree through score_lds_layout).
//   S: score tile [TM][n] of order keys; after the second half's selection it
//      holds the first half's lists [TM][KL] and the cartesian results [TM][KL].
//   R: query stage [TM][half] in phase A; per-row candidate buffers [TM][CAP]
//      and top-knn lists [TM][KL] in phases B and C.
// ---------------------------------------------------------------------------
constexpr int kMaxPairs = 280;  // candidate pairs (a+1)(b+1) <= knn for knn = 64

// The candidate pairs of the cartesian step for every knn <= 64: slot s of
// knn is ab[off[knn] + s] = a | b << 8, in a-major order, b ascending, over
// the pairs (a+1)(b+1) <= knn (so slot order is the flat a * knn + b order).
constexpr int pair_count(int knn) {
  int c = 0;
  for (int a = 0; a < knn; ++a) c += knn / (a + 1);
  return c;
}
constexpr int pair_table_size() {
  int c = 0;
  for (int k = 1; k <= 64; ++k) c += pair_count(k);
  return c;
}
struct PairTable {
  int off[66];
  uint16_t ab[pair_table_size()];
};
constexpr PairTable make_pair_table() {
  PairTable t{};
  int o = 0;
  for (int k = 1; k <= 64; ++k) {
    t.off[k] = o;
    for (int a = 0; a < k; ++a)
      for (int b = 0; b < k / (a + 1); ++b) t.ab[o++] = (uint16_t)(a | (b << 8));
  }
  t.off[65] = o;
  return t;
}
__constant__ PairTable kPairTable = make_pair_table();
struct ScoreLds {
  int s_bytes, r_bytes, cap, cstride, kl, cand_off, list_off, total;
};

// Largest n_keys a TM-token tile serves: the tile fits the LDS, and a lane of
// the selection holds at most 64 words of its row.
__host__ __device__ constexpr int score_max_n(int TM, int esz) {
  return (kMaxLds / (TM * esz) < kMaxN ? kMaxLds / (TM * esz) : kMaxN) < 64 * (kThreads / TM) * (4 / esz)
             ? (kMaxLds / (TM * esz) < kMaxN ? kMaxLds / (TM * esz) : kMaxN) & ~63
             : 64 * (kThreads / TM) * (4 / esz);
}

__host__ __device__ inline int score_cap(int knn, int lpr) {
  int c = 2 * knn;
  const int fb = kCandCap * lpr / 64;  // a wave's candidate buffers double as its fallback scratch
  c = c > fb ? c : fb;
  return (c + 3) & ~3;
}

__host__ __device__ inline ScoreLds score_lds_layout(int TM, int n, int half, int knn, int esz, int key_bytes) {
  ScoreLds L;
  const int lpr = kThreads / TM;
  L.cap = score_cap(knn, lpr);
  L.cstride = L.cap + 4;  // 4 zero keys after the last candidate
  L.kl = (knn + 3) & ~3;
  const int tile = TM * n * esz;
  const int c_bytes = 2 * TM * L.kl * key_bytes;
  L.s_bytes = ((tile > c_bytes ? tile : c_bytes) + 15) & ~15;
  const int q_bytes = TM * half * (esz == 2 ? 2 : 4);
  L.cand_off = 0;
  L.list_off = TM * L.cstride * key_bytes;
  const int sel_bytes = L.list_off + TM * L.kl * key_bytes;
  L.r_bytes = ((q_bytes > sel_bytes ? q_bytes : sel_bytes) + 15) & ~15;
  L.total = L.s_bytes + L.r_bytes;
  return L;
}

// ---------------------------------------------------------------------------
// Lane groups: LPR consecutive lanes (8, 16 or 32, aligned) own one row.
// Sums and scans over a group with DPP.
// ---------------------------------------------------------------------------
template <int LPR>
__device__ __forceinline__ uint32_t group_sum(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  x += (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  if (LPR >= 8) x += (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xF, 0xF, false);   // row_half_mirror
  if (LPR >= 16) x += (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x140, 0xF, 0xF, false);  // row_mirror
  if (LPR >= 32) x += (uint32_t)__shfl_xor((int)x, 16);
  return x;
}
// inclusive prefix sum over the group (sub = lane index inside the group)
template <int LPR>
__device__ __forceinline__ uint32_t group_scan(uint32_t x, int sub) {
  uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += sub >= 1 ? y : 0u;
  y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += sub >= 2 ? y : 0u;
  if (LPR >= 8) {
    y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += sub >= 4 ? y : 0u;
  }
  if (LPR >= 16) {
    y = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, false);  // row_shr:8
    x += sub >= 8 ? y : 0u;
  }
  if (LPR >= 32) {  // add the first 16 lanes' total (their last lane's prefix)
    y = (uint32_t)__shfl((int)x, (int)(threadIdx.x & 32) + 15);
    x += sub >= 16 ? y : 0u;
  }
  return x;
}

// Whether fewer than knn of the group's values v[0, NV) (all lanes) reach
// trial. Values of B <= 16 bits are counted without compares: v - trial
// wraps to a set top bit exactly when v < trial.
template <int LPR, int NV, int B>
__device__ __forceinline__ bool group_count_ge_below(const uint32_t* v, uint32_t trial, int knn) {
  uint32_t c = 0;
  if (B <= 16) {
    uint32_t below = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) below += (v[i] - trial) >> 31;
    c = (uint32_t)NV - below;
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i) c += v[i] >= trial ? 1u : 0u;
  }
  return group_sum<LPR>(c) < (uint32_t)knn;
}

// Best-first top-knn of the C (knn <= C <= LPR * MAXM) unique keys cand[0, C)
// of one row, by its lane group: each lane counts, for its keys
// cand[sub + LPR i], the keys above them, and emit(rank, key) is called for
// the ranks below knn. cand[C, C + 4) must read as 0 (below every key).
template <typename Key, int LPR, int MAXM, typename F>
__device__ __forceinline__ void group_rank(const Key* cand, uint32_t C, int knn, int sub, F emit) {
  Key mine[MAXM];
  uint32_t rk[MAXM];
#pragma unroll
  for (int i = 0; i < MAXM; ++i) {
    const uint32_t j = (uint32_t)(sub + LPR * i);
    mine[i] = j < C ? cand[j] : (Key)0;
    rk[i] = 0;
  }
  constexpr int PER16 = 16 / (int)sizeof(Key);
  uint4 q = *(const uint4*)cand;  // 16 bytes ahead of their use
  for (uint32_t j = 0; j < C; j += PER16) {
    const uint4 qn = *(const uint4*)(cand + (j + PER16 < C ? j + PER16 : j));
    const Key* kq = (const Key*)&q;
#pragma unroll
    for (int u = 0; u < PER16; ++u)
#pragma unroll
      for (int i = 0; i < MAXM; ++i) rk[i] += kq[u] > mine[i] ? 1u : 0u;
    q = qn;
  }
#pragma unroll
  for (int i = 0; i < MAXM; ++i)
    if (mine[i] != 0 && rk[i] < (uint32_t)knn) emit(rk[i], mine[i]);
}

// ---------------------------------------------------------------------------
// C: cartesian top-knn of one row per lane group, over the pairs
// (a+1)(b+1) <= knn (every other pair is preceded, in (value, flat index)
// order, by at least knn of them): T = the knn-th largest pair value, by a bit
// search between a lower bound and the best pair, then the pairs >= T are
// ranked. l0r / l1r: the row's two lists (best first), cand: its candidate
// buffer (cap + 4 keys), finr: the ranked pair-slot keys out. Rows whose
// candidates overflow cap are redone exactly by their wave, one at a time,
// with wscr as scratch; rows(rr) gives the (l0, l1, fin) lists of the wave's
// row rr for that. Rows with active = false select nothing.
// ---------------------------------------------------------------------------
template <typename Key>
struct CartRow {
  const Key* l0;
  const Key* l1;
  Key* fin;
};

template <typename TIN, int LPR, int MAXM, int MAXS, typename RowsF>
__device__ __forceinline__ void cartesian_rows(const typename Sel<TIN>::Key* l0r, const typename Sel<TIN>::Key* l1r,
                                               typename Sel<TIN>::Key* cand, typename Sel<TIN>::Key* finr, int cap,
                                               int knn, int sub, bool active, typename Sel<TIN>::Key* wscr,
                                               RowsF rows) {
  typedef Sel<TIN> SL;
  typedef typename SL::Key Key;
  constexpr int KBITS = 8 * (int)sizeof(typename SL::Store);
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const uint16_t* pairs = kPairTable.ab + kPairTable.off[knn];
  const int npairs = kPairTable.off[knn + 1] - kPairTable.off[knn];
  // value (order key) of pair slot s; candidates are keyed by the slot,
  // whose order is the flat a * knn + b order
  auto pair_okey = [&](const Key* a, const Key* b, int s) -> uint32_t {
    const uint32_t ab = pairs[s];
    return SL::okey_of(SL::value(SL::key_okey(a[ab & 0xFFu])) + SL::value(SL::key_okey(b[ab >> 8])));
  };
  // the knn-th pair value lies between the knn-th of the pairs (a, 0) or
  // (0, b) and the best pair; bits above their highest difference are shared
  uint32_t Tlo, Thi;
  {
    const float v0 = SL::value(SL::key_okey(l0r[0]));
    const float w0 = SL::value(SL::key_okey(l1r[0]));
    const uint32_t ta = SL::okey_of(SL::value(SL::key_okey(l0r[knn - 1])) + w0);
    const uint32_t tb = SL::okey_of(v0 + SL::value(SL::key_okey(l1r[knn - 1])));
    Tlo = ta > tb ? ta : tb;
    Thi = SL::okey_of(v0 + w0);
  }
  // pair values of this lane's slots sub + LPR i (0 past the last), the
  // threshold T, and the compaction of the pairs >= T; NS = slots per lane
  auto cartesian = [&](auto ns_tag, uint32_t& ctotal_out) -> bool {
    constexpr int NS = decltype(ns_tag)::value;
    uint32_t cv[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int s = sub + LPR * i;
      cv[i] = s < npairs ? pair_okey(l0r, l1r, s) : 0u;
    }
    const uint32_t d = Tlo ^ Thi;
    const int hb = d == 0 ? -1 : 31 - __builtin_clz(d);
    uint32_t T = hb < 0 ? Tlo : (Thi & ~((2u << hb) - 1u));
    for (int bit = hb; bit >= 0; --bit) {
      const uint32_t trial = T | (1u << bit);
      if (!group_count_ge_below<LPR, NS, KBITS>(cv, trial, knn)) T = trial;
    }
    T = T > 0u ? T : 1u;
    uint32_t ccnt = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) ccnt += cv[i] >= T ? 1u : 0u;
    const uint32_t cincl = group_scan<LPR>(ccnt, sub);
    const uint32_t ctotal = group_sum<LPR>(ccnt);
    ctotal_out = ctotal;
    const bool ov = ctotal > (uint32_t)cap;
    if (!ov) {
      uint32_t p = cincl - ccnt;
#pragma unroll
      for (int i = 0; i < NS; ++i)
        if (cv[i] >= T) cand[p++] = SL::make(cv[i], (uint32_t)(sub + LPR * i));
      if (sub == 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) cand[ctotal + u] = (Key)0;
      }
    }
    return ov;
  };
  uint32_t ctotal = 0;
  bool coverflow;
  if (npairs <= LPR * ((pair_count(16) + LPR - 1) / LPR))
    coverflow = cartesian(std::integral_constant<int, (pair_count(16) + LPR - 1) / LPR>(), ctotal);
  else if (npairs <= LPR * ((pair_count(32) + LPR - 1) / LPR))
    coverflow = cartesian(std::integral_constant<int, (pair_count(32) + LPR - 1) / LPR>(), ctotal);
  else
    coverflow = cartesian(std::integral_constant<int, MAXS>(), ctotal);
  coverflow = coverflow && active;
  __builtin_amdgcn_wave_barrier();
  auto to_fin = [&](uint32_t rank, Key k) { finr[rank] = k; };
  if (!coverflow && active) {
    if (cap <= 8 * LPR)
      group_rank<Key, LPR, 8>(cand, ctotal, knn, sub, to_fin);
    else
      group_rank<Key, LPR, MAXM>(cand, ctotal, knn, sub, to_fin);
  }
  __builtin_amdgcn_wave_barrier();
  {
    const uint64_t ov = __ballot(coverflow);
    for (int rr = 0; rr < RPW; ++rr) {
      if (!((ov >> (rr * LPR)) & 1ull)) continue;
      const CartRow<Key> row = rows(rr);
      const Key top = exact_topk<Key>(
          [&](int s) -> Key { return s < npairs ? SL::make(pair_okey(row.l0, row.l1, s), (uint32_t)s) : (Key)0; },
          npairs, knn, wscr);
      if (lane < knn) row.fin[lane] = top;
      __builtin_amdgcn_wave_barrier();
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <typename TIN, int IDW, int TM, int KSC>
__global__ __launch_bounds__(kThreads) void pkm_score_topk_kernel(
    const TIN* __restrict__ Q, const TIN* __restrict__ Kt, int kpack, int64_t Ntok, int H, int n, int half, int knn,
    TIN* __restrict__ out_scores, int64_t* __restrict__ out_idx, int64_t* __restrict__ out_i1,
    int64_t* __restrict__ out_i2, TIN* __restrict__ out_s1, TIN* __restrict__ out_s2) {
  typedef Sel<TIN> SL;
  typedef typename SL::Store Store;
  typedef typename SL::Key Key;
  constexpr int RT = TM / 16;  // row tiles
  constexpr int CB = 4;        // column tiles per batch
  constexpr int ESZ = (int)sizeof(TIN);
  constexpr int EPC = 16 / ESZ;  // input elements per 16-byte chunk
  constexpr int LPR = kThreads / TM;  // lanes per row in the selection phases
  constexpr int RPW = 64 / LPR;       // rows per wave
  constexpr int EPW = 4 / (int)sizeof(Store);  // score-tile elements per 32-bit word
  constexpr int MAXG = score_max_n(TM, (int)sizeof(Store)) / LPR / EPW / 4;  // 16-byte chunks of a row per lane
  constexpr int KBITS = 8 * (int)sizeof(Store);                          // bits of an order key
  constexpr int MAXM = (2 * 64 > kCandCap * LPR / 64 ? 2 * 64 : kCandCap * LPR / 64) / LPR;  // cap / LPR
  constexpr int MAXS = (kMaxPairs + LPR - 1) / LPR;  // pair slots per lane
  // 32-bit keys (bf16 scores): both lists fit one index word and the
  // cartesian step runs as its own kernel (pkm_score_cartesian_kernel)
  constexpr bool kSplitC = sizeof(Key) == 4;
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = (int)(blockIdx.x % (unsigned)H);
  const int64_t t0 = (int64_t)(blockIdx.x / (unsigned)H) * TM;
  const ScoreLds L = score_lds_layout(TM, n, half, knn, (int)sizeof(Store), (int)sizeof(Key));
  const TileMap M = tile_map(n);
  Store* S = (Store*)smem;
  unsigned char* R = smem + L.s_bytes;
  uint4* QS = (uint4*)R;  // phase A: query stage

  // selection: row r = this lane's group, sub = lane inside the group
  const int r = threadIdx.x / LPR;
  const int sub = threadIdx.x & (LPR - 1);
  Key* cand = (Key*)(R + L.cand_off) + r * L.cstride;
  Key* list = (Key*)(R + L.list_off) + r * L.kl;
  Key* l0 = (Key*)smem + r * L.kl;             // phase C: the first half's list, in the free tile,
  Key* fin = (Key*)smem + (TM + r) * L.kl;     // and the ranked pairs
  const uint16_t* pairs = kPairTable.ab + kPairTable.off[knn];
  const int64_t t = t0 + r;
  const bool live = t < Ntok;
  const int64_t th = t * H + h;
  const int64_t orow = th * knn;

  const int kdim = 2 * half;
  const int CH = half / EPC;  // 16-byte chunks per query half row (4 per k-step)
  const int KS = half / SL::KSTEP;
  // Query stage layout, in 16-byte chunks: chunk c = 4 j + g of row q (the
  // g-th quarter of k-step j) sits at (j * TM + q) * 4 + (g ^ ((q >> 2) & 3)),
  // so the A fragment of a k-step is one lane-invariant offset away from a
  // per-lane base, and the 8 lanes an LDS cycle serves hit distinct banks.
  const int qlane = (lane & 15) * 4 + ((lane >> 4) ^ ((lane >> 2) & 3));
  // key chunk of lane (column lane & 15, quarter lane >> 4) inside a tile row
  // block, and the chunk stride of a k-step: row-major keys, or tiles packed
  // chunk-major by score_keys_pack_kernel (a k-step's operands one contiguous KB)
  const int klane = kpack ? lane : (lane & 15) * CH + (lane >> 4);
  const int kss = kpack ? 64 : 4;
  const int ncol = n / 16;
  // this wave's column tiles are w, w + 8, ...; batches of CB of them
  const int ntw = (ncol - w + kWaves - 1) / kWaves;
  const int nsteps = ((ntw + CB - 1) / CB) * KS;


  // A tile row is read as 16-byte chunks interleaved over the lane group:
  // lane sub reads chunks LPR (i ^ x) + sub, i < NG, with x = row & 1 when
  // LPR = 8 so that the two rows an LDS pass serves use different banks. Each
  // chunk is one group of the threshold (n / (4 EPW) groups per row).
  const int NCH = n / (4 * EPW);  // chunks per row
  const int NG = (NCH + LPR - 1) / LPR;
  const int cx = (LPR == 8 && NCH % (2 * LPR) == 0) ? (r & 1) : 0;

#pragma unroll 1
  for (int hc = 0; hc < 2; ++hc) {
    const TIN* Kc = Kt + (int64_t)(2 * h + hc) * n * half;
    // ---- A0: stage the query half [TM][half] (zeros past the last token)
    if constexpr (KSC > 0 && (TM * 4 * KSC) % kThreads == 0) {
      // compile-time trip count (CH = 4 KSC chunks per row): every load is
      // in flight before the first store
      constexpr int CHC = 4 * KSC;
      constexpr int NI = TM * CHC / kThreads;
      uint4 v[NI];
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int i = (int)threadIdx.x + j * kThreads;
        const int q = i / CHC, c = i % CHC;
        const int64_t tq = t0 + q;
        v[j] = make_uint4(0u, 0u, 0u, 0u);
        if (tq < Ntok) v[j] = ld16(Q + (tq * H + h) * kdim + hc * half + c * EPC);
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int i = (int)threadIdx.x + j * kThreads;
        const int q = i / CHC, c = i % CHC;
        QS[((c >> 2) * TM + q) * 4 + ((c & 3) ^ ((q >> 2) & 3))] = v[j];
      }
    } else {
      for (int i = threadIdx.x; i < TM * CH; i += kThreads) {
        const int q = i / CH, c = i - (i / CH) * CH;
        const int64_t tq = t0 + q;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (tq < Ntok) v = ld16(Q + (tq * H + h) * kdim + hc * half + c * EPC);
        QS[((c >> 2) * TM + q) * 4 + ((c & 3) ^ ((q >> 2) & 3))] = v;
      }
    }
    __syncthreads();

    // ---- A: scores of this wave's column tiles, one step = one k-step of a
    // batch of CB tiles. The keys of step s + 2 (from L2) are loaded while
    // step s runs, in a ring of 3 register slots continued across batch
    // boundaries, so the loads of the next batch overlap the epilogue of the
    // current one; the queries of a step come from LDS at its start.
    float qn[RT];  // idw: squared norm of query row rt*16 + (lane & 15)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float s = 0.f;
      if (IDW) {
        for (int j = 0; j < KS; ++j) s += SL::sumsq(QS[(j * TM + rt * 16) * 4 + qlane]);
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
      }
      qn[rt] = s;
    }
    f32x4_t acc[RT][CB];
    float kn[CB];
    auto reset = [&]() {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int k = 0; k < CB; ++k) acc[rt][k] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < CB; ++k) kn[k] = 0.f;
    };
    // operands of k-step ks of batch jb (ks may run past the batch into the
    // next one; steps past the last read step 0's, in range, unused); tiles
    // past the last one read tile 0 and their scores are dropped
    const uint4* Kc4 = (const uint4*)Kc;
    const int nbw = nsteps / KS;
    auto load_b = [&](uint4* b, int jb, int ks) {
      if (ks >= KS) ks -= KS, ++jb;
      if (jb >= nbw) jb = 0, ks = 0;
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        const int tile = w + kWaves * (CB * jb + k);
        const int tl = tile < ncol ? tile : 0;
        b[k] = (Kc4 + (16 * tl * CH + kss * ks))[klane];
      }
    };
    auto load_a = [&](uint4* a, int ks) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) a[rt] = QS[(ks * TM + rt * 16) * 4 + qlane];
    };
    auto mma = [&](const uint4* a, const uint4* b) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int k = 0; k < CB; ++k) SL::mma(a[rt], b[k], acc[rt][k]);
      if (IDW) {
#pragma unroll
        for (int k = 0; k < CB; ++k) kn[k] += SL::sumsq(b[k]);
      }
    };
    // epilogue of batch jb: order keys of the rounded scores into the tile
    // (lane: rows rt*16 + 4 (lane >> 4) + e, column 16 tile + (lane & 15))
    auto epilogue = [&](int jb) {
      if (IDW) {
#pragma unroll
        for (int k = 0; k < CB; ++k) {
          kn[k] += __shfl_xor(kn[k], 16);
          kn[k] += __shfl_xor(kn[k], 32);  // squared norm of key 16*tile + (lane & 15)
        }
      }
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        const int tile = w + kWaves * (CB * jb + k);
        if (tile >= ncol) continue;
        // the 4 rows 4g + e of a lane share rho, so one position serves them
        const int pos = tile_pos(M, 4 * (lane >> 4), 16 * tile + (lane & 15));
        Store* St = S + 4 * (lane >> 4) * n + pos;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float sc[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float s = acc[rt][k][e];
            if (IDW) {
              float d2 = __shfl(qn[rt], 4 * (lane >> 4) + e) + kn[k] - 2.f * s;
              d2 = d2 > 0.f ? d2 : 0.f;
              s = -logf(1e-3f + d2);
            }
            sc[e] = s;
          }
          if (sizeof(Store) == 2) {
            // two rows per conversion: order keys of a packed bf16 pair
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
              const uint32_t k2 = okey16x2(pack2_bf16(sc[e] + 0.0f, sc[e + 1] + 0.0f));
              St[(rt * 16 + e) * n] = (Store)k2;
              St[(rt * 16 + e + 1) * n] = (Store)(k2 >> 16);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) St[(rt * 16 + e) * n] = (Store)SL::okey_of(sc[e]);
          }
        }
      }
    };
    uint4 a[RT], b0[CB], b1[CB], b2[CB];
    reset();
    load_b(b0, 0, 0);
    load_b(b1, 0, 1);
    __builtin_amdgcn_sched_barrier(0);
    // k-step ks of batch jb runs on the ring slot b and loads the step two
    // ahead into bn
    auto body = [&](int jb, int ks, const uint4* b, uint4* bn) {
      load_a(a, ks);
      load_b(bn, jb, ks + 2);
      __builtin_amdgcn_sched_barrier(0);
      mma(a, b);
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int jb = 0; jb < nbw; ++jb) {
      if (KSC > 0) {
        // compile-time k-steps: one straight run per batch, so the waits
        // before each step cover only that step's loads
#pragma unroll
        for (int ks = 0; ks < KSC; ++ks) {
          if (ks % 3 == 0)
            body(jb, ks, b0, b2);
          else if (ks % 3 == 1)
            body(jb, ks, b1, b0);
          else
            body(jb, ks, b2, b1);
        }
      } else {
        for (int ks = 0; ks < KS; ks += 3) {
          body(jb, ks, b0, b2);
          if (ks + 1 < KS) body(jb, ks + 1, b1, b0);
          if (ks + 2 < KS) body(jb, ks + 2, b2, b1);
        }
      }
      epilogue(jb);
      reset();
      // the next batch's first two steps are in flight in the slots after the
      // last one used: rotate them to b0, b1 (after the epilogue, so the moves
      // rarely wait for the loads)
      const int rot = (KSC > 0 ? KSC : KS) % 3;
      if (rot == 1) {
#pragma unroll
        for (int k = 0; k < CB; ++k) {
          b0[k] = b1[k];
          b1[k] = b2[k];
        }
      } else if (rot == 2) {
#pragma unroll
        for (int k = 0; k < CB; ++k) {
          const uint4 x = b0[k];
          b0[k] = b2[k];
          b1[k] = x;
        }
      }
    }
    __syncthreads();  // score tile complete; the query stage is free
    // the first half's list of this row (parked in the index output), needed in C
    Key park[(64 + LPR - 1) / LPR];
#pragma unroll
    for (int i = 0; i < (64 + LPR - 1) / LPR; ++i) {
      const int j = sub + LPR * i;
      park[i] = (!kSplitC && hc == 1 && live && j < knn) ? (Key)out_idx[orow + j] : (Key)0;
    }

    // ---- sub-score outputs (every key), coalesced over the workgroup
    TIN* out_s = hc == 0 ? out_s1 : out_s2;
    if (out_s != nullptr) {
      for (int i = threadIdx.x; i < TM * n; i += kThreads) {
        const int q = i / n, col = i - (i / n) * n;
        if (t0 + q < Ntok) SL::put(out_s, ((t0 + q) * H + h) * n + col, S[q * n + tile_pos(M, q, col)]);
      }
    }

    // ---- B: top-knn of row r by its lane group.
    // T0 = the knn-th largest group maximum is a lower bound of the knn-th
    // largest score (knn disjoint groups each hold a score >= T0), so the
    // top-knn are among the scores >= T0; they are compacted into cand and
    // ranked. More than cap of them (e.g. many equal scores) leave the row to
    // the exact search of its wave below.
    // chunk i of this lane (zeros past the row)
    const uint32_t* Sw = (const uint32_t*)(S + r * n);
    auto chunk_of = [&](int i) { return LPR * (i ^ cx) + sub; };
    auto load_chunk = [&](int i) -> uint4 {
      const int c = chunk_of(i);
      return c < NCH ? *(const uint4*)(Sw + 4 * c) : make_uint4(0u, 0u, 0u, 0u);
    };
    auto word_max = [&](uint32_t x) -> uint32_t {
      if (EPW == 2) {
        const uint32_t lo = x & 0xFFFFu, hi = x >> 16;
        return lo > hi ? lo : hi;
      }
      return x;
    };
    uint32_t gm[MAXG];
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const uint4 v = g < NG ? load_chunk(g) : make_uint4(0u, 0u, 0u, 0u);
      uint32_t m = word_max(v.x);
      m = word_max(v.y) > m ? word_max(v.y) : m;
      m = word_max(v.z) > m ? word_max(v.z) : m;
      gm[g] = word_max(v.w) > m ? word_max(v.w) : m;
    }
    uint32_t T0 = 0;
    for (int bit = KBITS - 1; bit >= 0; --bit) {
      const uint32_t trial = T0 | (1u << bit);
      if (!group_count_ge_below<LPR, MAXG, KBITS>(gm, trial, knn)) T0 = trial;
    }
    // candidates: elements >= T0, in the chunks whose maximum reaches it
    // (T0 >= 1 when any exist: chunks past the row are 0)
    const uint32_t T0e = T0 > 0u ? T0 : 1u;
    uint32_t act = 0;
#pragma unroll
    for (int g = 0; g < MAXG; ++g) act |= (gm[g] >= T0e ? 1u : 0u) << g;
    uint32_t cnt = 0;
    for (uint32_t m = act; m != 0; m &= m - 1) {
      const uint4 v = load_chunk(__builtin_ctz(m));
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4 * EPW; ++j) {
        const uint32_t x = EPW == 2 ? ((vw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu) : vw[j];
        cnt += x >= T0e ? 1u : 0u;
      }
    }
    const uint32_t incl = group_scan<LPR>(cnt, sub);
    const uint32_t total = group_sum<LPR>(cnt);
    const bool overflow = total > (uint32_t)L.cap;
    if (!overflow) {
      uint32_t p = incl - cnt;
      // column of element j of chunk c: c * (E / slots) + off[j] when a chunk
      // of E elements spans whole groups of slots positions
      constexpr int E = 4 * EPW;
      const bool whole = M.slots <= E;
      int off[E];
#pragma unroll
      for (int j = 0; j < E; ++j) off[j] = tile_col(M, r, j);
      const int cstep = whole ? (E >> M.lslots) : 0;
      for (uint32_t m = act; m != 0; m &= m - 1) {
        const int g = __builtin_ctz(m);
        const uint4 v = load_chunk(g);
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
        const int c = chunk_of(g);
#pragma unroll
        for (int j = 0; j < E; ++j) {
          const uint32_t x = EPW == 2 ? ((vw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu) : vw[j];
          if (x >= T0e) {
            const int col = whole ? c * cstep + off[j] : tile_col(M, r, c * E + j);
            cand[p++] = SL::make(x, (uint32_t)col);
          }
        }
      }
      if (sub == 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) cand[total + u] = (Key)0;
      }
    }
    __builtin_amdgcn_wave_barrier();
    auto to_list = [&](uint32_t rank, Key k) { list[rank] = k; };
    if (!overflow) {
      if (L.cap <= 8 * LPR)
        group_rank<Key, LPR, 8>(cand, total, knn, sub, to_list);
      else
        group_rank<Key, LPR, MAXM>(cand, total, knn, sub, to_list);
    }
    __builtin_amdgcn_wave_barrier();
    // exact search for the rows of this wave that overflowed, one at a time;
    // the wave's candidate buffers are its scratch
    Key* wscr = (Key*)(R + L.cand_off) + (w * RPW) * L.cstride;
    {
      const uint64_t ov = __ballot(overflow);
      for (int rr = 0; rr < RPW; ++rr) {
        if (!((ov >> (rr * LPR)) & 1ull)) continue;
        const int row = w * RPW + rr;
        const Store* Srow = S + row * n;
        const Key best = n <= 512    ? exact_topk_row<SL, 8>(Srow, M, row, n, knn, wscr)
                         : n <= 1024 ? exact_topk_row<SL, 16>(Srow, M, row, n, knn, wscr)
                                     : exact_topk_row<SL, 32>(Srow, M, row, n, knn, wscr);
        if (lane < knn) ((Key*)(R + L.list_off) + row * L.kl)[lane] = best;
        __builtin_amdgcn_wave_barrier();
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (hc == 0) {
      // park the first half's list in the index output until the cartesian step
      if (live) {
        for (int j = sub; j < knn; j += LPR) {
          const Key k = list[j];
          out_idx[orow + j] = (int64_t)k;
          if (out_i1 != nullptr) out_i1[orow + j] = (int64_t)SL::key_idx(k);
        }
      }
      __syncthreads();  // before the next half overwrites the tile and the shared region
      continue;
    }
    if (live && out_i2 != nullptr) {
      for (int j = sub; j < knn; j += LPR) out_i2[orow + j] = (int64_t)SL::key_idx(list[j]);
    }
    if constexpr (kSplitC) {
      // 32-bit keys: the second half's list joins the first in the high words
      // of the index output; the cartesian step runs as its own kernel
      if (live) {
        for (int j = sub; j < knn; j += LPR) ((uint32_t*)(out_idx + orow + j))[1] = (uint32_t)list[j];
      }
      continue;
    } else {
      __syncthreads();  // every row selected: the tile is free for the first half's lists
#pragma unroll
      for (int i = 0; i < (64 + LPR - 1) / LPR; ++i) {
        const int j = sub + LPR * i;
        if (j < knn) l0[j] = park[i];
      }
      __builtin_amdgcn_wave_barrier();  // the first half's list of a row is written and read by its own lanes
      cartesian_rows<TIN, LPR, MAXM, MAXS>(l0, list, cand, fin, L.cap, knn, sub, true, wscr, [&](int rr) {
        const int row = w * RPW + rr;
        return CartRow<Key>{(const Key*)smem + row * L.kl, (const Key*)(R + L.list_off) + row * L.kl,
                            (Key*)smem + (TM + row) * L.kl};
      });
      // outputs: the pair's rounded sum and slot id i_0[a] * n + i_1[b]
      if (live) {
        for (int j = sub; j < knn; j += LPR) {
          const Key k = fin[j];
          const uint32_t ab = pairs[SL::key_idx(k)];
          SL::put(out_scores, orow + j, SL::key_okey(k));
          out_idx[orow + j] = (int64_t)SL::key_idx(l0[ab & 0xFFu]) * n + (int64_t)SL::key_idx(list[ab >> 8]);
        }
      }
    }
  }
}


// C as its own kernel for 32-bit keys: the lists of row i (token, head) are
// the low (first half) and high (second half) words of out_idx[i * knn + j];
// the scores and slot ids replace them. A lane group of LPR lanes per row,
// kThreads / LPR rows per workgroup.
template <typename TIN, int LPR>
__global__ __launch_bounds__(kThreads) void pkm_score_cartesian_kernel(int64_t rows, int n, int knn,
                                                                      TIN* __restrict__ out_scores,
                                                                      int64_t* __restrict__ out_idx) {
  typedef Sel<TIN> SL;
  typedef typename SL::Key Key;
  static_assert(sizeof(Key) == 4, "two lists per index word");
  constexpr int RPB = kThreads / LPR;
  constexpr int RPW = 64 / LPR;
  constexpr int MAXM = (2 * 64 > kCandCap * LPR / 64 ? 2 * 64 : kCandCap * LPR / 64) / LPR;
  constexpr int MAXS = (kMaxPairs + LPR - 1) / LPR;
  extern __shared__ __align__(16) unsigned char smem[];
  const int cap = score_cap(knn, LPR);
  const int cstride = cap + 4;
  const int kl = (knn + 3) & ~3;
  Key* lists = (Key*)smem;               // [RPB][2][kl]
  Key* fins = lists + RPB * 2 * kl;      // [RPB][kl]
  Key* cands = fins + RPB * kl;          // [RPB][cstride]
  const int r = threadIdx.x / LPR;
  const int sub = threadIdx.x & (LPR - 1);
  const int w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * RPB + r;
  const bool live = row < rows;
  const int64_t orow = row * knn;
  Key* l0 = lists + 2 * r * kl;
  Key* l1 = l0 + kl;
  Key* fin = fins + r * kl;
  {
    // every load (knn <= 64) is in flight before the first store
    constexpr int MAXJ = (64 + LPR - 1) / LPR;
    uint64_t v[MAXJ];
#pragma unroll
    for (int i = 0; i < MAXJ; ++i) {
      const int j = sub + LPR * i;
      v[i] = (live && j < knn) ? (uint64_t)out_idx[orow + j] : 0ull;
    }
#pragma unroll
    for (int i = 0; i < MAXJ; ++i) {
      const int j = sub + LPR * i;
      if (j < knn) {
        l0[j] = (Key)(uint32_t)v[i];
        l1[j] = (Key)(uint32_t)(v[i] >> 32);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();  // a row's lists are written and read by its own lanes
  cartesian_rows<TIN, LPR, MAXM, MAXS>(l0, l1, cands + r * cstride, fin, cap, knn, sub, live,
                                       cands + (w * RPW) * cstride, [&](int rr) {
                                         const int rw = w * RPW + rr;
                                         return CartRow<Key>{lists + 2 * rw * kl, lists + (2 * rw + 1) * kl,
                                                             fins + rw * kl};
                                       });
  if (live) {
    const uint16_t* pairs = kPairTable.ab + kPairTable.off[knn];
    for (int j = sub; j < knn; j += LPR) {
      const Key k = fin[j];
      const uint32_t ab = pairs[SL::key_idx(k)];
      SL::put(out_scores, orow + j, SL::key_okey(k));
      out_idx[orow + j] = (int64_t)SL::key_idx(l0[ab & 0xFFu]) * n + (int64_t)SL::key_idx(l1[ab >> 8]);
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming scoring: bfloat16 dot scores, knn <= 32, half key dim 128 or 256.
//
// One workgroup of 8 waves, two per SIMD, owns 256 tokens of one (head, half):
// while one wave of a SIMD runs its selection on the vector ALUs, the other
// wave's MFMAs keep the matrix core busy (a wave does not overlap its own
// vector work with its own MFMAs). The keys of the half stream through LDS in
// blocks of 64 (double-buffered, direct global->LDS loads, every key read once
// per workgroup). A wave multiplies them with its 32 tokens' query halves,
// held in accumulation registers, on 32x32x16 bf16 MFMA: A = 32 keys from LDS
// (read four steps ahead), B = the 32 tokens. In the MFMA's output lane l
// holds 16 scores of token l % 32, keys 8 a + 4 (l / 32) + b (a, b < 4) of
// the 32-key tile: every token has two lanes, l and l + 32, and each selects
// over its own half of the token's keys. A block's 32 scores of a lane are 16
// words of two bf16.
//
// Selection per lane, exact, on the unique keys
// (order key of the bf16 score << 16) | (0xFFFF - index'),
// where index' is the key index less 4 (l / 32): the same for both lanes of a
// word position (wave-uniform constants), and within a lane in the order of
// the true index. The final merge restores the true index.
//   * T: the lane's best 32 keys merged so far, sorted, in registers.
//   * The first block's 32 scores of a lane are sorted into T directly.
//   * theta: the larger of T[31] and a bound on the token's 32nd best value
//     over both lanes, min(T_lo[a - 1], T_hi[31 - a]) maximised over a in
//     {12, 16, 20}: 32 keys of the two lists are at least that large.
//     Neither exceeds the token's knn-th best value (knn <= 32), so no key of
//     the token's top knn is rejected.
//   * Every score whose bf16 value can reach theta is appended to the lane's
//     LDS slots, branch-free (the slots are written, the count moves on a
//     pass). The test is one float compare of the raw word
//     (bf16 bits << 16) | (0xFFFF - index') against tau, the smallest raw
//     word of theta's value (NaN while theta = 0, which nothing is below): a
//     raw word is a float within its bf16 value's rounding interval, so every
//     key >= theta passes, and some equal-valued keys below theta too. A
//     block's appends run between the MFMAs of the next block (the first
//     block's words, already in T, are zeroed: none passes tau = +inf).
//   * After each block the workgroup merges if any of its lanes holds 16
//     slots (all waves at once, at the block's barrier): a chunk of up to 32
//     slots becomes keys (-0 counted as +0), sorted by Batcher's odd-even
//     merge sort (191 compare-exchanges), and the best 32 of T and the chunk,
//     max(T[i], C[31 - i]), are sorted by a bitonic half-cleaner cascade; a
//     wave whose counts leave a chunk's upper 16 slots unused merges it 16
//     wide (63 compare-exchanges), with the same result.
// At the end the two lanes of a token merge their lists (true indices):
// max(T_lo[i], T_hi[31 - i]) through the half-cleaner cascade is the token's
// best 32, stored (through an LDS transpose, two tokens' rows per store) as
// the low (first half) or high (second half) word of the index output, for
// the cartesian kernel below.
// ---------------------------------------------------------------------------
namespace stream {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTok = 32 * kWaves;  // tokens per workgroup
constexpr int kKB = 64;            // keys per staged block
constexpr int kBuf = 47;           // appended-score slots per lane
constexpr int kNet = 32;           // length of the sorted list
constexpr int kWpb = kKB / 4;      // words per block and lane (32 scores)

struct CeNet {
  int n;
  uint8_t a[192], b[192];
};
// Batcher's odd-even merge sort on N elements.
constexpr CeNet oem_net(int N) {
  CeNet t{};
  for (int p = 1; p < N; p <<= 1)
    for (int k = p; k >= 1; k >>= 1)
      for (int j = k % p; j + k < N; j += 2 * k)
        for (int i = 0; i < k && i + j + k < N; ++i)
          if ((i + j) / (2 * p) == (i + j + k) / (2 * p)) {
            t.a[t.n] = (uint8_t)(i + j);
            t.b[t.n] = (uint8_t)(i + j + k);
            ++t.n;
          }
  return t;
}
// Half-cleaner cascade: sorts a bitonic sequence of N elements.
constexpr CeNet clean_net(int N) {
  CeNet t{};
  for (int j = N / 2; j >= 1; j >>= 1)
    for (int i = 0; i < N; ++i)
      if (!(i & j)) {
        t.a[t.n] = (uint8_t)i;
        t.b[t.n] = (uint8_t)(i + j);
        ++t.n;
      }
  return t;
}
constexpr CeNet kSort32 = oem_net(32);
constexpr CeNet kSort16 = oem_net(16);
constexpr CeNet kClean32 = clean_net(32);
static_assert(kSort32.n == 191 && kSort16.n == 63 && kClean32.n == 80, "network sizes");

__device__ __forceinline__ void ce_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = a > b ? a : b, lo = a > b ? b : a;
  a = hi;
  b = lo;
}
// (positions as template arguments: register indices fixed at compile time)
template <int A, int B, int N>
__device__ __forceinline__ void ce_at(uint32_t (&x)[N]) {
  ce_desc(x[A], x[B]);
}
template <size_t... I>
__device__ __forceinline__ void sort32_desc(uint32_t (&x)[32], std::index_sequence<I...>) {
  (ce_at<kSort32.a[I], kSort32.b[I]>(x), ...);
}
template <size_t... I>
__device__ __forceinline__ void sort16_desc(uint32_t (&x)[16], std::index_sequence<I...>) {
  (ce_at<kSort16.a[I], kSort16.b[I]>(x), ...);
}
template <size_t... I>
__device__ __forceinline__ void clean32_desc(uint32_t (&x)[32], std::index_sequence<I...>) {
  (ce_at<kClean32.a[I], kClean32.b[I]>(x), ...);
}

// Inside the kernel keys use the order key okz(b) = b + 0x8000 for b >= 0 and
// 0x10000 - b for negative b (okey16 + 1), under which -0 and +0 are both
// 0x8000 and every other value keeps its order; 0 is no value's key. The lists
// leave the kernel in okey16 form (okz - 1 below 0x8000).
// Key of a raw slot word (bf16 bits << 16 | inverted index).
__device__ __forceinline__ uint32_t raw_key(uint32_t r) {
  const uint32_t sgn = (uint32_t)((int32_t)r >> 31);
  return (r ^ ((sgn & 0x7FFF0000u) | 0x80000000u)) + ((r >> 31) << 16);
}
__device__ __forceinline__ uint32_t key_to_okey16(uint32_t k) { return k - (k < 0x80000000u ? 0x10000u : 0u); }
// The smallest raw word (as a float) whose bf16 value is that of key th; NaN
// for th = 0, so that every score passes.
__device__ __forceinline__ float raw_floor(uint32_t th) {
  const uint32_t ok = th >> 16;
  if (ok == 0u) return __uint_as_float(0xFFFFFFFFu);
  // okz inverse; +0 (0x8000) stands for the -0 slots too, so it takes -0's bits
  const uint32_t b = ok > 0x8000u ? ok - 0x8000u : 0x10000u - ok;
  return __uint_as_float((b << 16) | ((b & 0x8000u) ? 0xFFFFu : 0u));
}
// a pair of bf16 scores with -0 written as +0
__device__ __forceinline__ uint32_t canon_pair(uint32_t p) {
  if ((p & 0xFFFFu) == 0x8000u) p &= 0xFFFF0000u;
  if ((p >> 16) == 0x8000u) p &= 0xFFFFu;
  return p;
}

// Merge slots [J0, J0 + W) (those below cnt, and below kBuf) into T, W = 32
// or 16. The sorted chunk, reversed and padded with zero keys to 32, meets T
// elementwise (the larger of each pair): the top 32 of both, as one bitonic
// sequence, which the cleaner sorts. With W = 16 the padding covers
// T[0 .. 16), which keeps its keys: the result equals the 32-wide merge of
// the same slots whenever the wave's counts leave slots [J0 + 16, J0 + 32)
// unused.
template <int J0, int W>
__device__ __forceinline__ void merge_chunk(uint32_t (&T)[kNet], const uint32_t* buf, uint32_t cnt) {
  static_assert(W == 32 || W == 16, "chunk width");
  uint32_t C[W];
#pragma unroll
  for (int j = 0; j < W; ++j) {
    // the load is unconditional (a slot past the count holds a stale word,
    // masked below), so that no branch surrounds it
    uint32_t r = 0u;
    if (J0 + j < kBuf) r = buf[(J0 + j) * kThreads];
    C[j] = (uint32_t)(J0 + j) < cnt ? raw_key(r) : 0u;
  }
  if constexpr (W == 32)
    sort32_desc(C, std::make_index_sequence<191>{});
  else
    sort16_desc(C, std::make_index_sequence<63>{});
#pragma unroll
  for (int j = 32 - W; j < 32; ++j) T[j] = T[j] > C[31 - j] ? T[j] : C[31 - j];
  clean32_desc(T, std::make_index_sequence<80>{});
}
// Merge slots [J0, J0 + 32) with the narrower chunk when no lane of the wave
// holds a count past J0 + 16 (or the slots end there).
template <int J0>
__device__ __forceinline__ void merge_span(uint32_t (&T)[kNet], const uint32_t* buf, uint32_t cnt) {
  if constexpr (kBuf - J0 <= 16) {
    merge_chunk<J0, 16>(T, buf, cnt);
  } else {
    if (__builtin_amdgcn_ballot_w64(cnt > (uint32_t)(J0 + 16)) != 0)
      merge_chunk<J0, 32>(T, buf, cnt);
    else
      merge_chunk<J0, 16>(T, buf, cnt);
  }
}
// theta: the larger of the lane's T[31] and the pair bound
// max_a min(T_lo[a - 1], T_hi[31 - a]) over both lanes of the token
// (v_permlane32_swap of a register with itself gives every lane the lower
// lanes' value as its first result and the upper lanes' as its second). Both
// are at most the token's 32nd best value, so at most its knn-th for every
// knn <= 32. Only theta's value is used (by raw_floor), so the lanes' index'
// encodings do not matter here.
__device__ __forceinline__ float tau_of(const uint32_t (&T)[kNet]) {
  uint32_t th = T[kNet - 1];
  constexpr int kSplit[3] = {12, 16, 20};
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    const int a = kSplit[s];
    const uint32_t lo = __builtin_amdgcn_permlane32_swap(T[a - 1], T[a - 1], false, false)[0];
    const uint32_t hi = __builtin_amdgcn_permlane32_swap(T[31 - a], T[31 - a], false, false)[1];
    const uint32_t m = lo < hi ? lo : hi;
    th = th > m ? th : m;
  }
  return raw_floor(th);
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Slot budget. Merges are decided once per 64-key block for the whole
// workgroup, and a merge takes every slot (two chunks: [0, 32) and
// [32, kBuf)). At the start of a block every lane holds at most kTrigger - 1
// slots, and a block appends at most 32, the last pair's second write one
// slot past its count: kTrigger + 31 slots suffice.
constexpr int kTrigger = 16;
static_assert(kTrigger + 31 <= kBuf && kBuf <= 64, "slot budget");

// A block's 32 scores of a lane are 16 words of two bf16: word w = 8 kt + j
// holds the scores of elements 2j and 2j + 1 of tile kt's accumulators, keys
// word_key(w) + 4 (lane / 32) and the next one of the block.
__host__ __device__ constexpr int word_key(int w) { return 32 * (w >> 3) + 8 * ((w & 7) >> 1) + 2 * (w & 1); }

// Append the two scores of word p (keys key, key + 1) that can reach theta;
// ns is the lane's slot count. Both slots ns and ns + 1 are written by one
// instruction: slot ns takes r0 if it passes and r1 otherwise, slot ns + 1
// takes r1, and the count moves by the number that pass (two carry-in adds),
// so the slots below the count are exactly the passing scores in order (slot
// ns + 1 lies past the count unless both pass, and is overwritten later).
__device__ __forceinline__ void append_pair(uint32_t p, uint32_t key, uint32_t* buf, uint32_t& ns, float tau,
                                            uint32_t hi_mask) {
  const uint32_t r0 = (p << 16) | (0xFFFFu - key);
  const uint32_t r1 = (p & hi_mask) | (0xFFFEu - key);
  const bool p0 = !(__uint_as_float(r0) < tau);
  const bool p1 = !(__uint_as_float(r1) < tau);
  uint32_t* s = buf + ns * kThreads;
  s[0] = p0 ? r0 : r1;
  s[kThreads] = r1;
  ns += (uint32_t)p0 + (uint32_t)p1;
}

// global_load_lds_dwordx4: lane i's 16 bytes at src go to LDS at dst + 16 i
// (dst wave-uniform). Issued as inline assembly, so that the compiler's
// waitcnt tracking does not treat every later LDS read as dependent on it
// (which turns its lgkmcnt waits into lgkmcnt(0)); the caller waits with
// s_waitcnt vmcnt(0) before the barrier that publishes the data.
// The LDS offset of dst is the low word of its flat address; M0 (reserved to
// the compiler) is restored after the load has read it.
__device__ __forceinline__ void dma16(const void* src, unsigned char* dst) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)dst);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(m0v)
      : "memory");
}

// Key block B (64 rows of HALF bf16) into the LDS block at byte pointer DST by
// direct global->LDS loads: load j of wave w fills the 16-byte chunks
// (w LOADS + j) 64 + lane of the block, and chunk slot q of row r holds the
// row's chunk q ^ (r & 15), so that the rows an LDS read serves hit distinct
// banks.
#define PKM_STREAM_STAGE(B, DST)                                                                       \
  {                                                                                                   \
    const int b_ = (B);                                                                               \
    unsigned char* d_ = (DST);                                                                        \
    _Pragma("unroll") for (int l_ = 0; l_ < LOADS; ++l_) {                                            \
      const int p_ = (w * LOADS + l_) * 64 + lane;                                                    \
      const int r_ = p_ / CPR, q_ = p_ % CPR;                                                         \
      const uint16_t* src_ = kb + (int64_t)(b_ * kKB + r_) * HALF + (q_ ^ (r_ & 15)) * 8;            \
      dma16(src_, d_ + (w * LOADS + l_) * 1024);                                                      \
    }                                                                                                 \
  }

// Q [Ntok, H, 2 HALF], Kt [2 H n, HALF] (bf16 bits); lists: out_idx as 32-bit
// words; out_i1/out_i2 [Ntok, H, knn]; with SUB, out_s1/out_s2 [Ntok, H, n]
// as pairs of bf16.
template <int KS, bool SUB>
__global__ __launch_bounds__(kThreads, 1) void pkm_score_stream_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kt, int64_t Ntok, int H, int n, int knn,
    uint32_t* __restrict__ lists, int64_t* __restrict__ out_i1, int64_t* __restrict__ out_i2,
    uint32_t* __restrict__ out_s1, uint32_t* __restrict__ out_s2) {
  constexpr int HALF = 16 * KS;
  constexpr int CPR = HALF / 8;               // 16-byte chunks per key row
  constexpr int BLK = kKB * HALF * 2;         // bytes per staged block
  constexpr int LOADS = BLK / 1024 / kWaves;  // 1 KB global->LDS loads per wave per block
  constexpr int STEPS = 2 * KS;               // MFMA steps per block: tile 0's k-steps, then tile 1's
  constexpr int LOOK = 4;                     // A fragments read this many steps ahead
  static_assert(LOADS * 1024 * kWaves == BLK && CPR >= 16 && STEPS >= kWpb, "block layout");
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* kst = smem;                                  // [2][kKB][CPR] 16-byte chunks
  uint32_t* buf = (uint32_t*)(smem + 2 * BLK) + threadIdx.x;  // slot j at buf[j * kThreads]
  uint32_t* flags = (uint32_t*)(smem + 2 * BLK) + kBuf * kThreads;  // [2][kWaves]

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H2 = 2 * H;
  // (half, head) fastest, head fastest of all: workgroups go round-robin to
  // the 8 XCDs, so with H a multiple of 8 an XCD's L2 serves fixed heads,
  // both halves (whose lists share the output's cache lines)
  const int hc = (int)(blockIdx.x % (unsigned)H2);
  const int64_t tile = blockIdx.x / (unsigned)H2;
  const int h = hc % H, c = hc / H;
  const int hk = 2 * h + c;                 // key rows (2h + c) n .. of this head-half
  const int64_t tw = tile * kTok + 32 * w;  // first token of this wave
  const int64_t tok = tw + (lane & 31);     // this lane's token
  const bool live = tok < Ntok;

  // B fragments: token tok; k = 16 s + 8 (lane / 32)
  u32x4_t bq[KS];
  {
    const uint16_t* qr = Q + ((live ? tok : 0) * H + h) * (2 * HALF) + c * HALF + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < KS; ++s) bq[s] = *(const u32x4_t*)(qr + 16 * s);
    if (!live) {
#pragma unroll
      for (int s = 0; s < KS; ++s) bq[s] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  // the B fragments live in accumulation registers (MFMA reads them there),
  // leaving the arch VGPRs to the selection and the A fragments
#pragma unroll
  for (int s = 0; s < KS; ++s) asm volatile("" : "+a"(bq[s]));
  // byte offset of A chunk 2 s + lane / 32 in the lane's (swizzled) row, s < 8;
  // s >= 8 adds 256 (the row's second 16 chunks)
  int aoff[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) aoff[s] = ((2 * s + (lane >> 5)) ^ (lane & 15)) * 16;

  const uint16_t* kb = Kt + (int64_t)hk * n * HALF;
  const int nb = n / kKB;

  uint32_t T[kNet];
#pragma unroll
  for (int i = 0; i < kNet; ++i) T[i] = 0u;
  uint32_t P[kWpb];
#pragma unroll
  for (int i = 0; i < kWpb; ++i) P[i] = 0u;
  uint32_t ns = 0;  // slot count
  // +inf until the second block's words are appended (P holds no scores, then
  // the first block's, which are in T already); tau_first once they are
  float tau = __uint_as_float(0x7F800000u), tau_first = 0.f;
  // this lane's half of the sub-score row (pairs of bf16: the lane's keys
  // 4 (lane / 32) + ... are at word 2 (lane / 32) + ...); a NULL output (the
  // caller asked for the other half only) writes nothing
  uint32_t* srow = nullptr;
  bool write_sub = false;
  if constexpr (SUB) {
    uint32_t* out_s = c == 0 ? out_s1 : out_s2;
    write_sub = live && out_s != nullptr;
    if (write_sub) srow = out_s + (tok * H + h) * (n / 2) + 2 * (lane >> 5);
  }
  // 0xFFFF0000 in a register: v_and_or_b32 takes it beside the scalar index
  uint32_t hi_mask = 0xFFFF0000u;
  asm volatile("" : "+v"(hi_mask));

  PKM_STREAM_STAGE(0, kst);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // Iteration j < nb: the MFMAs of block j interleaved with the appends of
  // block j - 1's words (P), which are replaced by block j's as its tiles
  // complete; block j + 1 is staged meanwhile. Iteration nb appends block
  // nb - 1's words. After each iteration the workgroup merges if any of its
  // lanes holds kTrigger slots (the waves decide together at the barrier, so
  // that they merge at the same time); after the last, each wave merges its
  // remaining slots.
#pragma unroll 1
  for (int j = 0; j <= nb; ++j) {
    if (j < nb) {
      const unsigned char* kcur = kst + (j & 1) * BLK;
      if (j + 1 < nb) {
        PKM_STREAM_STAGE(j + 1, kst + ((j + 1) & 1) * BLK);
      }
      const uint32_t kprev = (uint32_t)(j - 1) * kKB;  // key base of the words being appended
      const unsigned char* ar = kcur + (lane & 31) * (CPR * 16);
      f32x16_t X[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) X[kt] = f32x16_t{};
      u32x4_t A[STEPS];
#pragma unroll
      for (int t = 0; t < LOOK; ++t)
        A[t] = *(const u32x4_t*)(ar + (t / KS) * 32 * CPR * 16 + aoff[(t % KS) & 7] + ((t % KS) >> 3) * 256);
#pragma unroll
      for (int t = 0; t < STEPS; ++t) {
        const int kt = t / KS, st = t % KS;
        if (t + LOOK < STEPS) {
          const int t2 = t + LOOK;
          A[t2] = *(const u32x4_t*)(ar + (t2 / KS) * 32 * CPR * 16 + aoff[(t2 % KS) & 7] + ((t2 % KS) >> 3) * 256);
        }
        X[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, A[t]),
                                                        __builtin_bit_cast(bf16x8_t, bq[st]), X[kt], 0, 0, 0);
#pragma unroll
        for (int q = (t * kWpb) / STEPS; q < ((t + 1) * kWpb) / STEPS; ++q)
          append_pair(P[q], kprev + word_key(q), buf, ns, tau, hi_mask);
        if (t >= KS) {
          // tile 0 is complete: its words replace the appended ones
#pragma unroll
          for (int jj = ((t - KS) * 8) / KS; jj < ((t - KS + 1) * 8) / KS; ++jj)
            P[jj] = pack2_bf16(X[0][2 * jj], X[0][2 * jj + 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) P[8 + jj] = pack2_bf16(X[1][2 * jj], X[1][2 * jj + 1]);
      if constexpr (SUB) {
        if (write_sub) {
#pragma unroll
          for (int q = 0; q < kWpb; ++q) srow[(j * kKB + word_key(q)) >> 1] = canon_pair(P[q]);
        }
      }
      if (j == 0) {
        // the first block's 32 scores of the lane, sorted, are T
#pragma unroll
        for (int q = 0; q < kWpb; ++q) {
          T[2 * q] = raw_key((P[q] << 16) | (0xFFFFu - (uint32_t)word_key(q)));
          T[2 * q + 1] = raw_key((P[q] & hi_mask) | (0xFFFEu - (uint32_t)word_key(q)));
        }
        sort32_desc(T, std::make_index_sequence<191>{});
        tau_first = tau_of(T);
        // zero words (tiny positive raw words) stay below tau = +inf, where a
        // word holding an infinity (a NaN raw word) would pass again
#pragma unroll
        for (int q = 0; q < kWpb; ++q) P[q] = 0u;
      }
    } else {
#pragma unroll
      for (int q = 0; q < kWpb; ++q) append_pair(P[q], (uint32_t)(nb - 1) * kKB + word_key(q), buf, ns, tau, hi_mask);
    }
    if (j == 1) tau = tau_first;
    bool need;
    if (j < nb) {
      const bool mine = __builtin_amdgcn_ballot_w64(ns >= kTrigger) != 0;
      if (lane == 0) flags[(j & 1) * kWaves + w] = mine ? 1u : 0u;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      uint32_t any = 0;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) any |= flags[(j & 1) * kWaves + v];
      need = any != 0;
    } else {
      need = __builtin_amdgcn_ballot_w64(ns > 0u) != 0;
    }
    if (need) {
      // every slot: [0, 32), then [32, kBuf) where a lane holds more than 32
      merge_span<0>(T, buf, ns);
      if (__builtin_amdgcn_ballot_w64(ns > 32u) != 0) merge_span<32>(T, buf, ns);
      ns = 0u;
      if (j < nb) tau = tau_of(T);
    }
  }

  // The token's list: the upper lane's keys get their true index (0xFFFF -
  // index is 4 lower), then both lanes merge the pair's lists,
  // max(T_lo[i], T_hi[31 - i]) sorted by the cleaner (the same in both).
  const uint32_t fix = (lane >> 5) ? 4u : 0u;
#pragma unroll
  for (int i = 0; i < kNet; ++i) T[i] = T[i] != 0u ? T[i] - fix : 0u;
#pragma unroll
  for (int i = 0; i < kNet / 2; ++i) {
    const auto a = __builtin_amdgcn_permlane32_swap(T[i], T[i], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(T[31 - i], T[31 - i], false, false);
    T[i] = a[0] > b[1] ? a[0] : b[1];       // max(T_lo[i], T_hi[31 - i])
    T[31 - i] = b[0] > a[1] ? b[0] : a[1];  // max(T_lo[31 - i], T_hi[i])
  }
  clean32_desc(T, std::make_index_sequence<80>{});

  // Outputs through a [32][33] word tile per wave (LDS is idle once every wave
  // has merged), so that a store covers two tokens' contiguous rows: lane i
  // writes word i % 32 of token 2 m + i / 32 of the wave.
  __syncthreads();
  uint32_t* tp = (uint32_t*)smem + w * (32 * 33);
  if (lane < 32) {
#pragma unroll
    for (int q = 0; q < kNet; ++q) tp[lane * 33 + q] = key_to_okey16(T[q]);
  }
  __builtin_amdgcn_wave_barrier();
  int64_t* oi = c == 0 ? out_i1 : out_i2;
  const int q = lane & 31;
#pragma unroll 4
  for (int m = 0; m < 16; ++m) {
    const int tl = 2 * m + (lane >> 5);
    const int64_t t = tw + tl;
    const uint32_t k = tp[tl * 33 + q];
    if (t < Ntok && q < knn) {
      lists[(t * H + h) * (2 * (int64_t)knn) + 2 * q + c] = k;
      if (oi != nullptr) oi[(t * H + h) * knn + q] = (int64_t)(0xFFFFu - (k & 0xFFFFu));
    }
  }
}
#undef PKM_STREAM_STAGE

__host__ inline size_t lds_bytes(int half) {
  return (size_t)2 * kKB * half * 2 + (size_t)kBuf * kThreads * 4 + 2 * kWaves * 4;
}

}  // namespace stream

constexpr int kCartLpr = 8;  // lanes per row of the cartesian kernel
__host__ inline size_t cartesian_lds_bytes(int knn) {
  const int kl = (knn + 3) & ~3;
  return (size_t)(kThreads / kCartLpr) * (size_t)(3 * kl + score_cap(knn, kCartLpr) + 4) * 4;
}

// Dynamic LDS above 64 KiB is enabled once per device and kernel (idempotent,
// so a race between threads only repeats the call).
static int enable_lds(const void* fn, int bytes, std::atomic<uint64_t>& done, const char* what) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pkm_set_error(PKM_ERR_HIP, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  const uint64_t bit = 1ull << (dev & 63);
  if (!(done.load(std::memory_order_relaxed) & bit)) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess)
      return pkm_set_error(PKM_ERR_HIP, "%s: hipFuncSetAttribute failed: %s", what, hipGetErrorString(e));
    done.fetch_or(bit, std::memory_order_relaxed);
  }
  return PKM_OK;
}

// The cartesian step of the packed lists (32-bit keys: bf16 scores). The LDS
// attribute is set once per device, to the device maximum, so that every
// knn's layout fits.
template <typename TIN>
static int launch_cartesian(int64_t Ntok, int H, int n, int knn, int lds_max, void* out_scores, int64_t* out_idx,
                            hipStream_t st) {
  static_assert(sizeof(typename Sel<TIN>::Key) == 4, "packed lists need 32-bit keys");
  static std::atomic<uint64_t> cart_lds_enabled{0};
  const size_t cl = cartesian_lds_bytes(knn);
  if ((int)cl > lds_max)
    return pkm_set_error(PKM_ERR_UNSUPPORTED, "pkm_score_topk: knn %d needs %zu bytes of LDS for the cartesian step",
                         knn, cl);
  const int rc = enable_lds((const void*)pkm_score_cartesian_kernel<TIN, kCartLpr>, lds_max, cart_lds_enabled,
                            "pkm_score_topk");
  if (rc != PKM_OK) return rc;
  const int64_t rows = Ntok * H;
  const int64_t cblocks = (rows + kThreads / kCartLpr - 1) / (kThreads / kCartLpr);
  hipLaunchKernelGGL((pkm_score_cartesian_kernel<TIN, kCartLpr>), dim3((unsigned)cblocks), dim3(kThreads), cl, st,
                     rows, n, knn, (TIN*)out_scores, out_idx);
  return PKM_OK;
}

template <typename TIN, int IDW, int TM, int KSC>
static int launch_score_tm(const void* q, const void* keys, int kpack, int64_t Ntok, int H, int n, int half, int knn,
                           size_t lds, int lds_max, void* out_scores, int64_t* out_idx, int64_t* out_i1,
                           int64_t* out_i2, void* out_s1, void* out_s2, hipStream_t st) {
  static std::atomic<uint64_t> lds_enabled{0};
  int rc = enable_lds((const void*)pkm_score_topk_kernel<TIN, IDW, TM, KSC>, lds_max, lds_enabled, "pkm_score_topk");
  if (rc != PKM_OK) return rc;
  const int64_t blocks = ((Ntok + TM - 1) / TM) * H;
  {
    KernelSpan span("score_topk", st);
    hipLaunchKernelGGL((pkm_score_topk_kernel<TIN, IDW, TM, KSC>), dim3((unsigned)blocks), dim3(kThreads), lds, st,
                       (const TIN*)q, (const TIN*)keys, kpack, Ntok, H, n, half, knn, (TIN*)out_scores, out_idx, out_i1,
                       out_i2, (TIN*)out_s1, (TIN*)out_s2);
  }
  if constexpr (sizeof(typename Sel<TIN>::Key) == 4) return launch_cartesian<TIN>(Ntok, H, n, knn, lds_max, out_scores, out_idx, st);
  return PKM_OK;
}

// The streaming kernel (bf16 dot, knn <= 32), then the cartesian step.
template <int KS, bool SUB>
static int launch_stream(const void* q, const void* keys, int64_t Ntok, int H, int n, int knn, int lds_max,
                         void* out_scores, int64_t* out_idx, int64_t* out_i1, int64_t* out_i2, void* out_s1,
                         void* out_s2, hipStream_t st) {
  static std::atomic<uint64_t> lds_enabled{0};
  int rc = enable_lds((const void*)stream::pkm_score_stream_kernel<KS, SUB>, lds_max, lds_enabled, "pkm_score_topk");
  if (rc != PKM_OK) return rc;
  const int64_t blocks = ((Ntok + stream::kTok - 1) / stream::kTok) * 2 * H;
  {
    KernelSpan span("score_topk", st);
    hipLaunchKernelGGL((stream::pkm_score_stream_kernel<KS, SUB>), dim3((unsigned)blocks), dim3(stream::kThreads),
                       stream::lds_bytes(16 * KS), st, (const uint16_t*)q, (const uint16_t*)keys, Ntok, H, n, knn,
                       (uint32_t*)out_idx, out_i1, out_i2, (uint32_t*)out_s1, (uint32_t*)out_s2);
  }
  return launch_cartesian<bf16_t>(Ntok, H, n, knn, lds_max, out_scores, out_idx, st);
}

// Kernel variant for (TM, k-steps per half): the k-step counts of the common
// half key dims (128, 256, 512 elements) are compile-time.
template <typename TIN, int IDW, int TM>
static int launch_score_ks(const void* q, const void* keys, int kpack, int64_t Ntok, int H, int n, int half, int knn,
                           size_t lds, int lds_max, void* out_scores, int64_t* out_idx, int64_t* out_i1,
                           int64_t* out_i2, void* out_s1, void* out_s2, hipStream_t st) {
  switch (half / Sel<TIN>::KSTEP) {
    case 4:
      return launch_score_tm<TIN, IDW, TM, 4>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx,
                                              out_i1, out_i2, out_s1, out_s2, st);
    case 8:
      return launch_score_tm<TIN, IDW, TM, 8>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx,
                                              out_i1, out_i2, out_s1, out_s2, st);
    case 16:
      return launch_score_tm<TIN, IDW, TM, 16>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx,
                                               out_i1, out_i2, out_s1, out_s2, st);
    default:
      return launch_score_tm<TIN, IDW, TM, 0>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx,
                                              out_i1, out_i2, out_s1, out_s2, st);
  }
}

template <typename TIN, int IDW>
static int launch_score(int TM, const void* q, const void* keys, int kpack, int64_t Ntok, int H, int n, int half, int knn,
                        size_t lds, int lds_max, void* out_scores, int64_t* out_idx, int64_t* out_i1,
                        int64_t* out_i2, void* out_s1, void* out_s2, hipStream_t st) {
  switch (TM) {
    case 64:
      return launch_score_ks<TIN, IDW, 64>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx, out_i1,
                                           out_i2, out_s1, out_s2, st);
    case 32:
      return launch_score_ks<TIN, IDW, 32>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx, out_i1,
                                           out_i2, out_s1, out_s2, st);
    default:
      return launch_score_ks<TIN, IDW, 16>(q, keys, kpack, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx, out_i1,
                                           out_i2, out_s1, out_s2, st);
  }
}

}  // namespace pkm

using namespace pkm;

namespace pkm {
int score_topk_generic(const void* query, const void* keys, int64_t num_tokens, int64_t heads, int64_t n_keys,
                       int64_t half, int64_t knn, int score_type, int dtype, void* out_scores, int64_t* out_indices,
                       int64_t* out_i1, int64_t* out_i2, void* out_s1, void* out_s2, int lds_max, hipStream_t st);
}

namespace pkm {
// Key tiles in the order the tile kernel's k-steps read them: within each
// block of 16 consecutive keys (a column tile), 16-byte chunk c of the 16 keys
// becomes contiguous (chunk-major), so the B operands of one k-step are one
// contiguous KB instead of 64 bytes of 16 rows each. One thread per chunk.
__global__ __launch_bounds__(256) void score_keys_pack_kernel(const uint4* __restrict__ K, uint4* __restrict__ P,
                                                              int64_t chunks, int CH) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= chunks) return;
  const int64_t tsz = 16 * (int64_t)CH;
  const int64_t tile = o / tsz;
  const int w = (int)(o - tile * tsz);
  P[o] = K[tile * tsz + (int64_t)(w & 15) * CH + (w >> 4)];
}
}  // namespace pkm

static int score_topk_impl(const void* query, const void* keys, int64_t num_tokens, int64_t heads, int64_t n_keys,
                           int64_t half, int64_t knn, int score_type, int dtype, void* out_scores,
                           int64_t* out_indices, int64_t* out_sub_indices1, int64_t* out_sub_indices2,
                           void* out_sub_scores1, void* out_sub_scores2, void* workspace, size_t workspace_bytes,
                           void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16 || dtype == PKM_DTYPE_F16, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: dtype %d not supported (float32, bfloat16 and float16 are)", dtype);
  PKM_REQUIRE(score_type == PKM_SCORE_DOT || score_type == PKM_SCORE_IDW, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_topk: bad score type %d", score_type);
  PKM_REQUIRE(num_tokens >= 0 && heads >= 1 && heads < 65536 && n_keys >= 1 && half >= 1 && knn >= 1,
              PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: bad sizes");
  PKM_REQUIRE(knn <= n_keys, PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: knn %lld > n_keys %lld", (long long)knn,
              (long long)n_keys);
  if (num_tokens == 0) return PKM_OK;
  PKM_REQUIRE(query && keys && out_scores && out_indices, PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: null pointer");
  PKM_REQUIRE((uintptr_t)out_sub_scores1 % 4 == 0 && (uintptr_t)out_sub_scores2 % 4 == 0 &&
                  (uintptr_t)out_scores % (dtype == PKM_DTYPE_F32 ? 4 : 2) == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: score outputs must be 4-byte aligned");
  const int esz = dtype == PKM_DTYPE_BF16 ? 2 : 4;  // score-tile element = order key of the input dtype
  const int key_bytes = dtype == PKM_DTYPE_BF16 ? 4 : 8;
  int dev = 0, lds_max = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess)
    return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: device query failed: %s", hipGetErrorString(e));
  if (lds_max > kMaxLds) lds_max = kMaxLds;
  hipStream_t st = (hipStream_t)stream;
  // the tuned kernels: float32 / bfloat16, knn <= 64, n_keys a multiple of 64 up to kMaxN, half a multiple
  // of the MFMA k-step, 16-byte aligned operands; anything else takes the generic kernel (score_generic.hip)
  const int kstep = dtype == PKM_DTYPE_BF16 ? Sel<bf16_t>::KSTEP : Sel<float>::KSTEP;
  const bool tuned = dtype != PKM_DTYPE_F16 && knn <= 64 && n_keys % 64 == 0 && n_keys <= kMaxN && half % kstep == 0 &&
                     (uintptr_t)query % 16 == 0 && (uintptr_t)keys % 16 == 0;
  if (!tuned) {
    const int rc = score_topk_generic(query, keys, num_tokens, heads, n_keys, half, knn, score_type, dtype, out_scores,
                                      out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                      out_sub_scores2, lds_max, st);
    if (rc != PKM_OK) return rc;
    return pkm_check_launch("pkm_score_topk");
  }
  if (dtype == PKM_DTYPE_BF16 && score_type == PKM_SCORE_DOT && knn <= stream::kNet && (half == 128 || half == 256) &&
      (int)stream::lds_bytes((int)half) <= lds_max) {
    const int64_t blocks = ((num_tokens + stream::kTok - 1) / stream::kTok) * 2 * heads;
    PKM_REQUIRE(blocks < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: grid too large");
    const bool sub = out_sub_scores1 != nullptr || out_sub_scores2 != nullptr;
    auto* launch = half == 256 ? (sub ? launch_stream<16, true> : launch_stream<16, false>)
                               : (sub ? launch_stream<8, true> : launch_stream<8, false>);
    const int rc = launch(query, keys, num_tokens, (int)heads, (int)n_keys, (int)knn, lds_max, out_scores, out_indices,
                          out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, st);
    if (rc != PKM_OK) return rc;
    return pkm_check_launch("pkm_score_topk");
  }
  int TM = 64;
  while (TM > 16 && (score_lds_layout(TM, (int)n_keys, (int)half, (int)knn, esz, key_bytes).total > lds_max ||
                     n_keys > score_max_n(TM, esz)))
    TM /= 2;
  const int lds = score_lds_layout(TM, (int)n_keys, (int)half, (int)knn, esz, key_bytes).total;
  if (lds > lds_max) {  // a tile too large for the device's LDS: the generic kernel
    const int rc = score_topk_generic(query, keys, num_tokens, heads, n_keys, half, knn, score_type, dtype, out_scores,
                                      out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                      out_sub_scores2, lds_max, st);
    if (rc != PKM_OK) return rc;
    return pkm_check_launch("pkm_score_topk");
  }
  const int64_t blocks = ((num_tokens + TM - 1) / TM) * heads;
  PKM_REQUIRE(blocks < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: grid too large");
  int rc;
  const int H = (int)heads, n = (int)n_keys, hf = (int)half, k = (int)knn;
  // with a workspace of the keys' size: the keys packed tile-major first (one
  // pass over the table), so the kernel's key loads use whole cache lines
  const size_t key_bytes_all = (size_t)(2 * heads * n_keys) * (size_t)half * (dtype == PKM_DTYPE_BF16 ? 2 : 4);
  const int kpack = workspace != nullptr && workspace_bytes >= key_bytes_all && (uintptr_t)workspace % 16 == 0;
  if (kpack) {
    const int64_t chunks = (int64_t)(key_bytes_all / 16);
    const int CH = (int)(half * (dtype == PKM_DTYPE_BF16 ? 2 : 4) / 16);
    hipLaunchKernelGGL(score_keys_pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st,
                       (const uint4*)keys, (uint4*)workspace, chunks, CH);
    keys = workspace;
  }
  if (dtype == PKM_DTYPE_BF16) {
    rc = score_type == PKM_SCORE_DOT
             ? launch_score<bf16_t, 0>(TM, query, keys, kpack, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                       out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                       out_sub_scores2, st)
             : launch_score<bf16_t, 1>(TM, query, keys, kpack, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                       out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                       out_sub_scores2, st);
  } else {
    rc = score_type == PKM_SCORE_DOT
             ? launch_score<float, 0>(TM, query, keys, kpack, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                      out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                      out_sub_scores2, st)
             : launch_score<float, 1>(TM, query, keys, kpack, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                      out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                      out_sub_scores2, st);
  }
  if (rc != PKM_OK) return rc;
  return pkm_check_launch("pkm_score_topk");
}

extern "C" int pkm_score_topk(const void* query, const void* keys, int64_t num_tokens, int64_t heads, int64_t n_keys,
                              int64_t half, int64_t knn, int score_type, int dtype, void* out_scores,
                              int64_t* out_indices, int64_t* out_sub_indices1, int64_t* out_sub_indices2,
                              void* out_sub_scores1, void* out_sub_scores2, void* stream) {
  return score_topk_impl(query, keys, num_tokens, heads, n_keys, half, knn, score_type, dtype, out_scores,
                         out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, nullptr, 0,
                         stream);
}

extern "C" size_t pkm_score_topk_workspace_size(int64_t heads, int64_t n_keys, int64_t half, int dtype) {
  if (heads < 1 || n_keys < 1 || half < 1) return 0;
  return (size_t)(2 * heads * n_keys * half) * (dtype == PKM_DTYPE_F32 ? 4 : 2);
}

extern "C" int pkm_score_topk_ws(const void* query, const void* keys, int64_t num_tokens, int64_t heads,
                                 int64_t n_keys, int64_t half, int64_t knn, int score_type, int dtype,
                                 void* out_scores, int64_t* out_indices, int64_t* out_sub_indices1,
                                 int64_t* out_sub_indices2, void* out_sub_scores1, void* out_sub_scores2,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return score_topk_impl(query, keys, num_tokens, heads, n_keys, half, knn, score_type, dtype, out_scores,
                         out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, workspace,
                         workspace_bytes, stream);
}

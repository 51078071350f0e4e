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
//      1/8 of the key tiles from L2 (16-byte loads, keys read once per
//      workgroup) and computes the [TM x 16] score tiles on MFMA
//      (16x16x32 bf16 / 16x16x4 f32); the epilogue writes the order keys of
//      the rounded scores into the LDS score tile [TM][n] and keeps, per row,
//      the exact maximum of each of G = min(n, 128) column groups
//      (group = column mod 128) in registers.
//   B. Per row (one wave): T0 = knn-th largest group maximum is a lower bound
//      of the knn-th largest score (knn groups each hold a score >= T0), so
//      the top-knn are among the scores >= T0 (about 1.1 knn of them on
//      random data). 8-score chunks whose maximum (packed 16-bit max) is
//      below T0 are dropped, the scores of the remaining chunks are compacted
//      with wave ballots, and each candidate's rank is counted. More than
//      kCandCap candidates fall back to an exact threshold search over the row.
//   C. (after the second half) per token, the cartesian candidates restricted
//      to the pairs (a+1)(b+1) <= knn — every other pair is preceded, in
//      (value, flat index) order, by at least knn pairs. The knn pairs (a, 0)
//      and the knn pairs (0, b) bound the knn-th value from below, which again
//      leaves a few dozen candidates to rank.
// Workgroups map head-fastest onto the grid, so with 8 heads each XCD (and its
// L2) serves one head's keys.
#include <atomic>

#include "pkm_common.h"

namespace pkm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxN = 2048;       // n_keys limit
constexpr int kMaxPairSlots = 5;  // knn = 64 -> 280 candidate pairs
constexpr int kCandCap = 128;     // candidates ranked per row before the exact fallback
constexpr int kChunk = 8;         // scores per culling chunk
constexpr int kMaxLds = 160 * 1024;

// ---------------------------------------------------------------------------
// Order keys: monotone maps of the stored score bits to unsigned integers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t okey16(uint32_t b) { return b ^ ((b & 0x8000u) ? 0xFFFFu : 0x8000u); }
__device__ __forceinline__ uint32_t okey16_inv(uint32_t k) { return k ^ ((k & 0x8000u) ? 0x8000u : 0xFFFFu); }
__device__ __forceinline__ uint32_t okey32(uint32_t b) {
  return b ^ ((b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}
__device__ __forceinline__ uint32_t okey32_inv(uint32_t k) {
  return k ^ ((k & 0x80000000u) ? 0x80000000u : 0xFFFFFFFFu);
}

// Per score type: score-tile element (an order key), unique selection key,
// MFMA step. coarse() is the 16-bit key the thresholds compare.
template <typename TIN>
struct Sel;

template <>
struct Sel<bf16_t> {
  typedef uint16_t Store;  // order key of the bf16 score
  typedef uint32_t Key;    // (order key << 16) | (0xFFFF - index)
  static constexpr int KSTEP = 32;  // k per 16-byte fragment: one 16x16x32 MFMA
  static __device__ __forceinline__ uint32_t okey_of(float v) { return okey16(f32_to_bf16_bits(v + 0.0f)); }
  static __device__ __forceinline__ uint32_t coarse(uint32_t ok) { return ok; }
  static __device__ __forceinline__ Key make(uint32_t ok, uint32_t idx) { return (ok << 16) | (0xFFFFu - idx); }
  static __device__ __forceinline__ uint32_t key_okey(Key k) { return k >> 16; }
  static __device__ __forceinline__ uint32_t key_idx(Key k) { return 0xFFFFu - (k & 0xFFFFu); }
  static __device__ __forceinline__ float value(uint32_t ok) { return bf16_to_f32(okey16_inv(ok)); }
  static __device__ __forceinline__ void put(bf16_t* p, int64_t i, uint32_t ok) { p[i].x = (uint16_t)okey16_inv(ok); }
  // maximum coarse key of one 8-score chunk (16 bytes)
  static __device__ __forceinline__ uint32_t chunk_max(const Store* p) {
    const uint4 v = *(const uint4*)p;
    u16x2_t m = __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, v.x), __builtin_bit_cast(u16x2_t, v.y));
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, v.z));
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, v.w));
    return m.x > m.y ? m.x : m.y;
  }
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
  static __device__ __forceinline__ uint32_t coarse(uint32_t ok) { return ok >> 16; }  // truncated: a lower bound
  static __device__ __forceinline__ Key make(uint32_t ok, uint32_t idx) {
    return ((uint64_t)ok << 32) | (uint64_t)(0xFFFFFFFFu - idx);
  }
  static __device__ __forceinline__ uint32_t key_okey(Key k) { return (uint32_t)(k >> 32); }
  static __device__ __forceinline__ uint32_t key_idx(Key k) { return 0xFFFFFFFFu - (uint32_t)k; }
  static __device__ __forceinline__ float value(uint32_t ok) { return __uint_as_float(okey32_inv(ok)); }
  static __device__ __forceinline__ void put(float* p, int64_t i, uint32_t ok) { p[i] = __uint_as_float(okey32_inv(ok)); }
  static __device__ __forceinline__ uint32_t chunk_max(const Store* p) {
    const uint4 a = *(const uint4*)p, b = *(const uint4*)(p + 4);
    uint32_t m = a.x > a.y ? a.x : a.y;
    m = m > a.z ? m : a.z;
    m = m > a.w ? m : a.w;
    m = m > b.x ? m : b.x;
    m = m > b.y ? m : b.y;
    m = m > b.z ? m : b.z;
    m = m > b.w ? m : b.w;
    return m >> 16;
  }
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
__device__ __forceinline__ uint32_t shfl_key(uint32_t v, int src) { return (uint32_t)__shfl((int)v, src); }
__device__ __forceinline__ uint64_t shfl_key(uint64_t v, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src), hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t lane_key(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}
__device__ __forceinline__ uint64_t lane_key(uint64_t v, int src) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}

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
__device__ __forceinline__ Key exact_topk(F key_at, int nslots, int knn, Key* scr) {
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
// LDS layout (host and device agree through score_lds_layout).
// ---------------------------------------------------------------------------
struct ScoreLds {
  int s_bytes;     // score tile [TM][n] of order keys
  int r_bytes;     // shared region: query stage in phase A, else the three below
  int gmax_bytes;  // [TM][G] uint16 coarse keys of the group maxima
  int scr_bytes;   // per wave: kCandCap selection keys
  int list_bytes;  // per wave: n / kChunk uint16 chunk ids
  int total;
};

__host__ __device__ inline int score_groups(int n) { return n < 128 ? n : 128; }

__host__ __device__ inline ScoreLds score_lds_layout(int TM, int n, int half, int esz, int key_bytes) {
  ScoreLds L;
  L.s_bytes = ((TM * n * esz) + 15) & ~15;
  L.gmax_bytes = ((TM * score_groups(n) * 2) + 15) & ~15;
  L.scr_bytes = kCandCap * key_bytes;
  L.list_bytes = (((n / kChunk) * 2) + 15) & ~15;
  const int q_bytes = TM * half * (esz == 2 ? 2 : 4);
  const int sel_bytes = L.gmax_bytes + kWaves * (L.scr_bytes + L.list_bytes);
  L.r_bytes = q_bytes > sel_bytes ? q_bytes : sel_bytes;
  L.total = L.s_bytes + L.r_bytes;
  return L;
}

// Largest power of two (<= 8) dividing `chunks`, minus one: the XOR mask of
// the query-stage chunk swizzle (stays inside the row).
__host__ __device__ inline int chunk_swizzle_mask(int chunks) {
  int m = 1;
  while (m < 8 && chunks % (2 * m) == 0) m *= 2;
  return m - 1;
}

// Column swizzle of the score tile: the 4 rows an MFMA store writes at once
// (rows 4g + e, g = 0..3) land in different LDS banks. It permutes 16-score
// blocks inside 64-score blocks, so 8-score chunks stay contiguous.
__device__ __forceinline__ int s_phys(int row, int col) { return col ^ (((row >> 2) & 3) << 4); }

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <typename TIN, int IDW, int TM>
__global__ __launch_bounds__(kThreads) void pkm_score_topk_kernel(
    const TIN* __restrict__ Q, const TIN* __restrict__ Kt, int64_t Ntok, int H, int n, int half, int knn,
    TIN* __restrict__ out_scores, int64_t* __restrict__ out_idx, int64_t* __restrict__ out_i1,
    int64_t* __restrict__ out_i2, TIN* __restrict__ out_s1, TIN* __restrict__ out_s2) {
  typedef Sel<TIN> SL;
  typedef typename SL::Store Store;
  typedef typename SL::Key Key;
  constexpr int RT = TM / 16;  // row tiles
  constexpr int CB = 4;        // column tiles per batch
  constexpr int ESZ = (int)sizeof(TIN);
  constexpr int EPC = 16 / ESZ;  // input elements per 16-byte chunk
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int h = (int)(blockIdx.x % (unsigned)H);
  const int64_t t0 = (int64_t)(blockIdx.x / (unsigned)H) * TM;
  const ScoreLds L = score_lds_layout(TM, n, half, (int)sizeof(Store), (int)sizeof(Key));
  Store* S = (Store*)smem;
  unsigned char* R = smem + L.s_bytes;
  uint4* QS = (uint4*)R;        // phase A: query stage
  uint16_t* GM = (uint16_t*)R;  // phases B, C: group maxima
  Key* scr = (Key*)(R + L.gmax_bytes + w * L.scr_bytes);
  uint16_t* clist = (uint16_t*)(R + L.gmax_bytes + kWaves * L.scr_bytes + w * L.list_bytes);

  const int kdim = 2 * half;
  const int CH = half / EPC;  // 16-byte chunks per query half row
  const int cmask = chunk_swizzle_mask(CH);
  const int KS = half / SL::KSTEP;
  const int ncol = n / 16;
  const int G = score_groups(n);
  const int NC = n / kChunk;  // culling chunks per row

  // candidate pairs of the cartesian step: slot s -> (a, b), a-major, (a+1)(b+1) <= knn
  int pa[kMaxPairSlots], pb[kMaxPairSlots];
  int npairs = 0;
#pragma unroll
  for (int s = 0; s < kMaxPairSlots; ++s) pa[s] = pb[s] = 0;
  for (int a = 0; a < knn; ++a) {
    const int cnt = knn / (a + 1);
#pragma unroll
    for (int s = 0; s < kMaxPairSlots; ++s) {
      const int slot = 64 * s + lane;
      if (slot >= npairs && slot < npairs + cnt) {
        pa[s] = a;
        pb[s] = slot - npairs;
      }
    }
    npairs += cnt;
  }
  const int NP = (npairs + 63) / 64;

  for (int hc = 0; hc < 2; ++hc) {
    const TIN* Kc = Kt + (int64_t)(2 * h + hc) * n * half;
    // ---- A0: stage the query half [TM][half] (zeros past the last token)
    for (int i = threadIdx.x; i < TM * CH; i += kThreads) {
      const int r = i / CH, c = i - (i / CH) * CH;
      const int64_t t = t0 + r;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (t < Ntok) v = ld16(Q + (t * H + h) * kdim + hc * half + c * EPC);
      QS[r * CH + (c ^ (r & cmask))] = v;
    }
    __syncthreads();

    // ---- A: scores of this wave's column tiles (w, w+8, ...), batches of CB
    float gmax[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 4; ++e) gmax[rt][e] = -__builtin_inff();
    float qn[RT];  // idw: squared norm of query row rt*16 + (lane & 15)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float s = 0.f;
      if (IDW) {
        const int r = rt * 16 + (lane & 15);
        for (int j = 0; j < KS; ++j) {
          const int c = j * 4 + (lane >> 4);
          s += SL::sumsq(QS[r * CH + (c ^ (r & cmask))]);
        }
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
      }
      qn[rt] = s;
    }
    for (int jb = 0;; ++jb) {
      int tile[CB];
      bool tv[CB];
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        tile[k] = w + kWaves * (CB * jb + k);
        tv[k] = tile[k] < ncol;
      }
      if (!tv[0]) break;
      // keys of tiles past the end are read from tile 0 (in range) and their scores dropped
      const uint4* kb[CB];
#pragma unroll
      for (int k = 0; k < CB; ++k)
        kb[k] = (const uint4*)(Kc + (int64_t)(16 * (tv[k] ? tile[k] : 0) + (lane & 15)) * half) + (lane >> 4);
      f32x4_t acc[RT][CB];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int k = 0; k < CB; ++k) acc[rt][k] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      float kn[CB] = {0.f, 0.f, 0.f, 0.f};
      // k-step ks: 16-byte chunk 4*ks + (lane >> 4) of the query and key rows
      auto load_b = [&](uint4* b, int ks) {
#pragma unroll
        for (int k = 0; k < CB; ++k) b[k] = kb[k][4 * ks];
      };
      auto load_a = [&](uint4* a, int ks) {
        const int c = ks * 4 + (lane >> 4);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const int r = rt * 16 + (lane & 15);
          a[rt] = QS[r * CH + (c ^ (r & cmask))];
        }
      };
      auto step = [&](const uint4* a, const uint4* b) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int k = 0; k < CB; ++k) SL::mma(a[rt], b[k], acc[rt][k]);
        if (IDW) {
#pragma unroll
          for (int k = 0; k < CB; ++k) kn[k] += SL::sumsq(b[k]);
        }
      };
      // two k-steps per iteration on ping-pong registers: the key loads for
      // step ks+2 are issued while steps ks+1 runs, with no branch between a
      // load and its use (the clamped loads past the last step are unused)
      // (scheduling barriers keep the loads where they are issued: the
      // scheduler would otherwise sink them next to their use)
      uint4 b0[CB], b1[CB], a0[RT], a1[RT];
      load_b(b0, 0);
      load_b(b1, KS > 1 ? 1 : 0);
      load_a(a0, 0);
      __builtin_amdgcn_sched_barrier(0);
      int ks = 0;
      for (; ks + 1 < KS; ks += 2) {
        load_a(a1, ks + 1);
        __builtin_amdgcn_sched_barrier(0);
        step(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        const int k2 = ks + 2 < KS ? ks + 2 : KS - 1;
        load_b(b0, k2);
        load_a(a0, k2);
        __builtin_amdgcn_sched_barrier(0);
        step(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        load_b(b1, ks + 3 < KS ? ks + 3 : KS - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (ks < KS) step(a0, b0);
      if (IDW) {
#pragma unroll
        for (int k = 0; k < CB; ++k) {
          kn[k] += __shfl_xor(kn[k], 16);
          kn[k] += __shfl_xor(kn[k], 32);  // squared norm of key 16*tile + (lane & 15)
        }
      }
      // epilogue: order keys of the rounded scores into the tile, group maxima
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        if (!tv[k]) continue;
        const int col = 16 * tile[k] + (lane & 15);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int rr = 4 * (lane >> 4) + e;  // row inside the tile
            const int row = rt * 16 + rr;
            float s = acc[rt][k][e];
            if (IDW) {
              float d2 = __shfl(qn[rt], rr) + kn[k] - 2.f * s;
              d2 = d2 > 0.f ? d2 : 0.f;
              s = -logf(1e-3f + d2);
            }
            gmax[rt][e] = s > gmax[rt][e] ? s : gmax[rt][e];
            S[row * n + s_phys(row, col)] = (Store)SL::okey_of(s);
          }
        }
      }
    }
    __syncthreads();  // score tile complete; the query stage is free
    if (16 * w < G) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = rt * 16 + 4 * (lane >> 4) + e;
          GM[row * G + 16 * w + (lane & 15)] = (uint16_t)SL::coarse(SL::okey_of(gmax[rt][e]));
        }
    }
    __syncthreads();

    // ---- B: exact top-knn of each row (and C after the second half)
    TIN* out_s = hc == 0 ? out_s1 : out_s2;
    for (int r = w; r < TM; r += kWaves) {
      const int64_t t = t0 + r;
      if (t >= Ntok) continue;
      const int64_t th = t * H + h;
      const Store* Srow = S + r * n;
      if (out_s != nullptr) {
        for (int col = lane; col < n; col += 64) SL::put(out_s, th * n + col, Srow[s_phys(r, col)]);
      }
      // T0: knn-th largest group maximum
      const uint32_t gk0 = GM[r * G + lane];
      const uint32_t gk1 = G > 64 ? GM[r * G + 64 + lane] : 0u;
      uint32_t T0 = 0;
      for (int bit = 15; bit >= 0; --bit) {
        const uint32_t trial = T0 | (1u << bit);
        uint32_t c = (uint32_t)__popcll(__ballot(gk0 >= trial));
        if (G > 64) c += (uint32_t)__popcll(__ballot(gk1 >= trial));
        if (c >= (uint32_t)knn) T0 = trial;
      }
      // chunks whose maximum reaches T0
      uint32_t nact = 0;
      for (int c = lane; c - lane < NC; c += 64) {
        const bool act = c < NC && SL::chunk_max(Srow + s_phys(r, kChunk * c)) >= T0;
        const uint64_t m = __ballot(act);
        if (act) clist[nact + lanes_below_count(m)] = (uint16_t)c;
        nact += (uint32_t)__popcll(m);
      }
      __builtin_amdgcn_wave_barrier();
      // their scores >= T0, 64 per ballot
      uint32_t total = 0;
      for (uint32_t base = 0; base < nact * kChunk; base += 64) {
        const uint32_t slot = base + lane;
        bool cand = false;
        Key key = 0;
        if (slot < nact * kChunk) {
          const int col = kChunk * clist[slot / kChunk] + (int)(slot % kChunk);
          const uint32_t ok = Srow[s_phys(r, col)];
          cand = SL::coarse(ok) >= T0;
          key = SL::make(ok, (uint32_t)col);
        }
        wave_append(cand, key, scr, total);
      }
      __builtin_amdgcn_wave_barrier();
      Key best;
      if (total <= (uint32_t)kCandCap) {
        best = rank_select(scr, total, knn);
      } else {
        best = exact_topk<Key>([&](int col) { return SL::make(Srow[s_phys(r, col)], (uint32_t)col); }, n, knn, scr);
      }
      const int64_t orow = th * knn;
      if (hc == 0) {
        // park the first half's list in the index output until the cartesian step
        if (lane < knn) out_idx[orow + lane] = (int64_t)best;
        if (out_i1 != nullptr && lane < knn) out_i1[orow + lane] = (int64_t)SL::key_idx(best);
        continue;
      }
      if (out_i2 != nullptr && lane < knn) out_i2[orow + lane] = (int64_t)SL::key_idx(best);

      // ---- C: cartesian top-knn of this token
      const Key l0 = lane < knn ? (Key)out_idx[orow + lane] : (Key)0;
      const Key l1 = best;
      // lower bound of the knn-th pair value: the knn pairs (a, 0) and the knn pairs (0, b)
      const float v0 = SL::value(SL::key_okey(lane_key(l0, 0)));
      const float w0 = SL::value(SL::key_okey(lane_key(l1, 0)));
      const uint32_t ta = SL::okey_of(SL::value(SL::key_okey(lane_key(l0, knn - 1))) + w0);
      const uint32_t tb = SL::okey_of(v0 + SL::value(SL::key_okey(lane_key(l1, knn - 1))));
      const uint32_t Tc = ta > tb ? ta : tb;
      Key keys[kMaxPairSlots];
      uint32_t ctotal = 0;
#pragma unroll
      for (int s = 0; s < kMaxPairSlots; ++s) {
        keys[s] = 0;
        if (s < NP) {
          const Key k0 = shfl_key(l0, pa[s]);
          const Key k1 = shfl_key(l1, pb[s]);
          const uint32_t ok = SL::okey_of(SL::value(SL::key_okey(k0)) + SL::value(SL::key_okey(k1)));
          const bool valid = 64 * s + lane < npairs;
          if (valid) keys[s] = SL::make(ok, (uint32_t)(pa[s] * knn + pb[s]));
          wave_append(valid && ok >= Tc, keys[s], scr, ctotal);
        }
      }
      __builtin_amdgcn_wave_barrier();
      Key top;
      if (ctotal <= (uint32_t)kCandCap) {
        top = rank_select(scr, ctotal, knn);
      } else {
        top = exact_topk<Key>(
            [&](int slot) {
              Key k = 0;
#pragma unroll
              for (int s = 0; s < kMaxPairSlots; ++s)
                if (slot >> 6 == s) k = keys[s];
              return k;
            },
            64 * NP, knn, scr);
      }
      const uint32_t flat = SL::key_idx(top);
      int a = (int)(flat / (uint32_t)knn);
      int b = (int)(flat - (uint32_t)a * (uint32_t)knn);
      a = a < 63 ? a : 63;
      b = b < 63 ? b : 63;
      const uint32_t i0 = SL::key_idx(shfl_key(l0, a));
      const uint32_t i1 = SL::key_idx(shfl_key(l1, b));
      if (lane < knn) {
        SL::put(out_scores, orow + lane, SL::key_okey(top));
        out_idx[orow + lane] = (int64_t)i0 * n + (int64_t)i1;
      }
    }
    __syncthreads();  // before the next half overwrites the score tile and the shared region
  }
}

template <typename TIN, int IDW, int TM>
static int launch_score_tm(const void* q, const void* keys, int64_t Ntok, int H, int n, int half, int knn,
                           size_t lds, int lds_max, void* out_scores, int64_t* out_idx, int64_t* out_i1,
                           int64_t* out_i2, void* out_s1, void* out_s2, hipStream_t st) {
  // Dynamic LDS above 64 KiB is enabled once per device (idempotent, so a
  // race between threads only repeats the call).
  static std::atomic<uint64_t> lds_enabled{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: hipGetDevice failed: %s", hipGetErrorString(e));
  const uint64_t bit = 1ull << (dev & 63);
  if (!(lds_enabled.load(std::memory_order_relaxed) & bit)) {
    e = hipFuncSetAttribute((const void*)pkm_score_topk_kernel<TIN, IDW, TM>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, lds_max);
    if (e != hipSuccess)
      return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
    lds_enabled.fetch_or(bit, std::memory_order_relaxed);
  }
  const int64_t blocks = ((Ntok + TM - 1) / TM) * H;
  hipLaunchKernelGGL((pkm_score_topk_kernel<TIN, IDW, TM>), dim3((unsigned)blocks), dim3(kThreads), lds, st,
                     (const TIN*)q, (const TIN*)keys, Ntok, H, n, half, knn, (TIN*)out_scores, out_idx, out_i1,
                     out_i2, (TIN*)out_s1, (TIN*)out_s2);
  return PKM_OK;
}

template <typename TIN, int IDW>
static int launch_score(int TM, const void* q, const void* keys, int64_t Ntok, int H, int n, int half, int knn,
                        size_t lds, int lds_max, void* out_scores, int64_t* out_idx, int64_t* out_i1,
                        int64_t* out_i2, void* out_s1, void* out_s2, hipStream_t st) {
  switch (TM) {
    case 64:
      return launch_score_tm<TIN, IDW, 64>(q, keys, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx, out_i1,
                                           out_i2, out_s1, out_s2, st);
    case 32:
      return launch_score_tm<TIN, IDW, 32>(q, keys, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx, out_i1,
                                           out_i2, out_s1, out_s2, st);
    default:
      return launch_score_tm<TIN, IDW, 16>(q, keys, Ntok, H, n, half, knn, lds, lds_max, out_scores, out_idx, out_i1,
                                           out_i2, out_s1, out_s2, st);
  }
}

}  // namespace pkm

using namespace pkm;

extern "C" int pkm_score_topk(const void* query, const void* keys, int64_t num_tokens, int64_t heads, int64_t n_keys,
                              int64_t half, int64_t knn, int score_type, int dtype, void* out_scores,
                              int64_t* out_indices, int64_t* out_sub_indices1, int64_t* out_sub_indices2,
                              void* out_sub_scores1, void* out_sub_scores2, void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: dtype %d not supported (float32 and bfloat16 are)", dtype);
  PKM_REQUIRE(score_type == PKM_SCORE_DOT || score_type == PKM_SCORE_IDW, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_topk: bad score type %d", score_type);
  PKM_REQUIRE(num_tokens >= 0 && heads >= 1 && heads < 65536 && n_keys >= 1 && half >= 1 && knn >= 1,
              PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: bad sizes");
  PKM_REQUIRE(knn <= n_keys, PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: knn %lld > n_keys %lld", (long long)knn,
              (long long)n_keys);
  PKM_REQUIRE(knn <= 64 && n_keys % 64 == 0 && n_keys <= kMaxN, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: need knn <= 64 and n_keys a multiple of 64 up to %d (got knn %lld, n_keys %lld)",
              kMaxN, (long long)knn, (long long)n_keys);
  const int kstep = dtype == PKM_DTYPE_BF16 ? Sel<bf16_t>::KSTEP : Sel<float>::KSTEP;
  PKM_REQUIRE(half % kstep == 0, PKM_ERR_UNSUPPORTED, "pkm_score_topk: half key dim %lld must be a multiple of %d",
              (long long)half, kstep);
  if (num_tokens == 0) return PKM_OK;
  PKM_REQUIRE(query && keys && out_scores && out_indices, PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: null pointer");
  PKM_REQUIRE((uintptr_t)query % 16 == 0 && (uintptr_t)keys % 16 == 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_topk: query and keys must be 16-byte aligned");
  const int esz = dtype == PKM_DTYPE_BF16 ? 2 : 4;  // score-tile element = order key of the input dtype
  const int key_bytes = dtype == PKM_DTYPE_BF16 ? 4 : 8;
  int dev = 0, lds_max = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess)
    return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: device query failed: %s", hipGetErrorString(e));
  if (lds_max > kMaxLds) lds_max = kMaxLds;
  int TM = 64;
  while (TM > 16 && score_lds_layout(TM, (int)n_keys, (int)half, esz, key_bytes).total > lds_max) TM /= 2;
  const int lds = score_lds_layout(TM, (int)n_keys, (int)half, esz, key_bytes).total;
  PKM_REQUIRE(lds <= lds_max, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: n_keys %lld / half %lld need %d bytes of LDS, the device allows %d", (long long)n_keys,
              (long long)half, lds, lds_max);
  const int64_t blocks = ((num_tokens + TM - 1) / TM) * heads;
  PKM_REQUIRE(blocks < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: grid too large");
  hipStream_t st = (hipStream_t)stream;
  int rc;
  const int H = (int)heads, n = (int)n_keys, hf = (int)half, k = (int)knn;
  if (dtype == PKM_DTYPE_BF16) {
    rc = score_type == PKM_SCORE_DOT
             ? launch_score<bf16_t, 0>(TM, query, keys, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                       out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                       out_sub_scores2, st)
             : launch_score<bf16_t, 1>(TM, query, keys, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                       out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                       out_sub_scores2, st);
  } else {
    rc = score_type == PKM_SCORE_DOT
             ? launch_score<float, 0>(TM, query, keys, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                      out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                      out_sub_scores2, st)
             : launch_score<float, 1>(TM, query, keys, num_tokens, H, n, hf, k, (size_t)lds, lds_max, out_scores,
                                      out_indices, out_sub_indices1, out_sub_indices2, out_sub_scores1,
                                      out_sub_scores2, st);
  }
  if (rc != PKM_OK) return rc;
  return pkm_check_launch("pkm_score_topk");
}

// Product-key sub-key scoring, per-half top-k and cartesian top-k, gfx950.
//
// For every (token t, head h):
//   s_c[i] = score(q[t, h, c*half:(c+1)*half], keys[(2h+c)*n + i, :])   c = 0, 1; i < n
//            score = dot product, or idw: -log(1e-3 + |q - k|^2)
//   (v_c, i_c) = top-knn of s_c, sorted best first
//   cand[a, c'] = v_0[a] + v_1[c'],  id = i_0[a] * n + i_1[c']
//   (scores, ids) = top-knn of cand, sorted best first
// Reference: HashingMemory.get_indices (pkm/memory.py:250-289) and
// FastWeightProductKeyMemory.get_indices / compute_qk_scores (fwpkm/fwpkm.py:853-934).
// Rounding follows the reference's tensors: sub-scores are stored in the
// input dtype (a bf16 einsum output), the cartesian sums are rounded to it
// again (bf16 + bf16 in ATen), and top-k selects on the rounded values.
// Ties are broken by the smaller index (sub-key index, then flat a*knn + c'),
// which only matters for inputs the reference's topk leaves unspecified.
//
// One workgroup (4 waves) owns TM tokens of one head:
//   A. scores of one half for all n keys on MFMA (16x16x32 bf16 / 16x16x4 f32),
//      rounded and parked in LDS ([TM][n]);
//   B. exact top-knn of each row by one wave: bit-by-bit threshold search with
//      wave ballots, compaction of the selected entries, 64-lane bitonic sort;
//   C. per token, the cartesian candidates restricted to (a+1)(c+1) <= knn —
//      every other pair is dominated by at least knn pairs that precede it in
//      (value, flat index) order, so this is exact, ties included — and the
//      same exact top-knn.
#include <atomic>

#include "pkm_common.h"

namespace pkm {

// Order-preserving map float -> uint32 (a < b  <=>  key(a) < key(b)); key 0 is below every number.
__device__ __forceinline__ uint32_t float_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <typename T>
struct ScoreIO;
template <>
struct ScoreIO<float> {
  static constexpr int LO_BIT = 0;  // all 32 key bits are significant
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float x) { p[i] = x; }
};
template <>
struct ScoreIO<bf16_t> {
  static constexpr int LO_BIT = 16;  // bf16 values: the low 16 bits of the float are zero
  static __device__ __forceinline__ float round(float x) { return bf16_to_f32(f32_to_bf16_bits(x)); }
  static __device__ __forceinline__ float load(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i].x); }
  static __device__ __forceinline__ void store(bf16_t* p, int64_t i, float x) { p[i].x = (uint16_t)f32_to_bf16_bits(x); }
};

// MFMA fragments along k for C[16 x 16] += A[16 x KSTEP] * B[KSTEP x 16]:
// lane l holds row/col l % 16 and the k chunk (l / 16).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  static constexpr int KSTEP = 32;
  typedef uint4 frag;
  static __device__ __forceinline__ frag load(const bf16_t* row, int k0, int lane) {
    return ld16(row + k0 + 8 * (lane >> 4));
  }
  static __device__ __forceinline__ f32x4_t mma(const frag& a, const frag& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  static __device__ __forceinline__ float sumsq(const frag& a) {
    float f[8];
    VecTraits<bf16_t>::unpack(a, f);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = __builtin_fmaf(f[e], f[e], s);
    return s;
  }
};
template <>
struct Mfma<float> {
  static constexpr int KSTEP = 4;
  typedef float frag;
  static __device__ __forceinline__ frag load(const float* row, int k0, int lane) { return row[k0 + (lane >> 4)]; }
  static __device__ __forceinline__ f32x4_t mma(const frag& a, const frag& b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float sumsq(const frag& a) { return a * a; }
};

// 64-lane bitonic sort, best first: larger key, then smaller index.
__device__ __forceinline__ void bitonic64(uint32_t& key, uint32_t& idx) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint32_t pk = (uint32_t)__shfl_xor((int)key, j);
      const uint32_t pi = (uint32_t)__shfl_xor((int)idx, j);
      const bool p_better = pk > key || (pk == key && pi < idx);
      const bool lower = (lane & j) == 0;
      const bool best_first = (lane & k) == 0;
      const bool take = (lower == best_first) ? p_better : !p_better;
      if (take) {
        key = pk;
        idx = pi;
      }
    }
  }
}

// Exact top-knn (knn <= 64) of NV keys per lane. Slot (v, lane) has index
// v * 64 + lane and slots must be ordered like indices (ties go to the smaller
// index). Lane j < knn returns the j-th best (key, slot index); other lanes key 0.
template <int NVMAX>
__device__ __forceinline__ void wave_topk(const uint32_t* key, int NV, int knn, int lo_bit, uint2* scratch,
                                          uint32_t& okey, uint32_t& oslot) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  // Bits below lo_bit carry no order (keys of bf16 values: 0 for positive,
  // all ones for negative values); compare on the masked keys.
  const uint32_t mask = ~((1u << lo_bit) - 1u);
  // T = the largest masked value with at least knn keys >= T
  uint32_t T = 0;
  for (int bit = 31; bit >= lo_bit; --bit) {
    const uint32_t trial = T | (1u << bit);
    uint32_t c = 0;
#pragma unroll
    for (int v = 0; v < NVMAX; ++v)
      if (v < NV) c += (uint32_t)__popcll(__ballot(key[v] >= trial));
    if (c >= (uint32_t)knn) T = trial;
  }
  uint32_t gt = 0;
#pragma unroll
  for (int v = 0; v < NVMAX; ++v)
    if (v < NV) gt += (uint32_t)__popcll(__ballot((key[v] & mask) > T));
  const uint32_t need_eq = (uint32_t)knn - gt;
  // compaction in slot order: every key > T and the first need_eq keys == T
  uint32_t base = 0, eq_seen = 0;
#pragma unroll
  for (int v = 0; v < NVMAX; ++v) {
    if (v < NV) {
      const uint32_t km = key[v] & mask;
      const bool is_gt = km > T, is_eq = km == T;
      const uint64_t me = __ballot(is_eq);
      const bool sel = is_gt || (is_eq && eq_seen + (uint32_t)__popcll(me & below) < need_eq);
      const uint64_t ms = __ballot(sel);
      if (sel) scratch[base + (uint32_t)__popcll(ms & below)] = make_uint2(key[v], (uint32_t)(v * 64 + lane));
      base += (uint32_t)__popcll(ms);
      eq_seen += (uint32_t)__popcll(me);
    }
  }
  __builtin_amdgcn_wave_barrier();
  okey = 0;
  oslot = 0xFFFFFFFFu;
  if (lane < knn) {
    const uint2 e = scratch[lane];
    okey = e.x;
    oslot = e.y;
  }
  __builtin_amdgcn_wave_barrier();
  bitonic64(okey, oslot);
}

constexpr int kMaxNV = 32;  // n <= 2048 keys per half
constexpr int kMaxPairSlots = 5;  // knn = 64 -> 280 candidate pairs
constexpr int kMaxLds = 160 * 1024;  // LDS per CU on gfx950

template <typename TIN, int IDW>
__global__ __launch_bounds__(256) void pkm_score_topk_kernel(const TIN* __restrict__ Q, const TIN* __restrict__ Kt,
                                                             int64_t Ntok, int H, int n, int half, int knn, int TM,
                                                             TIN* __restrict__ out_scores,
                                                             int64_t* __restrict__ out_idx,
                                                             int64_t* __restrict__ out_i1, int64_t* __restrict__ out_i2,
                                                             TIN* __restrict__ out_s1, TIN* __restrict__ out_s2) {
  extern __shared__ __align__(16) unsigned char smem[];
  typedef Mfma<TIN> M;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * TM;
  const int h = blockIdx.y;
  const int kdim = 2 * half;
  TIN* S = (TIN*)smem;  // [TM][n] rounded scores of the current half
  const size_t s_bytes = (((size_t)TM * n * sizeof(TIN)) + 15) & ~(size_t)15;
  uint2* lists = (uint2*)(smem + s_bytes);    // [TM][2][64] (key, sub-key index), best first
  uint2* scratch = lists + (size_t)TM * 2 * 64;  // [4][64]
  uint32_t* pairs = (uint32_t*)(scratch + 4 * 64);  // candidate pairs (a << 16 | c), a-major

  // candidate pair table: all (a, c) with (a + 1) * (c + 1) <= knn
  int npairs = 0;
  for (int a = 0; a < knn; ++a) npairs += knn / (a + 1);
  if (w == 0) {
    const int cnt = lane < knn ? knn / (lane + 1) : 0;
    int x = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    const int off = x - cnt;
    for (int c = 0; c < cnt; ++c) pairs[off + c] = ((uint32_t)lane << 16) | (uint32_t)c;
  }

  const int RT = TM / 16;
  const int ncol = n / 16;
  for (int hc = 0; hc < 2; ++hc) {
    const TIN* Kc = Kt + (int64_t)(2 * h + hc) * n * half;  // [n][half]
    // --- A: scores -> LDS
    float qn[2] = {0.f, 0.f};  // squared norms of rows (lane % 16) of row tiles 0, 1 (idw)
    if (IDW) {
      for (int r = 0; r < RT; ++r) {
        const int64_t t = t0 + r * 16 + (lane & 15);
        float s = 0.f;
        if (t < Ntok) {
          const TIN* qrow = Q + (t * H + h) * kdim + hc * half;
          for (int k0 = 0; k0 < half; k0 += M::KSTEP) s += M::sumsq(M::load(qrow, k0, lane));
        }
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        qn[r] = s;
      }
    }
    for (int j = w; j < ncol; j += 4) {
      const TIN* krow = Kc + (int64_t)(j * 16 + (lane & 15)) * half;
      f32x4_t acc[2];
      acc[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      float kn = 0.f;
      for (int k0 = 0; k0 < half; k0 += M::KSTEP) {
        const typename M::frag b = M::load(krow, k0, lane);
        if (IDW) kn += M::sumsq(b);
        for (int r = 0; r < RT; ++r) {
          const int64_t t = t0 + r * 16 + (lane & 15);
          typename M::frag a;
          if (t < Ntok)
            a = M::load(Q + (t * H + h) * kdim + hc * half, k0, lane);
          else
            a = typename M::frag{};
          acc[r] = M::mma(a, b, acc[r]);
        }
      }
      if (IDW) {
        kn += __shfl_xor(kn, 16);
        kn += __shfl_xor(kn, 32);  // every lane: norm of key (lane % 16) = its C column
      }
      const int col = j * 16 + (lane & 15);
      for (int r = 0; r < RT; ++r) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 4 * (lane >> 4) + e;  // row inside the tile
          float s = acc[r][e];
          if (IDW) {
            const float qrow_n = __shfl(qn[r], row);
            float d2 = qrow_n + kn - 2.f * s;
            d2 = d2 > 0.f ? d2 : 0.f;
            s = -logf(1e-3f + d2);
          }
          ScoreIO<TIN>::store(S, (int64_t)(r * 16 + row) * n + col, s);
        }
      }
    }
    __syncthreads();
    // full sub-scores, when asked for (fast-weight PKM returns them)
    TIN* out_s = hc == 0 ? out_s1 : out_s2;
    if (out_s != nullptr) {
      for (int idx = threadIdx.x; idx < TM * n; idx += 256) {
        const int r = idx / n, col = idx - (idx / n) * n;
        const int64_t t = t0 + r;
        if (t < Ntok) out_s[(t * H + h) * n + col] = S[idx];
      }
    }
    // --- B: exact top-knn of every row
    const int NV = n / 64;
    for (int r = w; r < TM; r += 4) {
      if (t0 + r >= Ntok) continue;
      uint32_t key[kMaxNV];
#pragma unroll
      for (int v = 0; v < kMaxNV; ++v)
        key[v] = v < NV ? float_key(ScoreIO<TIN>::load(S, (int64_t)r * n + v * 64 + lane)) : 0u;
      uint32_t okey, oslot;
      wave_topk<kMaxNV>(key, NV, knn, ScoreIO<TIN>::LO_BIT, scratch + w * 64, okey, oslot);
      if (lane < knn) lists[((size_t)r * 2 + hc) * 64 + lane] = make_uint2(okey, oslot);
    }
    __syncthreads();
  }

  // --- C: cartesian top-knn per token
  for (int r = w; r < TM; r += 4) {
    const int64_t t = t0 + r;
    if (t >= Ntok) continue;
    const uint2* L1 = lists + ((size_t)r * 2 + 0) * 64;
    const uint2* L2 = lists + ((size_t)r * 2 + 1) * 64;
    uint32_t key[kMaxPairSlots];
    const int NP = (npairs + 63) / 64;
#pragma unroll
    for (int v = 0; v < kMaxPairSlots; ++v) {
      key[v] = 0u;
      const int s = v * 64 + lane;
      if (v < NP && s < npairs) {
        const uint32_t pr = pairs[s];
        const float v1 = key_float(L1[pr >> 16].x), v2 = key_float(L2[pr & 0xFFFFu].x);
        key[v] = float_key(ScoreIO<TIN>::round(v1 + v2));
      }
    }
    uint32_t okey, oslot;
    wave_topk<kMaxPairSlots>(key, NP, knn, ScoreIO<TIN>::LO_BIT, scratch + w * 64, okey, oslot);
    const int64_t orow = (t * H + h) * knn;
    if (lane < knn) {
      const uint32_t pr = pairs[oslot < (uint32_t)npairs ? oslot : 0u];
      const uint32_t a = pr >> 16, c = pr & 0xFFFFu;
      ScoreIO<TIN>::store(out_scores, orow + lane, key_float(okey));
      out_idx[orow + lane] = (int64_t)L1[a].y * n + (int64_t)L2[c].y;
      if (out_i1 != nullptr) out_i1[orow + lane] = (int64_t)L1[lane].y;
      if (out_i2 != nullptr) out_i2[orow + lane] = (int64_t)L2[lane].y;
    }
  }
}

static size_t score_lds_bytes(int TM, int n, int esz) {
  const size_t s_bytes = (((size_t)TM * n * esz) + 15) & ~(size_t)15;
  return s_bytes + (size_t)TM * 2 * 64 * 8 + 4 * 64 * 8 + 64 * kMaxPairSlots * 4;
}

template <typename TIN, int IDW>
static int launch_score(const void* q, const void* keys, int64_t Ntok, int H, int n, int half, int knn, int TM,
                        void* out_scores, int64_t* out_idx, int64_t* out_i1, int64_t* out_i2, void* out_s1,
                        void* out_s2, hipStream_t st) {
  const size_t lds = score_lds_bytes(TM, n, (int)sizeof(TIN));
  // Dynamic LDS above 64 KiB is enabled once per device (idempotent, so a
  // race between threads only repeats the call).
  static std::atomic<uint64_t> lds_enabled{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: hipGetDevice failed: %s", hipGetErrorString(e));
  const uint64_t bit = 1ull << (dev & 63);
  if (!(lds_enabled.load(std::memory_order_relaxed) & bit)) {
    e = hipFuncSetAttribute((const void*)pkm_score_topk_kernel<TIN, IDW>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            kMaxLds);
    if (e != hipSuccess)
      return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
    lds_enabled.fetch_or(bit, std::memory_order_relaxed);
  }
  const dim3 grid((unsigned)((Ntok + TM - 1) / TM), (unsigned)H);
  hipLaunchKernelGGL((pkm_score_topk_kernel<TIN, IDW>), grid, dim3(256), lds, st, (const TIN*)q, (const TIN*)keys,
                     Ntok, H, n, half, knn, TM, (TIN*)out_scores, out_idx, out_i1, out_i2, (TIN*)out_s1,
                     (TIN*)out_s2);
  return PKM_OK;
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
  PKM_REQUIRE(knn <= 64 && n_keys % 64 == 0 && n_keys <= 64 * kMaxNV, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: need knn <= 64 and n_keys a multiple of 64 up to %d (got knn %lld, n_keys %lld)",
              64 * kMaxNV, (long long)knn, (long long)n_keys);
  const int kstep = dtype == PKM_DTYPE_BF16 ? 32 : 4;
  PKM_REQUIRE(half % kstep == 0, PKM_ERR_UNSUPPORTED, "pkm_score_topk: half key dim %lld must be a multiple of %d",
              (long long)half, kstep);
  if (num_tokens == 0) return PKM_OK;
  PKM_REQUIRE(query && keys && out_scores && out_indices, PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: null pointer");
  PKM_REQUIRE((uintptr_t)query % 16 == 0 && (uintptr_t)keys % 16 == 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_topk: query and keys must be 16-byte aligned");
  const int esz = dtype == PKM_DTYPE_BF16 ? 2 : 4;
  int dev = 0, lds_max = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess)
    return pkm_set_error(PKM_ERR_HIP, "pkm_score_topk: device query failed: %s", hipGetErrorString(e));
  if (lds_max > kMaxLds) lds_max = kMaxLds;
  int TM = 32;
  if (score_lds_bytes(TM, (int)n_keys, esz) > (size_t)lds_max) TM = 16;
  PKM_REQUIRE(score_lds_bytes(TM, (int)n_keys, esz) <= (size_t)lds_max, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: n_keys %lld needs %zu bytes of LDS, the device allows %d", (long long)n_keys,
              score_lds_bytes(TM, (int)n_keys, esz), lds_max);
  hipStream_t st = (hipStream_t)stream;
  int rc;
  const int H = (int)heads, n = (int)n_keys, hf = (int)half, k = (int)knn;
  if (dtype == PKM_DTYPE_BF16) {
    rc = score_type == PKM_SCORE_DOT
             ? launch_score<bf16_t, 0>(query, keys, num_tokens, H, n, hf, k, TM, out_scores, out_indices,
                                       out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, st)
             : launch_score<bf16_t, 1>(query, keys, num_tokens, H, n, hf, k, TM, out_scores, out_indices,
                                       out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, st);
  } else {
    rc = score_type == PKM_SCORE_DOT
             ? launch_score<float, 0>(query, keys, num_tokens, H, n, hf, k, TM, out_scores, out_indices,
                                      out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, st)
             : launch_score<float, 1>(query, keys, num_tokens, H, n, hf, k, TM, out_scores, out_indices,
                                      out_sub_indices1, out_sub_indices2, out_sub_scores1, out_sub_scores2, st);
  }
  if (rc != PKM_OK) return rc;
  return pkm_check_launch("pkm_score_topk");
}

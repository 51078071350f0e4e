// Product-key retrieval for the shapes the tuned kernels of score_topk.hip do
// not take, gfx950: any n_keys (up to 16384), any knn <= n_keys (up to 1024),
// any half key width, float32 / bfloat16 / float16 (HashingMemory.get_indices,
// pkm/memory.py:250-289; FastWeightProductKeyMemory.get_indices,
// fwpkm/fwpkm.py:853-934).
//
// One workgroup of 256 threads owns TM tokens of one head (TM from the LDS
// budget, at most 16), so each key row staged into LDS serves TM tokens.
//   1. per half: the TM x n sub-scores (float32 dot products in dimension
//      order, or idw), rounded to the dtype, as order keys in LDS (and to the
//      sub-score outputs);
//   2. per token and half: the top-knn by a radix select of the order keys
//      (4 passes of 8-bit digits), ties taken in sub-key order, then a
//      bitonic sort of the knn (order key, ~index) pairs: best first, equal
//      scores by the smaller sub-key;
//   3. per token: the (a + 1)(b + 1) <= knn pairs of the two lists (the only
//      ones that can reach the top-knn), enumerated a-major, scored
//      dtype(v1[a] + v2[b]), selected and sorted the same way (ties by the
//      smaller a * knn + b).
// Same results as the tuned kernels (the documented tie order included);
// slower, as the scores run on the vector ALUs from LDS.
#include "pkm_common.h"

namespace pkm {
namespace gen {

constexpr int kThreads = 256;
constexpr int kKC = 32;         // key rows per staged chunk
constexpr int kMaxTM = 16;      // tokens per workgroup
constexpr int kMaxN = 16384;    // n_keys limit
constexpr int kMaxKnn = 1024;   // knn limit

__device__ __forceinline__ uint32_t okey32(float f) {
  const uint32_t u = __float_as_uint(f + 0.0f);  // -0 counts as +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_okey32(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ float round_dt(float v, int dt) {
  return dt == PKM_DTYPE_F32 ? v : (dt == PKM_DTYPE_BF16 ? round_to<bf16_t>(v) : round_to<f16_t>(v));
}

// Exclusive prefix sum over the 256 threads; *total gets the sum.
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* scratch, uint32_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = (uint32_t)__shfl_up((int)x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pre += i < w ? scratch[i] : 0u;
    tot += scratch[i];
  }
  __syncthreads();
  *total = tot;
  return pre + x - v;
}

// The K largest of the order keys S[0, m) with ties in position order, as
// (key << 32) | (0xFFFFFFFF - position) in sel[0, K), unordered.
__device__ void select_topk(const uint32_t* S, int m, int K, uint64_t* sel, uint32_t* hist, uint32_t* sh) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0, need = (uint32_t)K;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < m; i += kThreads) {
      const uint32_t k = S[i];
      if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t cum = 0;
      int d = 255;
      for (; d > 0; --d) {
        if (cum + hist[d] >= need) break;
        cum += hist[d];
      }
      sh[0] = (uint32_t)d;
      sh[1] = need - cum;
    }
    __syncthreads();
    prefix |= sh[0] << shift;
    mask |= 0xFFu << shift;
    need = sh[1];
    __syncthreads();
  }
  // prefix = T, the K-th largest key: all keys > T, then the first `need` equal to T
  const uint32_t T = prefix;
  const int per = (m + kThreads - 1) / kThreads;
  const int i0 = tid * per, i1 = i0 + per < m ? i0 + per : m;
  uint32_t gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t k = S[i];
    gt += k > T ? 1u : 0u;
    eq += k == T ? 1u : 0u;
  }
  uint32_t tot_gt, tot_eq;
  uint32_t o_gt = block_scan(gt, sh + 4, &tot_gt);
  uint32_t o_eq = block_scan(eq, sh + 4, &tot_eq);
  for (int i = i0; i < i1; ++i) {
    const uint32_t k = S[i];
    const uint64_t v = ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
    if (k > T) {
      sel[o_gt++] = v;
    } else if (k == T) {
      if (o_eq < need) sel[tot_gt + o_eq] = v;
      ++o_eq;
    }
  }
  __syncthreads();
}

// Bitonic sort of A[0, len), len a power of two, largest first.
__device__ void sort_desc(uint64_t* A, int len) {
  for (int k = 2; k <= len; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < len; i += kThreads) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t a = A[i], b = A[p];
          const bool desc = (i & k) == 0;
          if (desc ? a < b : a > b) {
            A[i] = b;
            A[p] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// first a with coff[a + 1] > j (coff[0] = 0, increasing over a < knn)
__device__ __forceinline__ int pair_row(const uint32_t* coff, int knn, uint32_t j) {
  int lo = 0, hi = knn - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (coff[mid] <= j)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

struct Layout {
  size_t S, L, Lout, coff, qs, ks, qn, kn, hist, sh, total;
};

__host__ __device__ inline size_t al16(size_t x) { return (x + 15) & ~(size_t)15; }

__host__ __device__ inline int pair_total(int knn) {
  int m = 0;
  for (int a = 0; a < knn; ++a) m += knn / (a + 1) < knn ? knn / (a + 1) : knn;
  return m;
}

__host__ __device__ inline Layout layout(int TM, int n, int half, int knn, int kpad) {
  Layout l;
  size_t off = 0;
  const int M = pair_total(knn);
  const size_t s_words = (size_t)TM * n > (size_t)M ? (size_t)TM * n : (size_t)M;
  l.S = off;
  off = al16(off + s_words * 4);
  l.L = off;
  off = al16(off + (size_t)2 * TM * kpad * 8);
  l.Lout = off;
  off = al16(off + (size_t)kpad * 8);
  l.coff = off;
  off = al16(off + (size_t)(knn + 1) * 4);
  l.qs = off;
  off = al16(off + (size_t)TM * half * 4);
  l.ks = off;
  off = al16(off + (size_t)kKC * (half + 1) * 4);
  l.qn = off;
  off = al16(off + (size_t)TM * 4);
  l.kn = off;
  off = al16(off + (size_t)kKC * 4);
  l.hist = off;
  off = al16(off + 256 * 4);
  l.sh = off;
  off = al16(off + 16 * 4);
  l.total = off;
  return l;
}

__global__ __launch_bounds__(kThreads) void pkm_score_generic_kernel(
    const void* __restrict__ query, const void* __restrict__ keys, int dt, int64_t Ntok, int H, int n, int half,
    int knn, int kpad, int TM, int idw, void* __restrict__ out_scores, int64_t* __restrict__ out_idx,
    int64_t* __restrict__ out_i1, int64_t* __restrict__ out_i2, void* __restrict__ out_s1,
    void* __restrict__ out_s2) {
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout l = layout(TM, n, half, knn, kpad);
  uint32_t* S = (uint32_t*)(smem + l.S);
  uint64_t* Lst = (uint64_t*)(smem + l.L);  // [2][TM][kpad]
  uint64_t* Lout = (uint64_t*)(smem + l.Lout);
  uint32_t* coff = (uint32_t*)(smem + l.coff);
  float* qs = (float*)(smem + l.qs);  // [TM][half]
  float* ks = (float*)(smem + l.ks);  // [kKC][half + 1]
  float* qn = (float*)(smem + l.qn);
  float* kn = (float*)(smem + l.kn);
  uint32_t* hist = (uint32_t*)(smem + l.hist);
  uint32_t* sh = (uint32_t*)(smem + l.sh);
  const int tid = threadIdx.x;
  const int h = (int)(blockIdx.x % (unsigned)H);
  const int64_t t0 = (int64_t)(blockIdx.x / (unsigned)H) * TM;
  const int nt = (int)(Ntok - t0 < TM ? Ntok - t0 : TM);
  const int ks_stride = half + 1;  // padded rows: the threads of a dot step read distinct banks

  for (int c = 0; c < 2; ++c) {
    for (int e = tid; e < TM * half; e += kThreads) {
      const int t = e / half, d = e - (e / half) * half;
      qs[e] = t < nt ? load_scalar(query, dt, ((t0 + t) * H + h) * 2 * half + (int64_t)c * half + d) : 0.f;
    }
    __syncthreads();
    if (idw && tid < TM) {
      float s = 0.f;
      for (int d = 0; d < half; ++d) s = __builtin_fmaf(qs[tid * half + d], qs[tid * half + d], s);
      qn[tid] = s;
    }
    void* out_s = c == 0 ? out_s1 : out_s2;
    for (int i0 = 0; i0 < n; i0 += kKC) {
      const int kc = n - i0 < kKC ? n - i0 : kKC;
      const int64_t kbase = ((int64_t)(2 * h + c) * n + i0) * half;
      for (int e = tid; e < kc * half; e += kThreads) {
        const int r = e / half, d = e - (e / half) * half;
        ks[r * ks_stride + d] = load_scalar(keys, dt, kbase + e);
      }
      __syncthreads();
      if (idw && tid < kc) {
        float s = 0.f;
        for (int d = 0; d < half; ++d) s = __builtin_fmaf(ks[tid * ks_stride + d], ks[tid * ks_stride + d], s);
        kn[tid] = s;
      }
      __syncthreads();
      for (int p = tid; p < TM * kc; p += kThreads) {
        const int t = p / kc, r = p - (p / kc) * kc;
        const float* qr = qs + t * half;
        const float* kr = ks + r * ks_stride;
        float dot = 0.f;
        for (int d = 0; d < half; ++d) dot = __builtin_fmaf(qr[d], kr[d], dot);
        float s = dot;
        if (idw) {
          float d2 = qn[t] + kn[r] - 2.f * dot;
          d2 = d2 > 0.f ? d2 : 0.f;
          s = -logf(1e-3f + d2);
        }
        const float sr = round_dt(s, dt);
        S[t * n + i0 + r] = okey32(sr);
        if (out_s != nullptr && t < nt) store_scalar(out_s, dt, ((t0 + t) * H + h) * n + i0 + r, sr);
      }
      __syncthreads();
    }
    int64_t* out_ic = c == 0 ? out_i1 : out_i2;
    for (int t = 0; t < nt; ++t) {
      uint64_t* L = Lst + ((size_t)c * TM + t) * kpad;
      select_topk(S + t * n, n, knn, L, hist, sh);
      for (int j = knn + tid; j < kpad; j += kThreads) L[j] = 0ull;
      __syncthreads();
      sort_desc(L, kpad);
      if (out_ic != nullptr)
        for (int j = tid; j < knn; j += kThreads)
          out_ic[((t0 + t) * H + h) * knn + j] = (int64_t)(0xFFFFFFFFu - (uint32_t)L[j]);
      __syncthreads();
    }
  }

  // cartesian: the (a + 1)(b + 1) <= knn pairs, a-major
  if (tid == 0) {
    uint32_t run = 0;
    for (int a = 0; a < knn; ++a) {
      coff[a] = run;
      run += (uint32_t)(knn / (a + 1) < knn ? knn / (a + 1) : knn);
    }
    coff[knn] = run;
  }
  __syncthreads();
  const uint32_t M = coff[knn];
  for (int t = 0; t < nt; ++t) {
    const uint64_t* L1 = Lst + (size_t)t * kpad;
    const uint64_t* L2 = Lst + ((size_t)TM + t) * kpad;
    for (uint32_t j = tid; j < M; j += kThreads) {
      const int a = pair_row(coff, knn, j);
      const int b = (int)(j - coff[a]);
      const float v = from_okey32((uint32_t)(L1[a] >> 32)) + from_okey32((uint32_t)(L2[b] >> 32));
      S[j] = okey32(round_dt(v, dt));
    }
    __syncthreads();
    select_topk(S, (int)M, knn, Lout, hist, sh);
    for (int j = knn + tid; j < kpad; j += kThreads) Lout[j] = 0ull;
    __syncthreads();
    sort_desc(Lout, kpad);
    const int64_t row = (t0 + t) * H + h;
    for (int j = tid; j < knn; j += kThreads) {
      const uint64_t v = Lout[j];
      const uint32_t pos = 0xFFFFFFFFu - (uint32_t)v;
      const int a = pair_row(coff, knn, pos);
      const int b = (int)(pos - coff[a]);
      const int64_t i1 = (int64_t)(0xFFFFFFFFu - (uint32_t)L1[a]);
      const int64_t i2 = (int64_t)(0xFFFFFFFFu - (uint32_t)L2[b]);
      out_idx[row * knn + j] = i1 * n + i2;
      store_scalar(out_scores, dt, row * knn + j, from_okey32((uint32_t)(v >> 32)));
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Dense sub-score gradient for any n_keys and knn (pkm_score_grad_dense's
// semantics): one wave per (token, head) row; the two gradient rows of the
// row live in LDS, lane 0 adds the selected scores' gradients in j order,
// then the dense upstream gradients are added and the rows written out.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void score_grad_dense_generic_kernel(const int64_t* __restrict__ idx,
                                                                      const void* __restrict__ d, int dt, int64_t NH,
                                                                      int H, int n, int knn,
                                                                      const void* __restrict__ dsub0,
                                                                      const void* __restrict__ dsub1,
                                                                      void* __restrict__ dS, int64_t Ntok) {
  extern __shared__ __align__(16) float rows[];  // [2][n]
  const int lane = threadIdx.x;
  const int64_t th = blockIdx.x;
  const int64_t t = th / H;
  const int h = (int)(th - t * H);
  for (int i = lane; i < 2 * n; i += 64) rows[i] = 0.f;
  __syncthreads();
  if (lane == 0) {
    for (int j = 0; j < knn; ++j) {
      const int64_t id = idx[th * knn + j];
      if (id < 0 || id >= (int64_t)n * n) continue;
      const float v = load_scalar(d, dt, th * knn + j);
      const int a = (int)(id / n), b = (int)(id - (id / n) * n);
      rows[a] += v;
      rows[n + b] += v;
    }
  }
  __syncthreads();
  for (int c = 0; c < 2; ++c) {
    const void* ds = c == 0 ? dsub0 : dsub1;
    const int64_t obase = (((int64_t)h * 2 + c) * Ntok + t) * n;
    for (int i = lane; i < n; i += 64) {
      float v = rows[c * n + i];
      if (ds != nullptr) v += load_scalar(ds, dt, th * n + i);
      store_scalar(dS, dt, obase + i, v);
    }
  }
}

}  // namespace gen

// Host side, called from score_topk.hip / score_grad.hip for the shapes their
// tuned kernels do not take.
int score_topk_generic(const void* query, const void* keys, int64_t num_tokens, int64_t heads, int64_t n_keys,
                       int64_t half, int64_t knn, int score_type, int dtype, void* out_scores, int64_t* out_indices,
                       int64_t* out_i1, int64_t* out_i2, void* out_s1, void* out_s2, int lds_max, hipStream_t st) {
  PKM_REQUIRE(n_keys <= gen::kMaxN && knn <= gen::kMaxKnn, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: n_keys %lld (up to %d) and knn %lld (up to %d) not supported", (long long)n_keys,
              gen::kMaxN, (long long)knn, gen::kMaxKnn);
  int kpad = 1;
  while (kpad < knn) kpad <<= 1;
  int TM = gen::kMaxTM;
  while (TM > 1 && (int)gen::layout(TM, (int)n_keys, (int)half, (int)knn, kpad).total > lds_max) TM >>= 1;
  const size_t lds = gen::layout(TM, (int)n_keys, (int)half, (int)knn, kpad).total;
  PKM_REQUIRE((int)lds <= lds_max, PKM_ERR_UNSUPPORTED,
              "pkm_score_topk: n_keys %lld, half %lld and knn %lld need %zu bytes of LDS, the device allows %d",
              (long long)n_keys, (long long)half, (long long)knn, lds, lds_max);
  const int64_t blocks = ((num_tokens + TM - 1) / TM) * heads;
  PKM_REQUIRE(blocks < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_topk: grid too large");
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)gen::pkm_score_generic_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds_max);
    PKM_REQUIRE(e == hipSuccess, PKM_ERR_HIP, "pkm_score_topk: LDS limit: %s", hipGetErrorString(e));
    attr_set = true;
  }
  hipLaunchKernelGGL(gen::pkm_score_generic_kernel, dim3((unsigned)blocks), dim3(gen::kThreads), lds, st, query, keys,
                     dtype, num_tokens, (int)heads, (int)n_keys, (int)half, (int)knn, kpad, TM,
                     score_type == PKM_SCORE_IDW ? 1 : 0, out_scores, out_indices, out_i1, out_i2, out_s1, out_s2);
  return PKM_OK;
}

int score_grad_dense_generic(const int64_t* indices, const void* d_scores, int dtype, int64_t num_tokens,
                             int64_t heads, int64_t n_keys, int64_t knn, const void* d_sub1, const void* d_sub2,
                             void* d_sub_dense, int lds_max, hipStream_t st) {
  const size_t lds = (size_t)2 * n_keys * sizeof(float);
  PKM_REQUIRE((int)lds <= lds_max, PKM_ERR_UNSUPPORTED, "pkm_score_grad_dense: n_keys %lld too large",
              (long long)n_keys);
  const int64_t NH = num_tokens * heads;
  PKM_REQUIRE(NH < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_dense: too many rows");
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)gen::score_grad_dense_generic_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds_max);
    PKM_REQUIRE(e == hipSuccess, PKM_ERR_HIP, "pkm_score_grad_dense: LDS limit: %s", hipGetErrorString(e));
    attr_set = true;
  }
  hipLaunchKernelGGL(gen::score_grad_dense_generic_kernel, dim3((unsigned)NH), dim3(64), lds, st, indices, d_scores,
                     dtype, NH, (int)heads, (int)n_keys, (int)knn, d_sub1, d_sub2, d_sub_dense, num_tokens);
  return PKM_OK;
}

}  // namespace pkm

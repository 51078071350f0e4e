// Dense gradient of the sub-key scores from the product-key top-k gradient, gfx950.
//
// For every (token t, head h) with selected ids idx[t,h,j] = i_0 * n + i_1 and
// upstream gradient d[t,h,j] of the selected scores (scores = s_0[i_0] + s_1[i_1]):
//   dS[h, c, t, i] = sum_{j : i_c(idx[t,h,j]) == i} d[t,h,j]   (+ d_sub_c[t, h, i])
// for c = 0, 1 and all i < n, in float32 (j ascending), rounded once to dtype.
// The layout [heads, 2, tokens, n_keys] makes dS[h, c] the left operand of the
// per-(head, half) products dq = dS @ K_c and dK_c = dS^T @ q_c.
// Reference: autograd of memory.py:267-285 / fwpkm.py:904-921 — the gradient
// of topk + gather + expand-add w.r.t. the full sub-score matrices.
//
// One wave per (t, h): lane j < knn holds its pair (i_0, i_1, d); each lane
// sums d over the lanes with the same sub-key (broadcast loop in j order) and
// the first such lane writes the sum into an LDS row of zeros, which is then
// copied out with vector stores (the dense upstream gradient added on the way).
// Ids outside [0, n*n) are ignored.
#include "pkm_common.h"

namespace pkm {

constexpr int kGradWaves = 4;
constexpr int kGradMaxN = 2048;

template <typename T>
struct GradIO;
template <>
struct GradIO<float> {
  static __device__ __forceinline__ void load4(const float* p, float* v) {
    const float4 x = *(const float4*)p;
    v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
  }
  static __device__ __forceinline__ float load1(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store4(float* p, const float* v) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <>
struct GradIO<bf16_t> {
  static __device__ __forceinline__ void load4(const bf16_t* p, float* v) {
    const uint2 x = *(const uint2*)p;
    v[0] = __uint_as_float(x.x << 16), v[1] = __uint_as_float(x.x & 0xffff0000u);
    v[2] = __uint_as_float(x.y << 16), v[3] = __uint_as_float(x.y & 0xffff0000u);
  }
  static __device__ __forceinline__ float load1(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i].x); }
  static __device__ __forceinline__ void store4(bf16_t* p, const float* v) {
    *(uint2*)p = make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
  }
};

template <typename T>
__global__ __launch_bounds__(64 * kGradWaves) void score_grad_dense_kernel(
    const int64_t* __restrict__ idx, const T* __restrict__ d, int64_t NH, int H, int n, int knn,
    const T* __restrict__ dsub0, const T* __restrict__ dsub1, T* __restrict__ dS, int64_t Ntok) {
  extern __shared__ __align__(16) float rowbuf[];  // [kGradWaves][2][n]
  typedef GradIO<T> IO;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t th = (int64_t)blockIdx.x * kGradWaves + w;
  if (th >= NH) return;  // whole wave leaves; no block barrier follows
  const int64_t t = th / H;
  const int h = (int)(th - t * H);
  float* row0 = rowbuf + (int64_t)w * 2 * n;
  float* row1 = row0 + n;
  for (int i = lane * 4; i < n; i += 256) {
    *(float4*)(row0 + i) = make_float4(0.f, 0.f, 0.f, 0.f);
    *(float4*)(row1 + i) = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  int a = -1, b = -1;
  float dv = 0.f;
  if (lane < knn) {
    const int64_t id = idx[th * knn + lane];
    if (id >= 0 && id < (int64_t)n * n) {
      a = (int)(id / n);
      b = (int)(id - (int64_t)a * n);
      dv = IO::load1(d, th * knn + lane);
    }
  }
  // per lane: sums over the lanes sharing its sub-key, in lane order
  float s0 = 0.f, s1 = 0.f;
  bool first0 = true, first1 = true;
  for (int j = 0; j < knn; ++j) {
    const int aj = __builtin_amdgcn_readlane(a, j);
    const int bj = __builtin_amdgcn_readlane(b, j);
    const float dj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dv), j));
    if (aj == a) {
      s0 += dj;
      if (j < lane) first0 = false;
    }
    if (bj == b) {
      s1 += dj;
      if (j < lane) first1 = false;
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (a >= 0 && first0) row0[a] = s0;
  if (b >= 0 && first1) row1[b] = s1;
  __builtin_amdgcn_wave_barrier();
  T* out0 = dS + ((int64_t)(2 * h) * Ntok + t) * n;
  T* out1 = dS + ((int64_t)(2 * h + 1) * Ntok + t) * n;
  const int64_t sub = th * n;
  for (int i = lane * 4; i < n; i += 256) {
    float v0[4], v1[4], u[4];
    const float4 x0 = *(const float4*)(row0 + i), x1 = *(const float4*)(row1 + i);
    v0[0] = x0.x, v0[1] = x0.y, v0[2] = x0.z, v0[3] = x0.w;
    v1[0] = x1.x, v1[1] = x1.y, v1[2] = x1.z, v1[3] = x1.w;
    if (dsub0 != nullptr) {
      IO::load4(dsub0 + sub + i, u);
#pragma unroll
      for (int e = 0; e < 4; ++e) v0[e] += u[e];
    }
    if (dsub1 != nullptr) {
      IO::load4(dsub1 + sub + i, u);
#pragma unroll
      for (int e = 0; e < 4; ++e) v1[e] += u[e];
    }
    IO::store4(out0 + i, v0);
    IO::store4(out1 + i, v1);
  }
}

// ---------------------------------------------------------------------------
// Sparse score backward (dot scores, bf16): dq = dS_c @ K_c and
// dK_c = dS_c^T @ q_c on MFMA without materialising dS. Each row of dS_c has
// at most knn nonzeros (the selected pairs' sub-keys); they are listed per
// (t, h, c), and every MFMA tile of dS is built in LDS from the lists.
// ---------------------------------------------------------------------------
typedef __bf16 sg_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float sg_f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void sg_mma(const uint4& a, const uint4& b, sg_f32x4_t& c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sg_bf16x8_t, a), __builtin_bit_cast(sg_bf16x8_t, b),
                                              c, 0, 0, 0);
}

constexpr uint32_t kNoEntry = 0xFFFFFFFFu;  // unused list slot
constexpr int kSgRows = 128;                // output rows per workgroup (tokens for dq, keys for dk)
constexpr int kSgChunk = 64;                // reduction chunk (keys for dq, tokens for dk)
constexpr int kSgLd = kSgChunk + 8;         // LDS row pitch in bf16 (16-byte pad: distinct banks per row)
constexpr int kSgMaxHalf = 256;             // dims per half: 4 waves x 64
constexpr int kSgThreads = 512;             // 8 waves: 2 (rows, 64 each) x 4 (dims, 64 each)

// Per (t, h, c): slot j holds (sub-key << 16) | bf16(sum of d over the pairs
// j' with the same sub-key, float32 in j' order) for the first such j, else
// kNoEntry: the nonzeros of dS_c[t, :] (the dense kernel's values).
__global__ __launch_bounds__(64 * kGradWaves) void score_grad_lists_kernel(const int64_t* __restrict__ idx,
                                                                           const bf16_t* __restrict__ d, int64_t NH,
                                                                           int n, int knn,
                                                                           uint32_t* __restrict__ lists) {
  const int lane = threadIdx.x & 63;
  const int64_t th = (int64_t)blockIdx.x * kGradWaves + (threadIdx.x >> 6);
  if (th >= NH) return;
  int a = -1, b = -1;
  float dv = 0.f;
  if (lane < knn) {
    const int64_t id = idx[th * knn + lane];
    if (id >= 0 && id < (int64_t)n * n) {
      a = (int)(id / n);
      b = (int)(id - (int64_t)a * n);
      dv = bf16_to_f32(d[th * knn + lane].x);
    }
  }
  float s0 = 0.f, s1 = 0.f;
  bool first0 = true, first1 = true;
  for (int j = 0; j < knn; ++j) {
    const int aj = __builtin_amdgcn_readlane(a, j);
    const int bj = __builtin_amdgcn_readlane(b, j);
    const float dj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dv), j));
    if (aj == a) {
      s0 += dj;
      if (j < lane) first0 = false;
    }
    if (bj == b) {
      s1 += dj;
      if (j < lane) first1 = false;
    }
  }
  if (lane < knn) {
    lists[(th * 2 + 0) * knn + lane] = (a >= 0 && first0) ? (((uint32_t)a << 16) | f32_to_bf16_bits(s0)) : kNoEntry;
    lists[(th * 2 + 1) * knn + lane] = (b >= 0 && first1) ? (((uint32_t)b << 16) | f32_to_bf16_bits(s1)) : kNoEntry;
  }
}

// Kt[hc][dim][key] = keys[hc * n + key][dim] (32 x 32 tiles through LDS).
__global__ __launch_bounds__(256) void keys_transpose_kernel(const bf16_t* __restrict__ keys, int n, int half,
                                                             bf16_t* __restrict__ Kt) {
  __shared__ uint16_t tile[32][33];
  const int hc = blockIdx.z;
  const int k0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const bf16_t* src = keys + (int64_t)hc * n * half;
  bf16_t* dst = Kt + (int64_t)hc * half * n;
  for (int r = ty; r < 32; r += 8) {
    const int key = k0 + r, dim = d0 + tx;
    tile[r][tx] = (key < n && dim < half) ? src[(int64_t)key * half + dim].x : (uint16_t)0;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int dim = d0 + r, key = k0 + tx;
    if (dim < half && key < n) dst[(int64_t)dim * n + key].x = tile[tx][r];
  }
}

// MFMA over one staged chunk: wave (wm, wd) accumulates rows [64 wm, +64) x
// dims [64 wd, +64) from A [rows][chunk] and B [dims][chunk] (both [.][kSgLd]).
__device__ __forceinline__ void sg_chunk_mma(const uint16_t* As, const uint16_t* Bs, int wm, int wd, int lane,
                                             int half, sg_f32x4_t (&acc)[4][4]) {
  const int r = lane & 15, kq = 8 * (lane >> 4);
#pragma unroll
  for (int ks = 0; ks < kSgChunk / 32; ++ks) {
    uint4 a[4], b[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) a[mt] = *(const uint4*)(As + (64 * wm + 16 * mt + r) * kSgLd + 32 * ks + kq);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) b[nt] = *(const uint4*)(Bs + (64 * wd + 16 * nt + r) * kSgLd + 32 * ks + kq);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      if (64 * wd + 16 * nt < half) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) sg_mma(a[mt], b[nt], acc[mt][nt]);
      }
    }
  }
}

__device__ __forceinline__ void sg_zero(uint16_t* p, int elems) {
  for (int i = threadIdx.x; i < elems / 8; i += kSgThreads) *(uint4*)(p + 8 * i) = make_uint4(0u, 0u, 0u, 0u);
}

// dq[t, h, c*half + dim] = sum_key dS_c[t, key] * K_c[key, dim]:
// workgroup = 128 tokens of one (h, c); chunks of 64 keys.
template <int EPT>  // list entries per thread (knn <= 4 * EPT)
__global__ __launch_bounds__(kSgThreads) void score_dq_kernel(const uint32_t* __restrict__ lists,
                                                              const bf16_t* __restrict__ Kt, int64_t Ntok, int H,
                                                              int n, int half, int knn, bf16_t* __restrict__ dq) {
  __shared__ __align__(16) uint16_t As[kSgRows * kSgLd];     // [token][key of the chunk]
  __shared__ __align__(16) uint16_t Bs[kSgMaxHalf * kSgLd];  // [dim][key of the chunk]
  const int hc = blockIdx.y, h = hc >> 1, c = hc & 1;
  const int64_t t0 = (int64_t)blockIdx.x * kSgRows;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wd = w >> 1;
  // this thread's list entries: token tl = tid / 4, slots (tid % 4) + 4 s
  const int tl = tid >> 2;
  const int64_t t = t0 + tl;
  uint32_t ent[EPT];
#pragma unroll
  for (int s = 0; s < EPT; ++s) {
    const int j = (tid & 3) + 4 * s;
    ent[s] = (t < Ntok && j < knn) ? lists[((t * H + h) * 2 + c) * knn + j] : kNoEntry;
  }
  const bf16_t* Kc = Kt + (int64_t)hc * half * n;
  sg_f32x4_t acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = sg_f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < n; k0 += kSgChunk) {
    sg_zero(As, kSgRows * kSgLd);
    // B: Kt[dim][k0 .. k0 + 64) for dim < half (8 x 16 bytes per dim)
    for (int i = tid; i < half * (kSgChunk / 8); i += kSgThreads) {
      const int dim = i >> 3, q8 = i & 7;
      *(uint4*)(Bs + dim * kSgLd + 8 * q8) = *(const uint4*)(Kc + (int64_t)dim * n + k0 + 8 * q8);
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < EPT; ++s) {
      const uint32_t e = ent[s];
      const int key = (int)(e >> 16) - k0;
      if (e != kNoEntry && key >= 0 && key < kSgChunk) As[tl * kSgLd + key] = (uint16_t)(e & 0xFFFFu);
    }
    __syncthreads();
    sg_chunk_mma(As, Bs, wm, wd, lane, half, acc);
    __syncthreads();
  }
  // acc[mt][nt][e]: token 64 wm + 16 mt + 4 (lane / 16) + e, dim 64 wd + 16 nt + lane % 16
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t tt = t0 + 64 * wm + 16 * mt + 4 * (lane >> 4) + e;
      if (tt >= Ntok) continue;
      bf16_t* row = dq + (tt * H + h) * 2 * half + (int64_t)c * half;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int dim = 64 * wd + 16 * nt + (lane & 15);
        if (dim < half) row[dim].x = (uint16_t)f32_to_bf16_bits(acc[mt][nt][e]);
      }
    }
  }
}

// Partial dK_c[key, dim] = sum over tokens of the split of dS_c[t, key] q_c[t, dim]:
// workgroup = 128 keys of one (h, c) and one token split; chunks of 64 tokens.
template <int EPT>  // list entries per thread and chunk (knn <= 8 * EPT)
__global__ __launch_bounds__(kSgThreads) void score_dk_kernel(const uint32_t* __restrict__ lists,
                                                              const bf16_t* __restrict__ Q, int64_t Ntok, int H,
                                                              int n, int half, int knn, int64_t tok_split,
                                                              float* __restrict__ part) {
  __shared__ __align__(16) uint16_t As[kSgRows * kSgLd];     // [key][token of the chunk]
  __shared__ __align__(16) uint16_t Bs[kSgMaxHalf * kSgLd];  // [dim][token of the chunk]
  const int hc = blockIdx.y, h = hc >> 1, c = hc & 1;
  const int kb = blockIdx.x * kSgRows;
  const int64_t ts = (int64_t)blockIdx.z * tok_split;
  const int64_t te = ts + tok_split < Ntok ? ts + tok_split : Ntok;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wd = w >> 1;
  sg_f32x4_t acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = sg_f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int kdim = 2 * half;
  for (int64_t tc = ts; tc < te; tc += kSgChunk) {
    sg_zero(As, kSgRows * kSgLd);
    // B: q_c[t][dim] transposed to [dim][t]; a thread packs tokens 2p, 2p + 1 of 8 dims
    for (int i = tid; i < (kSgChunk / 2) * (half / 8); i += kSgThreads) {
      const int p = i & (kSgChunk / 2 - 1), dg = i / (kSgChunk / 2);
      const int64_t ta = tc + 2 * p, tb = ta + 1;
      uint4 va = make_uint4(0u, 0u, 0u, 0u), vb = va;
      if (ta < te) va = *(const uint4*)(Q + (ta * H + h) * kdim + c * half + 8 * dg);
      if (tb < te) vb = *(const uint4*)(Q + (tb * H + h) * kdim + c * half + 8 * dg);
      const uint32_t xa[4] = {va.x, va.y, va.z, va.w}, xb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        *(uint32_t*)(Bs + (8 * dg + 2 * e) * kSgLd + 2 * p) = (xa[e] & 0xFFFFu) | (xb[e] << 16);
        *(uint32_t*)(Bs + (8 * dg + 2 * e + 1) * kSgLd + 2 * p) = (xa[e] >> 16) | (xb[e] & 0xFFFF0000u);
      }
    }
    __syncthreads();
    // A: this chunk's entries with a key in the block; token tl = tid / 8, slots (tid % 8) + 8 s
    {
      const int tl = tid >> 3;
      const int64_t t = tc + tl;
#pragma unroll
      for (int s = 0; s < EPT; ++s) {
        const int j = (tid & 7) + 8 * s;
        if (t < te && j < knn) {
          const uint32_t e = lists[((t * H + h) * 2 + c) * knn + j];
          const int key = (int)(e >> 16) - kb;
          if (e != kNoEntry && key >= 0 && key < kSgRows) As[key * kSgLd + tl] = (uint16_t)(e & 0xFFFFu);
        }
      }
    }
    __syncthreads();
    sg_chunk_mma(As, Bs, wm, wd, lane, half, acc);
    __syncthreads();
  }
  // acc[mt][nt][e]: key kb + 64 wm + 16 mt + 4 (lane / 16) + e, dim 64 wd + 16 nt + lane % 16
  float* P = part + ((int64_t)blockIdx.z * gridDim.y + hc) * n * half;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = kb + 64 * wm + 16 * mt + 4 * (lane >> 4) + e;
      if (key >= n) continue;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int dim = 64 * wd + 16 * nt + (lane & 15);
        if (dim < half) P[(int64_t)key * half + dim] = acc[mt][nt][e];
      }
    }
  }
}

// dK[i] = bf16(sum over splits, in order, of the partials); i over 2H * n * half.
__global__ void score_dk_reduce_kernel(const float* __restrict__ part, int64_t total, int splits,
                                       bf16_t* __restrict__ dk) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int k = 0; k < splits; ++k) s += part[(int64_t)k * total + i];
    dk[i].x = (uint16_t)f32_to_bf16_bits(s);
  }
}

struct SparseGradPlan {
  int splits;
  int64_t tok_split;
  size_t lists, kt, part, total;
};

static SparseGradPlan sparse_grad_plan(int64_t N, int64_t H, int64_t n, int64_t half, int64_t knn) {
  SparseGradPlan p;
  if (N < 1) N = 1;  // sizes for no tokens: the smallest plan (d_keys is only cleared then)
  // token splits of dK: enough workgroups for the GPU (>= 512), chunks of 64 per split
  const int64_t wg = (n / kSgRows) * 2 * H;
  int64_t sp = (512 + wg - 1) / wg;
  const int64_t max_sp = (N + kSgChunk - 1) / kSgChunk;
  if (sp > max_sp) sp = max_sp;
  if (sp < 1) sp = 1;
  p.tok_split = ((N + sp - 1) / sp + kSgChunk - 1) / kSgChunk * kSgChunk;
  p.splits = (int)((N + p.tok_split - 1) / p.tok_split);
  if (p.splits < 1) p.splits = 1;
  auto a256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  p.lists = off;
  off += a256((size_t)N * H * 2 * knn * 4);
  p.kt = off;
  off += a256((size_t)2 * H * n * half * 2);
  p.part = off;
  off += a256((size_t)p.splits * 2 * H * n * half * 4);
  p.total = off;
  return p;
}

static bool sparse_grad_supported(int64_t n, int64_t half, int64_t knn) {
  return n % kSgRows == 0 && n <= 65535 && half % 16 == 0 && half <= kSgMaxHalf && knn >= 1 && knn <= 64;
}

}  // namespace pkm

using namespace pkm;

extern "C" int pkm_score_grad_dense(const int64_t* indices, const void* d_scores, int dtype, int64_t num_tokens,
                                    int64_t heads, int64_t n_keys, int64_t knn, const void* d_sub_scores1,
                                    const void* d_sub_scores2, void* d_sub_dense, void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "pkm_score_grad_dense: dtype %d not supported (float32 and bfloat16 are)", dtype);
  PKM_REQUIRE(num_tokens >= 0 && heads >= 1 && n_keys >= 1 && knn >= 1 && knn <= 64, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_grad_dense: bad sizes");
  PKM_REQUIRE(n_keys % 4 == 0 && n_keys <= kGradMaxN, PKM_ERR_UNSUPPORTED,
              "pkm_score_grad_dense: n_keys %lld must be a multiple of 4 up to %d", (long long)n_keys, kGradMaxN);
  if (num_tokens == 0) return PKM_OK;
  PKM_REQUIRE(indices && d_scores && d_sub_dense, PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_dense: null pointer");
  PKM_REQUIRE((uintptr_t)d_sub_dense % 16 == 0 && (uintptr_t)d_sub_scores1 % 16 == 0 &&
                  (uintptr_t)d_sub_scores2 % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_dense: dense buffers must be 16-byte aligned");
  const int64_t NH = num_tokens * heads;
  const int64_t blocks = (NH + kGradWaves - 1) / kGradWaves;
  PKM_REQUIRE(blocks < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_dense: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const size_t lds = (size_t)kGradWaves * 2 * n_keys * sizeof(float);
  if (dtype == PKM_DTYPE_BF16) {
    hipLaunchKernelGGL(score_grad_dense_kernel<bf16_t>, dim3((unsigned)blocks), dim3(64 * kGradWaves), lds, st,
                       indices, (const bf16_t*)d_scores, NH, (int)heads, (int)n_keys, (int)knn,
                       (const bf16_t*)d_sub_scores1, (const bf16_t*)d_sub_scores2, (bf16_t*)d_sub_dense, num_tokens);
  } else {
    hipLaunchKernelGGL(score_grad_dense_kernel<float>, dim3((unsigned)blocks), dim3(64 * kGradWaves), lds, st,
                       indices, (const float*)d_scores, NH, (int)heads, (int)n_keys, (int)knn,
                       (const float*)d_sub_scores1, (const float*)d_sub_scores2, (float*)d_sub_dense, num_tokens);
  }
  return pkm_check_launch("pkm_score_grad_dense");
}

extern "C" size_t pkm_score_grad_sparse_workspace_size(int64_t num_tokens, int64_t heads, int64_t n_keys,
                                                       int64_t half, int64_t knn) {
  if (num_tokens < 0 || heads < 1 || !sparse_grad_supported(n_keys, half, knn)) return 0;
  return sparse_grad_plan(num_tokens, heads, n_keys, half, knn).total;
}

extern "C" int pkm_score_grad_sparse(const int64_t* indices, const void* d_scores, int dtype, int64_t num_tokens,
                                     int64_t heads, int64_t n_keys, int64_t half, int64_t knn, const void* query,
                                     const void* keys, void* d_query, void* d_keys, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED, "pkm_score_grad_sparse: dtype %d not supported (bfloat16 is)",
              dtype);
  PKM_REQUIRE(num_tokens >= 0 && heads >= 1, PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_sparse: bad sizes");
  PKM_REQUIRE(sparse_grad_supported(n_keys, half, knn), PKM_ERR_UNSUPPORTED,
              "pkm_score_grad_sparse: n_keys %lld (a multiple of %d), half %lld (a multiple of 16 up to %d) and "
              "knn %lld (up to 64) not supported",
              (long long)n_keys, kSgRows, (long long)half, kSgMaxHalf, (long long)knn);
  const int64_t total = 2 * heads * n_keys * half;
  const unsigned reduce_blocks = (unsigned)((total + 255) / 256 < 16384 ? (total + 255) / 256 : 16384);
  if (num_tokens == 0) {  // no tokens: d_keys = 0 (a sum over no splits)
    if (d_keys != nullptr)
      hipLaunchKernelGGL(score_dk_reduce_kernel, dim3(reduce_blocks), dim3(256), 0, (hipStream_t)stream,
                         (const float*)nullptr, total, 0, (bf16_t*)d_keys);
    return pkm_check_launch("pkm_score_grad_sparse");
  }
  PKM_REQUIRE(indices && d_scores && query && keys, PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_sparse: null input");
  const SparseGradPlan pl = sparse_grad_plan(num_tokens, heads, n_keys, half, knn);
  PKM_REQUIRE(workspace != nullptr && workspace_bytes >= pl.total && (uintptr_t)workspace % 256 == 0,
              PKM_ERR_WORKSPACE, "pkm_score_grad_sparse: workspace of %zu bytes given, %zu needed (256-byte aligned)",
              workspace_bytes, pl.total);
  PKM_REQUIRE((uintptr_t)query % 16 == 0 && (uintptr_t)keys % 16 == 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_grad_sparse: query and keys must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint32_t* lists = (uint32_t*)(ws + pl.lists);
  const int64_t NH = num_tokens * heads;
  hipLaunchKernelGGL(score_grad_lists_kernel, dim3((unsigned)((NH + kGradWaves - 1) / kGradWaves)),
                     dim3(64 * kGradWaves), 0, st, indices, (const bf16_t*)d_scores, NH, (int)n_keys, (int)knn, lists);
  const unsigned tb = (unsigned)((num_tokens + kSgRows - 1) / kSgRows);
  if (d_query != nullptr) {
    bf16_t* Kt = (bf16_t*)(ws + pl.kt);
    hipLaunchKernelGGL(keys_transpose_kernel, dim3((unsigned)(n_keys / 32), (unsigned)((half + 31) / 32),
                                                   (unsigned)(2 * heads)),
                       dim3(256), 0, st, (const bf16_t*)keys, (int)n_keys, (int)half, Kt);
    if (knn <= 32)
      hipLaunchKernelGGL(score_dq_kernel<8>, dim3(tb, (unsigned)(2 * heads)), dim3(kSgThreads), 0, st,
                         (const uint32_t*)lists, (const bf16_t*)Kt, num_tokens, (int)heads, (int)n_keys, (int)half,
                         (int)knn, (bf16_t*)d_query);
    else
      hipLaunchKernelGGL(score_dq_kernel<16>, dim3(tb, (unsigned)(2 * heads)), dim3(kSgThreads), 0, st,
                         (const uint32_t*)lists, (const bf16_t*)Kt, num_tokens, (int)heads, (int)n_keys, (int)half,
                         (int)knn, (bf16_t*)d_query);
  }
  if (d_keys != nullptr) {
    float* part = (float*)(ws + pl.part);
    const dim3 grid((unsigned)(n_keys / kSgRows), (unsigned)(2 * heads), (unsigned)pl.splits);
    if (knn <= 32)
      hipLaunchKernelGGL(score_dk_kernel<4>, grid, dim3(kSgThreads), 0, st, (const uint32_t*)lists,
                         (const bf16_t*)query, num_tokens, (int)heads, (int)n_keys, (int)half, (int)knn, pl.tok_split,
                         part);
    else
      hipLaunchKernelGGL(score_dk_kernel<8>, grid, dim3(kSgThreads), 0, st, (const uint32_t*)lists,
                         (const bf16_t*)query, num_tokens, (int)heads, (int)n_keys, (int)half, (int)knn, pl.tok_split,
                         part);
    hipLaunchKernelGGL(score_dk_reduce_kernel, dim3(reduce_blocks), dim3(256), 0, st, (const float*)part, total,
                       pl.splits, (bf16_t*)d_keys);
  }
  return pkm_check_launch("pkm_score_grad_sparse");
}

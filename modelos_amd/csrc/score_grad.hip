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
constexpr int kSgPitch = kSgChunk;          // bf16 per LDS tile row: 8 slots of 16 bytes
constexpr int kSgMaxHalf = 256;             // dims per half: 4 waves x 64
constexpr int kSgThreads = 512;             // 8 waves: 2 (rows, 64 each) x 4 (dims, 64 each)
constexpr int kSgA = kSgRows * kSgPitch;    // bf16 per dS tile (16 KB)
constexpr int kSgB = kSgMaxHalf * kSgPitch; // bf16 per operand tile (32 KB)
constexpr int kListThreads = 256;

// Offset of (row, col) in a [rows][64] bf16 LDS tile whose 16-byte slot s of
// row r is stored at slot s ^ (r & 7): eight consecutive rows read at one
// column slot cover all banks once.
__device__ __forceinline__ int sg_swz(int row, int col) {
  return row * kSgPitch + ((((col >> 3) ^ row) & 7) << 3) + (col & 7);
}

// Workgroup order that keeps consecutive logical workgroups on one XCD
// (workgroups are dealt to the 8 XCDs round robin): logical g runs on XCD
// g / (count / 8) when the count is a multiple of 8.
__device__ __forceinline__ int sg_logical_block() {
  const int L = blockIdx.x, cnt = gridDim.x;
  return (cnt & 7) == 0 ? (L & 7) * (cnt >> 3) + (L >> 3) : L;
}

// Per (t, h, c): the distinct sub-keys of the row's pairs, in order of first
// occurrence, as (sub-key << 16) | bf16(sum of d over the pairs with that
// sub-key, float32 in j order), then kNoEntry up to knn: the nonzeros of
// dS_c[t, :] (the dense kernel's values). A group of G lanes takes one
// (t, h); each lane compares its pair with the group's G pairs from LDS
// (16-byte broadcast reads), and a ballot places the first occurrences.
template <int G>
__global__ __launch_bounds__(kListThreads) void score_grad_lists_kernel(const int64_t* __restrict__ idx,
                                                                        const bf16_t* __restrict__ d, int64_t NH,
                                                                        int n, int knn,
                                                                        uint32_t* __restrict__ lists) {
  __shared__ __align__(16) uint32_t s_pk[kListThreads];
  __shared__ __align__(16) float s_d[kListThreads];
  const int tid = threadIdx.x, jl = tid % G, gb = tid - jl;
  const int64_t th = (int64_t)blockIdx.x * (kListThreads / G) + tid / G;
  uint32_t pk = kNoEntry;
  float dv = 0.f;
  if (th < NH && jl < knn) {
    const int64_t id = idx[th * knn + jl];
    if (id >= 0 && id < (int64_t)n * n) {  // n <= 65535: the id fits 32 bits
      const uint32_t u = (uint32_t)id, a = u / (uint32_t)n;
      pk = (a << 16) | (u - a * (uint32_t)n);
      dv = bf16_to_f32(d[th * knn + jl].x);
    }
  }
  s_pk[tid] = pk;
  s_d[tid] = dv;
  __syncthreads();
  const uint32_t ua = pk >> 16, ub = pk & 0xFFFFu;  // 0xFFFF (no sub-key) for an unused slot
  float s0 = 0.f, s1 = 0.f;
  bool first0 = true, first1 = true;
#pragma unroll
  for (int j0 = 0; j0 < G; j0 += 4) {
    const uint4 kq = *(const uint4*)&s_pk[gb + j0];
    const float4 dq = *(const float4*)&s_d[gb + j0];
    const uint32_t kk[4] = {kq.x, kq.y, kq.z, kq.w};
    const float dd[4] = {dq.x, dq.y, dq.z, dq.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool m0 = (kk[e] >> 16) == ua, m1 = (kk[e] & 0xFFFFu) == ub;
      s0 = m0 ? s0 + dd[e] : s0;
      s1 = m1 ? s1 + dd[e] : s1;
      if (j0 + e < jl) {
        first0 = first0 && !m0;
        first1 = first1 && !m1;
      }
    }
  }
  const bool valid = pk != kNoEntry;
  const bool put0 = valid && first0, put1 = valid && first1;
  // this group's lanes of the wave-wide ballots; slot = first occurrences before this lane
  const int gw = (tid & 63) - jl;  // the group's first lane in the wave
  const uint64_t gmask = G == 64 ? ~0ull : ((1ull << G) - 1);
  const uint64_t below = (1ull << jl) - 1;
  const uint64_t b0 = (__ballot(put0) >> gw) & gmask, b1 = (__ballot(put1) >> gw) & gmask;
  if (th < NH) {
    uint32_t* row0 = lists + (th * 2 + 0) * knn;
    uint32_t* row1 = row0 + knn;
    if (put0) row0[__popcll(b0 & below)] = (ua << 16) | f32_to_bf16_bits(s0);
    if (put1) row1[__popcll(b1 & below)] = (ub << 16) | f32_to_bf16_bits(s1);
    if (jl < knn && jl >= __popcll(b0)) row0[jl] = kNoEntry;
    if (jl < knn && jl >= __popcll(b1)) row1[jl] = kNoEntry;
  }
}

// Lists and dq in one pass for knn <= 32. One-wave workgroups, each looping
// over the tokens t = wi, wi + per_head, ... of one head h, with the next
// row's pairs loaded while the current row is processed. Per row (t, h):
// lane j of each half-wave takes pair j; lanes 0-31 build the list of
// sub-key half c = 0, lanes 32-63 that of c = 1 (same values and order as
// score_grad_lists_kernel), into LDS and the global lists; then half-wave c
// gathers dq[t, h, c*half + 8 j .. + 8] = sum over its list, in order, of
// v * keys[(2h + c) n + key][...] (float32, rounded once), 16 key rows in
// flight. The workgroups of one head stay on one XCD (its key slices in L2).
// v * k is formed by v_dot2 of (k_lo, k_hi) with (v, 0) or (0, v): exact
// bf16 products added to the float32 sum with one rounding, as an FMA.
constexpr int kRowBatch = 16;
__global__ __launch_bounds__(64) void score_grad_rows_kernel(const int64_t* __restrict__ idx,
                                                             const bf16_t* __restrict__ d,
                                                             const bf16_t* __restrict__ keys, int64_t Ntok, int H,
                                                             int n, int half, int knn, int per_head,
                                                             uint32_t* __restrict__ lists, bf16_t* __restrict__ dq) {
  __shared__ __align__(16) uint32_t s_key[2][32];
  __shared__ __align__(16) float s_d[32];
  __shared__ __align__(16) uint32_t s_list[2][32];
  const int g = sg_logical_block();
  const int h = g / per_head, wi = g - h * per_head;
  const int lane = threadIdx.x, c = lane >> 5, j = lane & 31;
  const bool pair = j < knn;
  // key rows of head h (both halves) from one wave-uniform base; 32-bit byte offsets
  const char* Kh = (const char*)(keys + (int64_t)2 * h * n * half);
  const uint32_t row_bytes = (uint32_t)half * 2, lane_off = (uint32_t)c * n * row_bytes + 16u * j;
  const bool dims = 8 * j < half;
  int64_t id = -1;
  uint32_t draw = 0;
  if (wi < Ntok && pair) {
    const int64_t th = (int64_t)wi * H + h;
    id = idx[th * knn + j];
    draw = d[th * knn + j].x;
  }
  for (int64_t t = wi; t < Ntok; t += per_head) {
    const int64_t th = t * H + h;
    uint32_t my = 0xFFFFFFFFu;  // this lane's sub-key of half c (none: matches no sub-key)
    float dv = 0.f;
    if (pair && id >= 0 && id < (int64_t)n * n) {  // n <= 65535: the id fits 32 bits
      const uint32_t u = (uint32_t)id, a = u / (uint32_t)n;
      my = c ? u - a * (uint32_t)n : a;
      dv = bf16_to_f32(draw);
    }
    // the next row's pairs, in flight during this row
    const int64_t tn = t + per_head;
    id = -1;
    if (tn < Ntok && pair) {
      const int64_t thn = tn * H + h;
      id = idx[thn * knn + j];
      draw = d[thn * knn + j].x;
    }
    s_key[c][j] = my;
    if (c == 0) s_d[j] = dv;
    __syncthreads();
    float sum = 0.f;  // starts at +0 and never becomes -0: adding +0 on a mismatch keeps it
    bool first = true;
#pragma unroll
    for (int j0 = 0; j0 < 32; j0 += 4) {
      const uint4 kq = *(const uint4*)&s_key[c][j0];
      const float4 dq4 = *(const float4*)&s_d[j0];
      const uint32_t kk[4] = {kq.x, kq.y, kq.z, kq.w};
      const float dd[4] = {dq4.x, dq4.y, dq4.z, dq4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool m = kk[e] == my;
        sum += m ? dd[e] : 0.f;
        if (j0 + e < j) first = first && !m;
      }
    }
    const bool put = my != 0xFFFFFFFFu && first;
    const uint32_t bits = (uint32_t)(__ballot(put) >> (32 * c));
    const int cnt = __popc(bits);
    const int pos = __popc(bits & ((1u << j) - 1));
    const uint32_t entry = (my << 16) | f32_to_bf16_bits(sum);
    if (put) s_list[c][pos] = entry;
    uint32_t* L = lists + (th * 2 + c) * knn;
    if (put) L[pos] = entry;
    if (pair && j >= cnt) L[j] = kNoEntry;
    __syncthreads();
    if (dims) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int b0 = 0; b0 < cnt; b0 += kRowBatch) {
        uint32_t e[kRowBatch];
        uint4 kv[kRowBatch];
#pragma unroll
        for (int q = 0; q < kRowBatch; q += 4) {
          const uint4 eq = *(const uint4*)&s_list[c][b0 + q];
          e[q] = eq.x;
          e[q + 1] = eq.y;
          e[q + 2] = eq.z;
          e[q + 3] = eq.w;
        }
#pragma unroll
        for (int q = 0; q < kRowBatch; ++q) {
          kv[q] = make_uint4(0u, 0u, 0u, 0u);
          if (b0 + q < cnt) kv[q] = *(const uint4*)(Kh + (lane_off + (e[q] >> 16) * row_bytes));
        }
#pragma unroll
        for (int q = 0; q < kRowBatch; ++q) {
          if (b0 + q < cnt) {
            const bf16x2_t vlo = __builtin_bit_cast(bf16x2_t, e[q] & 0xFFFFu);  // (v, 0)
            const bf16x2_t vhi = __builtin_bit_cast(bf16x2_t, e[q] << 16);      // (0, v)
            const uint32_t x[4] = {kv[q].x, kv[q].y, kv[q].z, kv[q].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const bf16x2_t kx = __builtin_bit_cast(bf16x2_t, x[i]);
              acc[2 * i] = __builtin_amdgcn_fdot2_f32_bf16(kx, vlo, acc[2 * i], false);
              acc[2 * i + 1] = __builtin_amdgcn_fdot2_f32_bf16(kx, vhi, acc[2 * i + 1], false);
            }
          }
        }
      }
      *(uint4*)(dq + (th * 2 + c) * half + 8 * j) =
          make_uint4(pack2_bf16(acc[0], acc[1]), pack2_bf16(acc[2], acc[3]), pack2_bf16(acc[4], acc[5]),
                     pack2_bf16(acc[6], acc[7]));
    }
  }
}

// MFMA over one staged chunk: wave (wm, wd) accumulates rows [64 wm, +64) x
// dims [64 wd, +64) from A [rows][chunk] and B [dims][chunk] (swizzled tiles).
// FULL: half == kSgMaxHalf (every wave's dims exist).
template <bool FULL>
__device__ __forceinline__ void sg_chunk_mma(const uint16_t* As, const uint16_t* Bs, int wm, int wd, int lane,
                                             int half, sg_f32x4_t (&acc)[4][4]) {
  const int r = lane & 15;
  uint4 a[2][4], b[2][4];
#pragma unroll
  for (int ks = 0; ks < kSgChunk / 32; ++ks) {
    const int so = (((4 * ks + (lane >> 4)) ^ r) & 7) << 3;  // row & 7 == r & 7 for every tile row below
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) a[ks][mt] = *(const uint4*)(As + (64 * wm + 16 * mt + r) * kSgPitch + so);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) b[ks][nt] = *(const uint4*)(Bs + (64 * wd + 16 * nt + r) * kSgPitch + so);
  }
#pragma unroll
  for (int ks = 0; ks < kSgChunk / 32; ++ks) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      if (FULL || 64 * wd + 16 * nt < half) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) sg_mma(a[ks][mt], b[ks][nt], acc[mt][nt]);
      }
    }
  }
}

__device__ __forceinline__ void sg_zero(uint16_t* p) {
#pragma unroll
  for (int i = threadIdx.x; i < kSgA / 8; i += kSgThreads) *(uint4*)(p + 8 * i) = make_uint4(0u, 0u, 0u, 0u);
}

// dq[t, h, c*half + e] = sum over the list of (t, h, c), in list order, of
// v * keys[(2h + c) n + key][e] (float32, rounded once): the row of dS_c @ K_c
// from its nonzeros. One wave per (t, h, c) (the list is wave-uniform: scalar
// loads, uniform early exit at the first empty slot), 4 dims per lane;
// workgroups of one (h, c) stay on one XCD so its key slice stays in that L2.
constexpr int kDqWaves = 4;
__global__ __launch_bounds__(64 * kDqWaves) void score_dq_gather_kernel(const uint32_t* __restrict__ lists,
                                                                        const bf16_t* __restrict__ keys,
                                                                        int64_t Ntok, int H, int n, int half, int knn,
                                                                        int tok_blocks, bf16_t* __restrict__ dq) {
  const int g = sg_logical_block();
  const int hc = g / tok_blocks, h = hc >> 1, c = hc & 1;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t t = (int64_t)(g - hc * tok_blocks) * kDqWaves + w;
  if (t >= Ntok) return;
  const bool active = 4 * lane < half;
  const uint32_t* L = lists + ((t * H + h) * 2 + c) * knn;
  const bf16_t* Kc = keys + (int64_t)hc * n * half + 4 * lane;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < knn; j0 += 8) {
    uint32_t e[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) e[jj] = j0 + jj < knn ? L[j0 + jj] : kNoEntry;
    if (e[0] == kNoEntry) break;  // entries are packed at the front
    uint2 kv[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      kv[jj] = make_uint2(0u, 0u);
      if (e[jj] != kNoEntry && active) kv[jj] = *(const uint2*)(Kc + (int64_t)(e[jj] >> 16) * half);
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if (e[jj] != kNoEntry) {
        const float v = bf16_to_f32((uint16_t)(e[jj] & 0xFFFFu));
        acc[0] = fmaf(v, bf16_to_f32((uint16_t)(kv[jj].x & 0xFFFFu)), acc[0]);
        acc[1] = fmaf(v, bf16_to_f32((uint16_t)(kv[jj].x >> 16)), acc[1]);
        acc[2] = fmaf(v, bf16_to_f32((uint16_t)(kv[jj].y & 0xFFFFu)), acc[2]);
        acc[3] = fmaf(v, bf16_to_f32((uint16_t)(kv[jj].y >> 16)), acc[3]);
      }
    }
  }
  if (active)
    *(uint2*)(dq + (t * H + h) * 2 * half + (int64_t)c * half + 4 * lane) =
        make_uint2(pack2_bf16(acc[0], acc[1]), pack2_bf16(acc[2], acc[3]));
}

// Partial dK_c[key, dim] = sum over the split's tokens of dS_c[t, key] q_c[t, dim]:
// workgroup = 128 keys of one (h, c) and one token split; chunks of 64 tokens,
// buffered as in score_dq_kernel (lists and query rows loaded a chunk ahead).
template <int EPT, bool FULL>  // list entries per thread and chunk (knn <= 8 * EPT); FULL: half == kSgMaxHalf
__global__ __launch_bounds__(kSgThreads) void score_dk_kernel(const uint32_t* __restrict__ lists,
                                                              const bf16_t* __restrict__ Q, int64_t Ntok, int H,
                                                              int n, int half, int knn, int64_t tok_split,
                                                              int kblocks, float* __restrict__ part) {
  __shared__ __align__(16) uint16_t As[3 * kSgA];  // [key][token of the chunk]
  __shared__ __align__(16) uint16_t Bs[2 * kSgB];  // [dim][token of the chunk]
  const int g = sg_logical_block();
  const int kbi = g % kblocks, rest = g / kblocks;
  const int HC = 2 * H;
  const int hc = rest % HC, split = rest / HC, h = hc >> 1, c = hc & 1;
  const int kb = kbi * kSgRows;
  const int64_t ts = (int64_t)split * tok_split;
  const int64_t te = ts + tok_split < Ntok ? ts + tok_split : Ntok;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wd = w >> 1;
  const int kdim = 2 * half;
  // list entries of a chunk: token tl = tid / 8, slots (tid % 8) + 8 s
  const int tl = tid >> 3;
  uint32_t ent[EPT];
  auto load_e = [&](int64_t tc) {
    const int64_t t = tc + tl;
#pragma unroll
    for (int s = 0; s < EPT; ++s) {
      const int j = (tid & 7) + 8 * s;
      ent[s] = (t < te && j < knn) ? lists[((t * H + h) * 2 + c) * knn + j] : kNoEntry;
    }
  };
  auto scatter = [&](uint16_t* A) {
#pragma unroll
    for (int s = 0; s < EPT; ++s) {
      const uint32_t e = ent[s];
      const int key = (int)(e >> 16) - kb;
      if (e != kNoEntry && (unsigned)key < (unsigned)kSgRows) A[sg_swz(key, tl)] = (uint16_t)(e & 0xFFFFu);
    }
  };
  // query staging, transposed to [dim][token]: item i = (token pair i % 32, 8-dim group i / 32)
  constexpr int BPT = (kSgChunk / 2) * (kSgMaxHalf / 8) / kSgThreads;
  uint4 qa[BPT], qb[BPT];
  auto load_b = [&](int64_t tc) {
#pragma unroll
    for (int r = 0; r < BPT; ++r) {
      const int i = tid + r * kSgThreads, p = i & (kSgChunk / 2 - 1), dg = i / (kSgChunk / 2);
      const int64_t ta = tc + 2 * p, tb = ta + 1;
      qa[r] = qb[r] = make_uint4(0u, 0u, 0u, 0u);
      if (FULL || 8 * dg < half) {
        if (ta < te) qa[r] = *(const uint4*)(Q + (ta * H + h) * kdim + c * half + 8 * dg);
        if (tb < te) qb[r] = *(const uint4*)(Q + (tb * H + h) * kdim + c * half + 8 * dg);
      }
    }
  };
  auto store_b = [&](uint16_t* B) {
#pragma unroll
    for (int r = 0; r < BPT; ++r) {
      const int i = tid + r * kSgThreads, p = i & (kSgChunk / 2 - 1), dg = i / (kSgChunk / 2);
      if (FULL || 8 * dg < half) {
        const uint32_t xa[4] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w}, xb[4] = {qb[r].x, qb[r].y, qb[r].z, qb[r].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int dim = 8 * dg + 2 * e;
          *(uint32_t*)(B + sg_swz(dim, 2 * p)) = (xa[e] & 0xFFFFu) | (xb[e] << 16);
          *(uint32_t*)(B + sg_swz(dim + 1, 2 * p)) = (xa[e] >> 16) | (xb[e] & 0xFFFF0000u);
        }
      }
    }
  };
  sg_f32x4_t acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = sg_f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int nch = (int)((te - ts + kSgChunk - 1) / kSgChunk);
  sg_zero(As);
  sg_zero(As + kSgA);
  load_e(ts);
  load_b(ts);
  __syncthreads();
  scatter(As);
  store_b(Bs);
  if (nch > 1) {
    load_e(ts + kSgChunk);
    load_b(ts + kSgChunk);
  }
  __syncthreads();
  int ia = 0;
  for (int i = 0; i < nch; ++i) {
    const int ia1 = ia == 2 ? 0 : ia + 1, ia2 = ia1 == 2 ? 0 : ia1 + 1;
    sg_zero(As + ia2 * kSgA);
    if (i + 1 < nch) {
      scatter(As + ia1 * kSgA);
      store_b(Bs + ((i + 1) & 1) * kSgB);
    }
    if (i + 2 < nch) {
      load_e(ts + (int64_t)(i + 2) * kSgChunk);
      load_b(ts + (int64_t)(i + 2) * kSgChunk);
    }
    sg_chunk_mma<FULL>(As + ia * kSgA, Bs + (i & 1) * kSgB, wm, wd, lane, half, acc);
    __syncthreads();
    ia = ia1;
  }
  // acc[mt][nt][e]: key kb + 64 wm + 16 mt + 4 (lane / 16) + e, dim 64 wd + 16 nt + lane % 16
  float* P = part + ((int64_t)split * HC + hc) * n * half;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = kb + 64 * wm + 16 * mt + 4 * (lane >> 4) + e;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int dim = 64 * wd + 16 * nt + (lane & 15);
        if (dim < half) P[(int64_t)key * half + dim] = acc[mt][nt][e];
      }
    }
  }
}

// Wide dK tiles: workgroup = 512 keys x 128 dims of one (h, c) and one token
// split, 16 waves of 64 x 64, chunks of 32 tokens (one MFMA k-step). Query
// rows are read by 2 workgroups and lists by 4 (a 128 x 256 tile reads them
// 8 times). LDS tiles are [rows][32] bf16 (64-byte rows, four 16-byte slots;
// slot s of row r stored at s ^ ((r >> 1) & 3): 8 consecutive rows read at
// one slot cover all banks once); dS tiles triple-buffered, query tiles
// double-buffered, one barrier per chunk.
constexpr int kWkKeys = 512;
constexpr int kWkDims = 128;
constexpr int kWkChunk = 32;
constexpr int kWkThreads = 1024;
constexpr int kWkA = kWkKeys * kWkChunk;  // bf16 per dS tile (32 KB)
constexpr int kWkB = kWkDims * kWkChunk;  // bf16 per query tile (8 KB)

__device__ __forceinline__ int wk_swz(int row, int col) {
  return row * kWkChunk + ((((col >> 3) ^ (row >> 1)) & 3) << 3) + (col & 7);
}

template <int EPT>  // list entries per thread and chunk (knn <= EPT)
__global__ __launch_bounds__(kWkThreads) void score_dk_wide_kernel(const uint32_t* __restrict__ lists,
                                                                   const bf16_t* __restrict__ Q, int64_t Ntok,
                                                                   int H, int n, int half, int knn,
                                                                   int64_t tok_split, int kblocks, int dblocks,
                                                                   float* __restrict__ part) {
  __shared__ __align__(16) uint16_t As[3 * kWkA];  // [key][token of the chunk]
  __shared__ __align__(16) uint16_t Bs[2 * kWkB];  // [dim][token of the chunk]
  const int g = sg_logical_block();
  const int dbi = g % dblocks, r1 = g / dblocks;
  const int kbi = r1 % kblocks, r2 = r1 / kblocks;
  const int HC = 2 * H;
  const int hc = r2 % HC, split = r2 / HC, h = hc >> 1, c = hc & 1;
  const int kb = kbi * kWkKeys, db = dbi * kWkDims;
  const int64_t ts = (int64_t)split * tok_split;
  const int64_t te = ts + tok_split < Ntok ? ts + tok_split : Ntok;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 7, wd = w >> 3;  // 8 key tiles x 2 dim tiles of 64
  const int kdim = 2 * half;
  // lists: token tid / 32 of the chunk, slots tid % 32 (+ 32 s)
  const int tl = tid >> 5;
  // query items: 16 token pairs x 16 groups of 8 dims, threads 0..255
  const bool qthread = tid < (kWkChunk / 2) * (kWkDims / 8);
  const int qp = tid & (kWkChunk / 2 - 1), qg = (tid >> 4) & (kWkDims / 8 - 1);
  struct Stage {
    uint32_t ent[EPT];
    uint4 qa, qb;
  };
  auto load = [&](Stage& S, int64_t tc) {
    const int64_t t = tc + tl;
#pragma unroll
    for (int s = 0; s < EPT; ++s) {
      const int j = (tid & 31) + 32 * s;
      S.ent[s] = (t < te && j < knn) ? lists[((t * H + h) * 2 + c) * knn + j] : kNoEntry;
    }
    S.qa = S.qb = make_uint4(0u, 0u, 0u, 0u);
    if (qthread) {
      const int64_t ta = tc + 2 * qp, tb = ta + 1;
      if (ta < te) S.qa = *(const uint4*)(Q + (ta * H + h) * kdim + c * half + db + 8 * qg);
      if (tb < te) S.qb = *(const uint4*)(Q + (tb * H + h) * kdim + c * half + db + 8 * qg);
    }
  };
  auto put = [&](const Stage& S, uint16_t* A, uint16_t* B) {
#pragma unroll
    for (int s = 0; s < EPT; ++s) {
      const uint32_t e = S.ent[s];
      const int key = (int)(e >> 16) - kb;
      if (e != kNoEntry && (unsigned)key < (unsigned)kWkKeys) A[wk_swz(key, tl)] = (uint16_t)(e & 0xFFFFu);
    }
    if (qthread) {
      const uint32_t xa[4] = {S.qa.x, S.qa.y, S.qa.z, S.qa.w}, xb[4] = {S.qb.x, S.qb.y, S.qb.z, S.qb.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int dim = 8 * qg + 2 * e;
        *(uint32_t*)(B + wk_swz(dim, 2 * qp)) = (xa[e] & 0xFFFFu) | (xb[e] << 16);
        *(uint32_t*)(B + wk_swz(dim + 1, 2 * qp)) = (xa[e] >> 16) | (xb[e] & 0xFFFF0000u);
      }
    }
  };
  auto zero = [&](uint16_t* A) {
#pragma unroll
    for (int i = tid; i < kWkA / 8; i += kWkThreads) *(uint4*)(A + 8 * i) = make_uint4(0u, 0u, 0u, 0u);
  };
  sg_f32x4_t acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = sg_f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const uint16_t* A, const uint16_t* B) {
    const int r = lane & 15, q = lane >> 4;
    uint4 a[4], b[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) a[mt] = *(const uint4*)(A + wk_swz(64 * wm + 16 * mt + r, 8 * q));
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) b[nt] = *(const uint4*)(B + wk_swz(64 * wd + 16 * nt + r, 8 * q));
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) sg_mma(a[mt], b[nt], acc[mt][nt]);
  };
  const int nch = (int)((te - ts + kWkChunk - 1) / kWkChunk);
  Stage st;
  zero(As);
  zero(As + kWkA);
  load(st, ts);
  __syncthreads();
  put(st, As, Bs);
  if (nch > 1) load(st, ts + kWkChunk);
  __syncthreads();
  int ia = 0;
  for (int i = 0; i < nch; ++i) {
    const int ia1 = ia == 2 ? 0 : ia + 1, ia2 = ia1 == 2 ? 0 : ia1 + 1;
    zero(As + ia2 * kWkA);  // chunk i-1's tile, multiplied before the last barrier
    if (i + 1 < nch) put(st, As + ia1 * kWkA, Bs + ((i + 1) & 1) * kWkB);
    if (i + 2 < nch) load(st, ts + (int64_t)(i + 2) * kWkChunk);
    mma(As + ia * kWkA, Bs + (i & 1) * kWkB);
    __syncthreads();
    ia = ia1;
  }
  // acc[mt][nt][e]: key kb + 64 wm + 16 mt + 4 (lane / 16) + e, dim db + 64 wd + 16 nt + lane % 16
  float* P = part + ((int64_t)split * HC + hc) * n * half;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = kb + 64 * wm + 16 * mt + 4 * (lane >> 4) + e;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) P[(int64_t)key * half + db + 64 * wd + 16 * nt + (lane & 15)] = acc[mt][nt][e];
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
  bool wide;  // score_dk_wide_kernel (512 x 128 tiles, 32-token chunks)
  int splits;
  int64_t tok_split;
  size_t lists, part, total;
};

static bool dk_wide_fits(int64_t n, int64_t half) { return n % kWkKeys == 0 && half % kWkDims == 0; }

static SparseGradPlan sparse_grad_plan(int64_t N, int64_t H, int64_t n, int64_t half, int64_t knn) {
  SparseGradPlan p;
  if (N < 1) N = 1;  // sizes for no tokens: the smallest plan (d_keys is only cleared then)
  p.wide = dk_wide_fits(n, half);
  // token splits of dK: enough workgroups for the GPU (256 of the wide tiles,
  // one per CU; 512 of the 128 x 256 tiles), whole chunks per split
  const int64_t chunk = p.wide ? kWkChunk : kSgChunk;
  const int64_t wg = p.wide ? (n / kWkKeys) * (half / kWkDims) * 2 * H : (n / kSgRows) * 2 * H;
  const int64_t target = p.wide ? 256 : 512;
  int64_t sp = (target + wg - 1) / wg;
  const int64_t max_sp = (N + chunk - 1) / chunk;
  if (sp > max_sp) sp = max_sp;
  if (sp < 1) sp = 1;
  p.tok_split = ((N + sp - 1) / sp + chunk - 1) / chunk * chunk;
  p.splits = (int)((N + p.tok_split - 1) / p.tok_split);
  if (p.splits < 1) p.splits = 1;
  auto a256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  p.lists = off;
  off += a256((size_t)N * H * 2 * knn * 4);
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

namespace pkm {
int score_grad_dense_generic(const int64_t* indices, const void* d_scores, int dtype, int64_t num_tokens,
                             int64_t heads, int64_t n_keys, int64_t knn, const void* d_sub1, const void* d_sub2,
                             void* d_sub_dense, int lds_max, hipStream_t st);
}

extern "C" int pkm_score_grad_dense(const int64_t* indices, const void* d_scores, int dtype, int64_t num_tokens,
                                    int64_t heads, int64_t n_keys, int64_t knn, const void* d_sub_scores1,
                                    const void* d_sub_scores2, void* d_sub_dense, void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16 || dtype == PKM_DTYPE_F16, PKM_ERR_UNSUPPORTED,
              "pkm_score_grad_dense: dtype %d not supported (float32, bfloat16 and float16 are)", dtype);
  PKM_REQUIRE(num_tokens >= 0 && heads >= 1 && n_keys >= 1 && knn >= 1, PKM_ERR_INVALID_ARGUMENT,
              "pkm_score_grad_dense: bad sizes");
  if (num_tokens == 0) return PKM_OK;
  PKM_REQUIRE(indices && d_scores && d_sub_dense, PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_dense: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const bool tuned = dtype != PKM_DTYPE_F16 && knn <= 64 && n_keys % 4 == 0 && n_keys <= kGradMaxN &&
                     (uintptr_t)d_sub_dense % 16 == 0 && (uintptr_t)d_sub_scores1 % 16 == 0 &&
                     (uintptr_t)d_sub_scores2 % 16 == 0;
  if (!tuned) {
    int dev = 0, lds_max = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess)
      return pkm_set_error(PKM_ERR_HIP, "pkm_score_grad_dense: device query failed: %s", hipGetErrorString(e));
    const int rc = score_grad_dense_generic(indices, d_scores, dtype, num_tokens, heads, n_keys, knn, d_sub_scores1,
                                            d_sub_scores2, d_sub_dense, lds_max, st);
    if (rc != PKM_OK) return rc;
    return pkm_check_launch("pkm_score_grad_dense");
  }
  const int64_t NH = num_tokens * heads;
  const int64_t blocks = (NH + kGradWaves - 1) / kGradWaves;
  PKM_REQUIRE(blocks < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_dense: too many rows");
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
  PKM_REQUIRE((uintptr_t)query % 16 == 0 && (uintptr_t)keys % 16 == 0 && (uintptr_t)d_query % 16 == 0 &&
                  (uintptr_t)d_keys % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_score_grad_sparse: query, keys, d_query, d_keys must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint32_t* lists = (uint32_t*)(ws + pl.lists);
  const int64_t NH = num_tokens * heads;
  if (d_query != nullptr && knn <= 32) {  // lists and dq in one pass
    // about 16 waves per CU on 256 CUs, split evenly over the heads
    int per_head = (int)((4096 + heads - 1) / heads);
    if ((int64_t)per_head > num_tokens) per_head = (int)num_tokens;
    hipLaunchKernelGGL(score_grad_rows_kernel, dim3((unsigned)(per_head * heads)), dim3(64), 0, st, indices,
                       (const bf16_t*)d_scores, (const bf16_t*)keys, num_tokens, (int)heads, (int)n_keys, (int)half,
                       (int)knn, per_head, lists, (bf16_t*)d_query);
  } else {
    if (knn <= 32)
      hipLaunchKernelGGL(score_grad_lists_kernel<32>,
                         dim3((unsigned)((NH + kListThreads / 32 - 1) / (kListThreads / 32))), dim3(kListThreads), 0,
                         st, indices, (const bf16_t*)d_scores, NH, (int)n_keys, (int)knn, lists);
    else
      hipLaunchKernelGGL(score_grad_lists_kernel<64>,
                         dim3((unsigned)((NH + kListThreads / 64 - 1) / (kListThreads / 64))), dim3(kListThreads), 0,
                         st, indices, (const bf16_t*)d_scores, NH, (int)n_keys, (int)knn, lists);
    if (d_query != nullptr) {
      const int tok_blocks = (int)((num_tokens + kDqWaves - 1) / kDqWaves);
      hipLaunchKernelGGL(score_dq_gather_kernel, dim3((unsigned)(tok_blocks * 2 * heads)), dim3(64 * kDqWaves), 0, st,
                         (const uint32_t*)lists, (const bf16_t*)keys, num_tokens, (int)heads, (int)n_keys, (int)half,
                         (int)knn, tok_blocks, (bf16_t*)d_query);
    }
  }
  if (d_keys != nullptr) {
    float* part = (float*)(ws + pl.part);
    if (pl.wide) {
      const int kblocks = (int)(n_keys / kWkKeys), dblocks = (int)(half / kWkDims);
      const dim3 grid((unsigned)(kblocks * dblocks * 2 * heads * pl.splits));
      auto dk_kernel = knn <= 32 ? score_dk_wide_kernel<1> : score_dk_wide_kernel<2>;
      hipLaunchKernelGGL(dk_kernel, grid, dim3(kWkThreads), 0, st, (const uint32_t*)lists, (const bf16_t*)query,
                         num_tokens, (int)heads, (int)n_keys, (int)half, (int)knn, pl.tok_split, kblocks, dblocks,
                         part);
    } else {
      const int kblocks = (int)(n_keys / kSgRows);
      const dim3 grid((unsigned)(kblocks * 2 * heads * pl.splits));
      auto dk_kernel = knn <= 32 ? (half == kSgMaxHalf ? score_dk_kernel<4, true> : score_dk_kernel<4, false>)
                                 : (half == kSgMaxHalf ? score_dk_kernel<8, true> : score_dk_kernel<8, false>);
      hipLaunchKernelGGL(dk_kernel, grid, dim3(kSgThreads), 0, st, (const uint32_t*)lists, (const bf16_t*)query,
                         num_tokens, (int)heads, (int)n_keys, (int)half, (int)knn, pl.tok_split, kblocks, part);
    }
    hipLaunchKernelGGL(score_dk_reduce_kernel, dim3(reduce_blocks), dim3(256), 0, st, (const float*)part, total,
                       pl.splits, (bf16_t*)d_keys);
  }
  return pkm_check_launch("pkm_score_grad_sparse");
}


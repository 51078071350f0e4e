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

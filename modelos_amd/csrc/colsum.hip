// Column sums of a row-major [rows, cols] matrix, gfx950: the bias gradient
// g.sum(0) of the PKM layer's Linear layers (autograd of nn.Linear's bias,
// pkm/memory.py:147-149, 305), float32 accumulation rounded once to the
// matrix dtype, deterministic.
//
//   part[b, j] = sum over rows i of block b (kColRB rows, in order) of x[i, j]
//   out[j]     = T(sum over blocks b, in order, of part[b, j])
// Stage 1: one 16-byte column vector per thread, kColRB rows with 4 rows'
// loads in flight (float32 / bfloat16 rows of whole 16-byte vectors), or one
// column per thread (any other width, float16, unaligned rows); stage 2: 64
// columns per workgroup, the blocks split over 4 thread slices (contiguous
// ranges, added in slice order). T is float32, bfloat16 or float16.
#include "pkm_common.h"

namespace pkm {

constexpr int kColRB = 32;  // rows per partial

template <typename T, typename TO>
__device__ __forceinline__ void colsum_store(TO* out, int64_t j, float v) {
  if (sizeof(TO) == 4)
    ((float*)out)[j] = v;
  else
    ((uint16_t*)out)[j] = (uint16_t)f32_to_bf16_bits(v);
}

// part == nullptr: the rows form one block and the sums go straight to out
template <typename T, typename TO>
__global__ __launch_bounds__(256) void colsum_partial_kernel(const T* __restrict__ x, int64_t rows, int cols,
                                                             float* __restrict__ part, TO* __restrict__ out) {
  constexpr int EPV = VecTraits<T>::EPV;
  const int nv = cols / EPV;
  const int c = blockIdx.x * 256 + threadIdx.x;  // column vector
  if (c >= nv) return;
  const int64_t r0 = (int64_t)blockIdx.y * kColRB;
  const int64_t r1 = r0 + kColRB < rows ? r0 + kColRB : rows;
  float acc[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc[e] = 0.f;
  int64_t i = r0;
  for (; i + 4 <= r1; i += 4) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = ld16(x + (i + u) * cols + c * EPV);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float f[EPV];
      VecTraits<T>::unpack(v[u], f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[e] += f[e];
    }
  }
  for (; i < r1; ++i) {
    float f[EPV];
    VecTraits<T>::unpack(ld16(x + i * cols + c * EPV), f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] += f[e];
  }
  if (part == nullptr) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) colsum_store<T, TO>(out, (int64_t)c * EPV + e, acc[e]);
    return;
  }
  float* pr = part + (int64_t)blockIdx.y * cols + c * EPV;
#pragma unroll
  for (int e = 0; e < EPV; e += 4) *(float4*)(pr + e) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
}

// One column per thread, element types by runtime code; same sums and order
// as the vector kernel.
__global__ __launch_bounds__(256) void colsum_partial_scalar_kernel(const void* __restrict__ x, int dt, int64_t rows,
                                                                    int cols, float* __restrict__ part,
                                                                    void* __restrict__ out, int odt) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * kColRB;
  const int64_t r1 = r0 + kColRB < rows ? r0 + kColRB : rows;
  float acc = 0.f;
  for (int64_t i = r0; i < r1; ++i) acc += load_scalar(x, dt, i * cols + c);
  if (part == nullptr)
    store_scalar(out, odt, c, acc);
  else
    part[(int64_t)blockIdx.y * cols + c] = acc;
}

__global__ __launch_bounds__(256) void colsum_reduce_kernel(const float* __restrict__ part, int64_t nb, int cols,
                                                            void* __restrict__ out, int odt) {
  __shared__ float ps[4][64];
  const int jl = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + jl;
  const int64_t per = (nb + 3) / 4;
  const int64_t b0 = sl * per, b1 = b0 + per < nb ? b0 + per : nb;
  float s = 0.f;
  if (j < cols) {
    int64_t b = b0;
    for (; b + 8 <= b1; b += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(b + u) * cols + j];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; b < b1; ++b) s += part[b * cols + j];
  }
  ps[sl][jl] = s;
  __syncthreads();
  if (sl == 0 && j < cols) {
    const float t = ((ps[0][jl] + ps[1][jl]) + ps[2][jl]) + ps[3][jl];
    store_scalar(out, odt, j, t);
  }
}

}  // namespace pkm

using namespace pkm;

extern "C" size_t pkm_column_sum_workspace_size(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return 0;
  return (size_t)((rows + kColRB - 1) / kColRB) * (size_t)cols * sizeof(float);
}

extern "C" int pkm_column_sum(const void* x, int64_t rows, int64_t cols, int dtype, int out_dtype, void* out,
                              void* workspace, size_t workspace_bytes, void* stream) {
  auto valid = [](int dt) { return dt == PKM_DTYPE_F32 || dt == PKM_DTYPE_BF16 || dt == PKM_DTYPE_F16; };
  PKM_REQUIRE(valid(dtype) && valid(out_dtype), PKM_ERR_UNSUPPORTED,
              "pkm_column_sum: dtypes %d -> %d not supported (float32, bfloat16, float16 are)", dtype, out_dtype);
  const int epv = dtype == PKM_DTYPE_F32 ? 4 : 8;
  PKM_REQUIRE(rows >= 0 && cols >= 1 && cols < (1 << 30), PKM_ERR_INVALID_ARGUMENT,
              "pkm_column_sum: bad sizes rows=%lld cols=%lld", (long long)rows, (long long)cols);
  PKM_REQUIRE(out != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_column_sum: null output");
  hipStream_t st = (hipStream_t)stream;
  const int C = (int)cols;
  const int64_t nb = (rows + kColRB - 1) / kColRB;
  const bool one = nb == 1;  // one block of rows: sums straight to out, no workspace
  const bool bf_in = dtype == PKM_DTYPE_BF16, bf_out = out_dtype == PKM_DTYPE_BF16;
  if (rows > 0) {
    PKM_REQUIRE(x != nullptr && (one || workspace != nullptr), PKM_ERR_INVALID_ARGUMENT,
                "pkm_column_sum: null pointer");
    PKM_REQUIRE((uintptr_t)(one ? nullptr : workspace) % 16 == 0, PKM_ERR_INVALID_ARGUMENT,
                "pkm_column_sum: workspace must be 16-byte aligned");
    PKM_REQUIRE(one || workspace_bytes >= pkm_column_sum_workspace_size(rows, cols), PKM_ERR_WORKSPACE,
                "pkm_column_sum: workspace of %zu bytes, %zu needed", workspace_bytes,
                pkm_column_sum_workspace_size(rows, cols));
    PKM_REQUIRE(nb < 65536, PKM_ERR_UNSUPPORTED, "pkm_column_sum: %lld rows exceed the partial grid",
                (long long)rows);
    float* part = one ? nullptr : (float*)workspace;
    const bool vec = C % epv == 0 && (uintptr_t)x % 16 == 0 && dtype != PKM_DTYPE_F16 && out_dtype != PKM_DTYPE_F16;
    if (vec) {
      const dim3 pgrid((unsigned)((C / epv + 255) / 256), (unsigned)nb);
#define PKM_COLSUM_P(TI, TO) \
  hipLaunchKernelGGL((colsum_partial_kernel<TI, TO>), pgrid, dim3(256), 0, st, (const TI*)x, rows, C, part, (TO*)out)
      if (bf_in && bf_out) PKM_COLSUM_P(bf16_t, bf16_t);
      else if (bf_in) PKM_COLSUM_P(bf16_t, float);
      else if (bf_out) PKM_COLSUM_P(float, bf16_t);
      else PKM_COLSUM_P(float, float);
#undef PKM_COLSUM_P
    } else {
      const dim3 pgrid((unsigned)((C + 255) / 256), (unsigned)nb);
      hipLaunchKernelGGL(colsum_partial_scalar_kernel, pgrid, dim3(256), 0, st, x, dtype, rows, C, part, out,
                         out_dtype);
    }
    if (one) return pkm_check_launch("pkm_column_sum");
  }
  // the partials in block order (no rows: out = 0, a sum over no partials)
  const dim3 rgrid((unsigned)((C + 63) / 64));
  hipLaunchKernelGGL(colsum_reduce_kernel, rgrid, dim3(256), 0, st, (const float*)workspace, nb, C, out, out_dtype);
  return pkm_check_launch("pkm_column_sum");
}

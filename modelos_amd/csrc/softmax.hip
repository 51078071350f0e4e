// Softmax of the selected product-key scores, forward and backward, gfx950
// (HashingMemory.forward, pkm/memory.py:218:
//   scores = F.softmax(scores.float(), dim=-1).type_as(scores)).
//
//   m    = max_j x[i, j]
//   p_j  = exp(x[i, j] - m) / sum_k exp(x[i, k] - m)         float32
//   y    = T(p)
// and, given dy, the gradient autograd forms through .float(), softmax and
// .type_as:
//   dx[i, j] = T(p_j * (dy_j - sum_k dy_k * p_k))            float32, p recomputed
// T is float32, bfloat16 or float16. Float32 / bfloat16 rows of 16, 32, 64 or
// 128 bytes are read as 16-byte vectors by a group of 1-8 lanes (sums in
// column order within a lane, the lanes' partials combined by a fixed xor
// tree); other rows of at most 64 float32 / bfloat16 entries by one lane
// each, in column order; longer rows (the fast-weight memory's softmax over
// heads x top-k, up to kSmMaxCols entries) and float16 rows by a wave each
// (lane l sums columns l, l + 64, ... in order, then a fixed xor tree).
#include "pkm_common.h"

namespace pkm {

constexpr int kSmLaneCols = 64;  // longest row one lane handles
constexpr int kSmMaxCols = 65536;

template <typename T, int MAXC>
__device__ __forceinline__ void sm_load_row(const T* __restrict__ row, int cols, float* v) {
#pragma unroll
  for (int j = 0; j < MAXC; ++j)
    if (j < cols) v[j] = sizeof(T) == 4 ? ((const float*)row)[j] : bf16_to_f32(((const uint16_t*)row)[j]);
}

template <typename T>
__device__ __forceinline__ void sm_store(T* __restrict__ row, int j, float v) {
  if (sizeof(T) == 4)
    ((float*)row)[j] = v;
  else
    ((uint16_t*)row)[j] = (uint16_t)f32_to_bf16_bits(v);
}

// p[j] = softmax of v[0, cols) (float32, column-order sums)
template <int MAXC>
__device__ __forceinline__ void sm_probs(const float* v, int cols, float* p) {
  float m = v[0];
#pragma unroll
  for (int j = 1; j < MAXC; ++j)
    if (j < cols) m = v[j] > m ? v[j] : m;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    if (j < cols) {
      p[j] = expf(v[j] - m);
      s += p[j];
    }
  }
#pragma unroll
  for (int j = 0; j < MAXC; ++j)
    if (j < cols) p[j] = p[j] / s;
}

template <typename T, int MAXC>
__global__ __launch_bounds__(256) void softmax_fwd_kernel(const T* __restrict__ x, int64_t rows, int cols,
                                                          T* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows) return;
  float v[MAXC], p[MAXC];
  sm_load_row<T, MAXC>(x + i * cols, cols, v);
  sm_probs<MAXC>(v, cols, p);
#pragma unroll
  for (int j = 0; j < MAXC; ++j)
    if (j < cols) sm_store<T>(y + i * cols, j, p[j]);
}

template <typename T, int MAXC>
__global__ __launch_bounds__(256) void softmax_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                                                          int64_t rows, int cols, T* __restrict__ dx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows) return;
  const int nc = cols;  // <= MAXC (dispatch)
  float v[MAXC], p[MAXC], g[MAXC];
  sm_load_row<T, MAXC>(x + i * cols, nc, v);
  sm_probs<MAXC>(v, nc, p);
  sm_load_row<T, MAXC>(dy + i * cols, nc, g);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXC; ++j)
    if (j < nc) s += g[j] * p[j];
#pragma unroll
  for (int j = 0; j < MAXC; ++j)
    if (j < nc) sm_store<T>(dx + i * cols, j, p[j] * (g[j] - s));
}

// Row of LPR 16-byte vectors per lane group (LPR lanes, consecutive).
template <int LPR>
__device__ __forceinline__ float sm_group_max(float v) {
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) {
    const float t = __shfl_xor(v, o);
    v = t > v ? t : v;
  }
  return v;
}
template <int LPR>
__device__ __forceinline__ float sm_group_sum(float v) {
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T, int LPR>
__device__ __forceinline__ void sm_vec_probs(const uint4& raw, float* p) {
  constexpr int EPV = VecTraits<T>::EPV;
  float f[EPV];
  VecTraits<T>::unpack(raw, f);
  float m = f[0];
#pragma unroll
  for (int k = 1; k < EPV; ++k) m = f[k] > m ? f[k] : m;
  m = sm_group_max<LPR>(m);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < EPV; ++k) {
    p[k] = expf(f[k] - m);
    s += p[k];
  }
  s = sm_group_sum<LPR>(s);
#pragma unroll
  for (int k = 0; k < EPV; ++k) p[k] = p[k] / s;
}

template <typename T, int LPR>
__global__ __launch_bounds__(256) void softmax_fwd_vec_kernel(const uint4* __restrict__ x, int64_t rows,
                                                              uint4* __restrict__ y) {
  constexpr int EPV = VecTraits<T>::EPV;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = gid / LPR < rows;  // every lane of a group takes part in the shuffles
  const uint4 raw = valid ? x[gid] : make_uint4(0u, 0u, 0u, 0u);
  float p[EPV];
  sm_vec_probs<T, LPR>(raw, p);
  if (valid) y[gid] = VecTraits<T>::pack(p);
}

template <typename T, int LPR>
__global__ __launch_bounds__(256) void softmax_bwd_vec_kernel(const uint4* __restrict__ dy, const uint4* __restrict__ x,
                                                              int64_t rows, uint4* __restrict__ dx) {
  constexpr int EPV = VecTraits<T>::EPV;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = gid / LPR < rows;
  const uint4 raw = valid ? x[gid] : make_uint4(0u, 0u, 0u, 0u);
  const uint4 graw = valid ? dy[gid] : make_uint4(0u, 0u, 0u, 0u);
  float p[EPV], g[EPV];
  sm_vec_probs<T, LPR>(raw, p);
  VecTraits<T>::unpack(graw, g);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < EPV; ++k) s += g[k] * p[k];
  s = sm_group_sum<LPR>(s);
  float o[EPV];
#pragma unroll
  for (int k = 0; k < EPV; ++k) o[k] = p[k] * (g[k] - s);
  if (valid) dx[gid] = VecTraits<T>::pack(o);
}

// ---------------------------------------------------------------------------
// A wave per row: any row length, any of the three dtypes (runtime dtype code).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sm_wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float t = __shfl_xor(v, o);
    v = t > v ? t : v;
  }
  return v;
}
__device__ __forceinline__ float sm_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// m and s of row `base` (max, and sum of exp(x - m)); every lane gets both
__device__ __forceinline__ void sm_wave_stats(const void* __restrict__ x, int dt, int64_t base, int cols, int lane,
                                              float* m_out, float* s_out) {
  float m = -__builtin_inff();
  for (int j = lane; j < cols; j += 64) {
    const float v = load_scalar(x, dt, base + j);
    m = v > m ? v : m;
  }
  m = sm_wave_max(m);
  float s = 0.f;
  for (int j = lane; j < cols; j += 64) s += expf(load_scalar(x, dt, base + j) - m);
  *m_out = m;
  *s_out = sm_wave_sum(s);
}

__global__ __launch_bounds__(256) void softmax_fwd_wave_kernel(const void* __restrict__ x, int64_t rows, int cols,
                                                               int dt, void* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float m, s;
  sm_wave_stats(x, dt, base, cols, lane, &m, &s);
  for (int j = lane; j < cols; j += 64) store_scalar(y, dt, base + j, expf(load_scalar(x, dt, base + j) - m) / s);
}

__global__ __launch_bounds__(256) void softmax_bwd_wave_kernel(const void* __restrict__ dy, const void* __restrict__ x,
                                                               int64_t rows, int cols, int dt, void* __restrict__ dx) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float m, s;
  sm_wave_stats(x, dt, base, cols, lane, &m, &s);
  float gs = 0.f;
  for (int j = lane; j < cols; j += 64)
    gs += load_scalar(dy, dt, base + j) * (expf(load_scalar(x, dt, base + j) - m) / s);
  gs = sm_wave_sum(gs);
  for (int j = lane; j < cols; j += 64) {
    const float p = expf(load_scalar(x, dt, base + j) - m) / s;
    store_scalar(dx, dt, base + j, p * (load_scalar(dy, dt, base + j) - gs));
  }
}

// lanes per row for the vector path (0: scalar path)
static int sm_vec_lanes(int64_t cols, int dtype, const void* a, const void* b, const void* c) {
  const int64_t bytes = cols * (dtype == PKM_DTYPE_BF16 ? 2 : 4);
  if ((((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15) != 0) return 0;
  if (bytes == 16 || bytes == 32 || bytes == 64 || bytes == 128) return (int)(bytes / 16);
  return 0;
}

}  // namespace pkm

using namespace pkm;

namespace {
int sm_check(const char* what, int64_t rows, int64_t cols, int dtype) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16 || dtype == PKM_DTYPE_F16, PKM_ERR_UNSUPPORTED,
              "%s: dtype %d not supported (float32, bfloat16, float16 are)", what, dtype);
  PKM_REQUIRE(rows >= 0 && cols >= 1 && cols <= kSmMaxCols, PKM_ERR_UNSUPPORTED,
              "%s: rows of %lld entries not supported (1 to %d are)", what, (long long)cols, kSmMaxCols);
  PKM_REQUIRE(rows < ((int64_t)1 << 31) && rows * cols < ((int64_t)1 << 40), PKM_ERR_INVALID_ARGUMENT,
              "%s: too many rows / elements", what);
  return PKM_OK;
}
// the wave-per-row kernels take rows longer than one lane holds, and float16
bool sm_wave_path(int64_t cols, int dtype) { return cols > kSmLaneCols || dtype == PKM_DTYPE_F16; }
}  // namespace

extern "C" int pkm_softmax_fwd(const void* x, int64_t rows, int64_t cols, int dtype, void* y, void* stream) {
  int rc = sm_check("pkm_softmax_fwd", rows, cols, dtype);
  if (rc != PKM_OK) return rc;
  if (rows == 0) return PKM_OK;
  PKM_REQUIRE(x && y, PKM_ERR_INVALID_ARGUMENT, "pkm_softmax_fwd: null pointer");
  const dim3 grid((unsigned)((rows + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (sm_wave_path(cols, dtype)) {
    hipLaunchKernelGGL(softmax_fwd_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, rows,
                       (int)cols, dtype, y);
    return pkm_check_launch("pkm_softmax_fwd");
  }
  const int C = (int)cols;
  const int lpr = sm_vec_lanes(cols, dtype, x, y, y);
  if (lpr > 0) {
    const dim3 vgrid((unsigned)((rows * lpr + 255) / 256));
    const bool bf = dtype == PKM_DTYPE_BF16;
#define PKM_SM_FWD(TT, L) \
  hipLaunchKernelGGL((softmax_fwd_vec_kernel<TT, L>), vgrid, dim3(256), 0, st, (const uint4*)x, rows, (uint4*)y)
    if (lpr == 1) { if (bf) PKM_SM_FWD(bf16_t, 1); else PKM_SM_FWD(float, 1); }
    else if (lpr == 2) { if (bf) PKM_SM_FWD(bf16_t, 2); else PKM_SM_FWD(float, 2); }
    else if (lpr == 4) { if (bf) PKM_SM_FWD(bf16_t, 4); else PKM_SM_FWD(float, 4); }
    else { if (bf) PKM_SM_FWD(bf16_t, 8); else PKM_SM_FWD(float, 8); }
#undef PKM_SM_FWD
    return pkm_check_launch("pkm_softmax_fwd");
  }
  if (dtype == PKM_DTYPE_BF16) {
    if (C <= 32)
      hipLaunchKernelGGL((softmax_fwd_kernel<bf16_t, 32>), grid, dim3(256), 0, st, (const bf16_t*)x, rows, C,
                         (bf16_t*)y);
    else
      hipLaunchKernelGGL((softmax_fwd_kernel<bf16_t, 64>), grid, dim3(256), 0, st, (const bf16_t*)x, rows, C,
                         (bf16_t*)y);
  } else {
    if (C <= 32)
      hipLaunchKernelGGL((softmax_fwd_kernel<float, 32>), grid, dim3(256), 0, st, (const float*)x, rows, C,
                         (float*)y);
    else
      hipLaunchKernelGGL((softmax_fwd_kernel<float, 64>), grid, dim3(256), 0, st, (const float*)x, rows, C,
                         (float*)y);
  }
  return pkm_check_launch("pkm_softmax_fwd");
}

extern "C" int pkm_softmax_bwd(const void* dy, const void* x, int64_t rows, int64_t cols, int dtype, void* dx,
                               void* stream) {
  int rc = sm_check("pkm_softmax_bwd", rows, cols, dtype);
  if (rc != PKM_OK) return rc;
  if (rows == 0) return PKM_OK;
  PKM_REQUIRE(dy && x && dx, PKM_ERR_INVALID_ARGUMENT, "pkm_softmax_bwd: null pointer");
  const dim3 grid((unsigned)((rows + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (sm_wave_path(cols, dtype)) {
    hipLaunchKernelGGL(softmax_bwd_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, dy, x, rows,
                       (int)cols, dtype, dx);
    return pkm_check_launch("pkm_softmax_bwd");
  }
  const int C = (int)cols;
  const int lpr = sm_vec_lanes(cols, dtype, dy, x, dx);
  if (lpr > 0) {
    const dim3 vgrid((unsigned)((rows * lpr + 255) / 256));
    const bool bf = dtype == PKM_DTYPE_BF16;
#define PKM_SM_BWD(TT, L)                                                                                       \
  hipLaunchKernelGGL((softmax_bwd_vec_kernel<TT, L>), vgrid, dim3(256), 0, st, (const uint4*)dy, (const uint4*)x, \
                     rows, (uint4*)dx)
    if (lpr == 1) { if (bf) PKM_SM_BWD(bf16_t, 1); else PKM_SM_BWD(float, 1); }
    else if (lpr == 2) { if (bf) PKM_SM_BWD(bf16_t, 2); else PKM_SM_BWD(float, 2); }
    else if (lpr == 4) { if (bf) PKM_SM_BWD(bf16_t, 4); else PKM_SM_BWD(float, 4); }
    else { if (bf) PKM_SM_BWD(bf16_t, 8); else PKM_SM_BWD(float, 8); }
#undef PKM_SM_BWD
    return pkm_check_launch("pkm_softmax_bwd");
  }
  if (dtype == PKM_DTYPE_BF16) {
    if (C <= 32)
      hipLaunchKernelGGL((softmax_bwd_kernel<bf16_t, 32>), grid, dim3(256), 0, st, (const bf16_t*)dy,
                         (const bf16_t*)x, rows, C, (bf16_t*)dx);
    else
      hipLaunchKernelGGL((softmax_bwd_kernel<bf16_t, 64>), grid, dim3(256), 0, st, (const bf16_t*)dy,
                         (const bf16_t*)x, rows, C, (bf16_t*)dx);
  } else {
    if (C <= 32)
      hipLaunchKernelGGL((softmax_bwd_kernel<float, 32>), grid, dim3(256), 0, st, (const float*)dy,
                         (const float*)x, rows, C, (float*)dx);
    else
      hipLaunchKernelGGL((softmax_bwd_kernel<float, 64>), grid, dim3(256), 0, st, (const float*)dy,
                         (const float*)x, rows, C, (float*)dx);
  }
  return pkm_check_launch("pkm_softmax_bwd");
}

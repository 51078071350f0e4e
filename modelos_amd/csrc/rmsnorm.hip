// RMS normalisation of the product-key query (the Qwen3RMSNorm of the query
// network, pkm/memory.py:311 and 341-349), forward and backward, gfx950.
//
//   r[i]    = rsqrt(mean_j x[i, j]^2 + eps)               float32
//   h[i, j] = T(x[i, j] * r[i])                           rounded to the row dtype T
//   y[i, j] = T(w[j] * h[i, j])
// and, given dy, the gradients the reference's autograd forms through those
// ops (pow, mean, rsqrt, mul, the casts):
//   g[i, j]  = T(dy[i, j] * w[j])
//   s[i]     = sum_j g[i, j] * x[i, j]                    float32
//   dx[i, j] = T(g[i, j] * r[i] + x[i, j] * (2 / D) * (-0.5 * s[i] * r[i]^3))
//   dw[j]    = T(sum_i T(dy[i, j] * h[i, j]))             float32 sum
// T is float32 or bfloat16 (x, w, y, dy, dx, dw all of it); r is kept from
// the forward for the backward.
//
// Layout: rows of D elements, row-major. One wave owns a row and holds it in
// registers (16-byte vectors, lane-strided so every load is one coalesced
// 1 KB access), so x is read once by the forward and x, dy once by the dx
// pass. dw is a column reduction over all rows: blocks of 256 threads, one
// 16-byte column vector per thread, sum RB rows each into float32 partials
// [N / RB, D], which a second pass adds in a fixed order (deterministic).
// Rows too long for registers (more than 8 vectors per lane) are read twice.
#include "pkm_common.h"

namespace pkm {

template <typename T>
struct NormIO;
template <>
struct NormIO<float> {
  static __device__ __forceinline__ float round(float v) { return v; }
};
template <>
struct NormIO<bf16_t> {
  static __device__ __forceinline__ float round(float v) { return bf16_to_f32(f32_to_bf16_bits(v)); }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---------------------------------------------------------------------------
// Forward: one wave per row, MAXV vectors of 16 bytes per lane at most.
// ---------------------------------------------------------------------------
template <typename T, int MAXV>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                          int64_t N, int D, float eps, T* __restrict__ y,
                                                          float* __restrict__ rs) {
  constexpr int EPV = VecTraits<T>::EPV;
  constexpr int HV = MAXV > 0 ? MAXV : 1;  // vectors held in registers (MAXV = 0: rows re-read)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const int NV = D / EPV;  // vectors per row
  const T* xr = x + row * D;
  float v[HV][EPV];
  float ss = 0.f;
  if (MAXV > 0) {
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int c = lane + 64 * i;
      if (c < NV) {
        VecTraits<T>::unpack(ld16(xr + c * EPV), v[i]);
#pragma unroll
        for (int e = 0; e < EPV; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
      }
    }
  } else {
    for (int c = lane; c < NV; c += 64) {
      VecTraits<T>::unpack(ld16(xr + c * EPV), v[0]);
#pragma unroll
      for (int e = 0; e < EPV; ++e) ss = __builtin_fmaf(v[0][e], v[0][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss * (1.0f / (float)D) + eps);
  if (lane == 0) rs[row] = r;
  T* yr = y + row * D;
  auto emit = [&](int c, const float* xv) {
    float wv[EPV], o[EPV];
    VecTraits<T>::unpack(ld16(w + c * EPV), wv);
#pragma unroll
    for (int e = 0; e < EPV; ++e) o[e] = wv[e] * NormIO<T>::round(xv[e] * r);
    st16_nt(yr + c * EPV, VecTraits<T>::pack(o));  // streamed out
  };
  if (MAXV > 0) {
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int c = lane + 64 * i;
      if (c < NV) emit(c, v[i]);
    }
  } else {
    for (int c = lane; c < NV; c += 64) {
      VecTraits<T>::unpack(ld16(xr + c * EPV), v[0]);
      emit(c, v[0]);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, dx: one wave per row.
// ---------------------------------------------------------------------------
template <typename T, int MAXV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_dx_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                                                             const T* __restrict__ w, const float* __restrict__ rs,
                                                             int64_t N, int D, T* __restrict__ dx) {
  constexpr int EPV = VecTraits<T>::EPV;
  constexpr int HV = MAXV > 0 ? MAXV : 1;  // vectors held in registers (MAXV = 0: rows re-read)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const int NV = D / EPV;
  const T* xr = x + row * D;
  const T* dyr = dy + row * D;
  float xv[HV][EPV], gv[HV][EPV];
  // g = T(dy * w) of vector c into gv[i], x into xv[i]
  auto load = [&](int c, int i) {
    float dv[EPV], wv[EPV];
    VecTraits<T>::unpack(ld16(xr + c * EPV), xv[i]);
    VecTraits<T>::unpack(ld16(dyr + c * EPV), dv);
    VecTraits<T>::unpack(ld16(w + c * EPV), wv);
#pragma unroll
    for (int e = 0; e < EPV; ++e) gv[i][e] = NormIO<T>::round(dv[e] * wv[e]);
  };
  float s = 0.f;
  if (MAXV > 0) {
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int c = lane + 64 * i;
      if (c < NV) {
        load(c, i);
#pragma unroll
        for (int e = 0; e < EPV; ++e) s = __builtin_fmaf(gv[i][e], xv[i][e], s);
      }
    }
  } else {
    for (int c = lane; c < NV; c += 64) {
      load(c, 0);
#pragma unroll
      for (int e = 0; e < EPV; ++e) s = __builtin_fmaf(gv[0][e], xv[0][e], s);
    }
  }
  s = wave_sum(s);
  const float r = rs[row];
  const float dvar = -0.5f * s * (r * r * r);  // d loss / d (mean x^2 + eps)
  const float k = dvar * (1.0f / (float)D) * 2.0f;
  T* dxr = dx + row * D;
  auto emit = [&](int c, int i) {
    float o[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) o[e] = gv[i][e] * r + xv[i][e] * k;
    *(uint4*)(dxr + c * EPV) = VecTraits<T>::pack(o);
  };
  if (MAXV > 0) {
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int c = lane + 64 * i;
      if (c < NV) emit(c, i);
    }
  } else {
    for (int c = lane; c < NV; c += 64) {
      load(c, 0);
      emit(c, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, dw: float32 partial column sums over RB rows per block.
// ---------------------------------------------------------------------------
constexpr int kNormRB = 64;  // rows per dw partial

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_bwd_dw_partial_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                                                                     const float* __restrict__ rs, int64_t N, int D,
                                                                     float* __restrict__ part) {
  constexpr int EPV = VecTraits<T>::EPV;
  const int NV = D / EPV;
  const int c = blockIdx.x * 256 + threadIdx.x;  // column vector
  const int64_t rb = blockIdx.y;
  if (c >= NV) return;
  float acc[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc[e] = 0.f;
  const int64_t r0 = rb * kNormRB;
  const int64_t r1 = r0 + kNormRB < N ? r0 + kNormRB : N;
  for (int64_t i = r0; i < r1; ++i) {
    float xv[EPV], dv[EPV];
    VecTraits<T>::unpack(ld16(x + i * D + c * EPV), xv);
    VecTraits<T>::unpack(ld16(dy + i * D + c * EPV), dv);
    const float r = rs[i];
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] += NormIO<T>::round(dv[e] * NormIO<T>::round(xv[e] * r));
  }
  float* pr = part + rb * D + c * EPV;
#pragma unroll
  for (int e = 0; e < EPV; e += 4) *(float4*)(pr + e) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
}

// Backward, dx and the dw partials in one pass (rows of at most 64 * 8 vectors):
// a wave takes kFusedRB consecutive rows, one at a time with the next row's x
// and dy in flight, writes dx as rmsnorm_bwd_dx_kernel does and adds
// T(dy * T(x * r)) of its lane columns into float32 partials in row order,
// stored as row block `wave` of part (the partial kernel's sums, over blocks
// of kFusedRB rows).
// ---------------------------------------------------------------------------
constexpr int kFusedRB = 16;

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_bwd_fused_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                                                                const T* __restrict__ w, const float* __restrict__ rs,
                                                                int64_t N, int D, T* __restrict__ dx,
                                                                float* __restrict__ part) {
  constexpr int EPV = VecTraits<T>::EPV;
  constexpr int HV = 8;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t r0 = wave * kFusedRB;
  if (r0 >= N) return;
  const int64_t r1 = r0 + kFusedRB < N ? r0 + kFusedRB : N;
  const int NV = D / EPV;
  uint4 wp[HV];
  float pacc[HV][EPV];
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int c = lane + 64 * i;
    wp[i] = c < NV ? ld16(w + c * EPV) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int e = 0; e < EPV; ++e) pacc[i][e] = 0.f;
  }
  uint4 xa[HV], da[HV], xb[HV], db[HV];
  auto load = [&](int64_t row, uint4 (&xv)[HV], uint4 (&dv)[HV]) {
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int c = lane + 64 * i;
      xv[i] = dv[i] = make_uint4(0u, 0u, 0u, 0u);
      if (c < NV) {
        xv[i] = ld16(x + row * D + c * EPV);
        dv[i] = ld16(dy + row * D + c * EPV);
      }
    }
  };
  auto process = [&](int64_t row, const uint4 (&xv)[HV], const uint4 (&dv)[HV]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      float fx[EPV], fd[EPV], fw[EPV];
      VecTraits<T>::unpack(xv[i], fx);
      VecTraits<T>::unpack(dv[i], fd);
      VecTraits<T>::unpack(wp[i], fw);
#pragma unroll
      for (int e = 0; e < EPV; ++e) s = __builtin_fmaf(NormIO<T>::round(fd[e] * fw[e]), fx[e], s);
    }
    s = wave_sum(s);
    const float r = rs[row];
    const float dvar = -0.5f * s * (r * r * r);  // d loss / d (mean x^2 + eps)
    const float k = dvar * (1.0f / (float)D) * 2.0f;
    T* dxr = dx + row * D;
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int c = lane + 64 * i;
      float fx[EPV], fd[EPV], fw[EPV], o[EPV];
      VecTraits<T>::unpack(xv[i], fx);
      VecTraits<T>::unpack(dv[i], fd);
      VecTraits<T>::unpack(wp[i], fw);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        o[e] = NormIO<T>::round(fd[e] * fw[e]) * r + fx[e] * k;
        pacc[i][e] += NormIO<T>::round(fd[e] * NormIO<T>::round(fx[e] * r));
      }
      if (c < NV) st16_nt(dxr + c * EPV, VecTraits<T>::pack(o));
    }
  };
  load(r0, xa, da);
  for (int64_t row = r0; row < r1; row += 2) {
    if (row + 1 < r1) load(row + 1, xb, db);
    process(row, xa, da);
    if (row + 1 < r1) {
      if (row + 2 < r1) load(row + 2, xa, da);
      process(row + 1, xb, db);
    }
  }
  float* pr = part + wave * D;
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int c = lane + 64 * i;
    if (c < NV) {
#pragma unroll
      for (int e = 0; e < EPV; e += 4)
        *(float4*)(pr + c * EPV + e) = make_float4(pacc[i][e], pacc[i][e + 1], pacc[i][e + 2], pacc[i][e + 3]);
    }
  }
}

// dw[j] = sum over the row blocks b (in order) of part[b, j]: 64 columns per
// block, the partials split over 4 thread slices (each summing a contiguous
// range of blocks, loads kept in flight), the slices added in order.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_bwd_dw_reduce_kernel(const float* __restrict__ part, int64_t nrb,
                                                                    int D, T* __restrict__ dw) {
  __shared__ float ps[4][64];
  const int jl = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + jl;
  const int64_t per = (nrb + 3) / 4;
  const int64_t b0 = sl * per, b1 = b0 + per < nrb ? b0 + per : nrb;
  float s = 0.f;
  if (j < D) {
    int64_t b = b0;
    for (; b + 8 <= b1; b += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(b + u) * D + j];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; b < b1; ++b) s += part[b * D + j];
  }
  ps[sl][jl] = s;
  __syncthreads();
  if (sl == 0 && j < D) {
    const float t = ((ps[0][jl] + ps[1][jl]) + ps[2][jl]) + ps[3][jl];
    if (sizeof(T) == 4)
      ((float*)dw)[j] = t;
    else
      ((uint16_t*)dw)[j] = (uint16_t)f32_to_bf16_bits(t);
  }
}

}  // namespace pkm

using namespace pkm;

namespace {
int norm_check(const char* what, int64_t N, int64_t D, int dtype) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "%s: dtype %d not supported (float32 and bfloat16 are)", what, dtype);
  PKM_REQUIRE(N >= 0 && D >= 1, PKM_ERR_INVALID_ARGUMENT, "%s: bad sizes", what);
  const int epv = dtype == PKM_DTYPE_BF16 ? 8 : 4;
  PKM_REQUIRE(D % epv == 0 && D < (1 << 30), PKM_ERR_UNSUPPORTED, "%s: row length %lld must be a multiple of %d",
              what, (long long)D, epv);
  return PKM_OK;
}
}  // namespace

extern "C" int pkm_rmsnorm_fwd(const void* x, const void* weight, int64_t rows, int64_t dim, int dtype, float eps,
                               void* y, float* rstd, void* stream) {
  int rc = norm_check("pkm_rmsnorm_fwd", rows, dim, dtype);
  if (rc != PKM_OK) return rc;
  if (rows == 0) return PKM_OK;
  PKM_REQUIRE(x && weight && y && rstd, PKM_ERR_INVALID_ARGUMENT, "pkm_rmsnorm_fwd: null pointer");
  PKM_REQUIRE(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)y) % 16 == 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_rmsnorm_fwd: x, weight and y must be 16-byte aligned");
  const int nv = (int)(dim / (dtype == PKM_DTYPE_BF16 ? 8 : 4));
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((rows + 3) / 4));
  const int D = (int)dim;
  if (dtype == PKM_DTYPE_BF16) {
    if (nv <= 64 * 8)
      hipLaunchKernelGGL((rmsnorm_fwd_kernel<bf16_t, 8>), grid, dim3(256), 0, st, (const bf16_t*)x,
                         (const bf16_t*)weight, rows, D, eps, (bf16_t*)y, rstd);
    else
      hipLaunchKernelGGL((rmsnorm_fwd_kernel<bf16_t, 0>), grid, dim3(256), 0, st, (const bf16_t*)x,
                         (const bf16_t*)weight, rows, D, eps, (bf16_t*)y, rstd);
  } else {
    if (nv <= 64 * 8)
      hipLaunchKernelGGL((rmsnorm_fwd_kernel<float, 8>), grid, dim3(256), 0, st, (const float*)x,
                         (const float*)weight, rows, D, eps, (float*)y, rstd);
    else
      hipLaunchKernelGGL((rmsnorm_fwd_kernel<float, 0>), grid, dim3(256), 0, st, (const float*)x,
                         (const float*)weight, rows, D, eps, (float*)y, rstd);
  }
  return pkm_check_launch("pkm_rmsnorm_fwd");
}

extern "C" size_t pkm_rmsnorm_bwd_workspace_size(int64_t rows, int64_t dim) {
  if (rows <= 0 || dim <= 0) return 0;
  return (size_t)((rows + kFusedRB - 1) / kFusedRB) * (size_t)dim * sizeof(float);
}

extern "C" int pkm_rmsnorm_bwd(const void* dy, const void* x, const void* weight, const float* rstd, int64_t rows,
                               int64_t dim, int dtype, void* dx, void* dweight, void* workspace,
                               size_t workspace_bytes, void* stream) {
  int rc = norm_check("pkm_rmsnorm_bwd", rows, dim, dtype);
  if (rc != PKM_OK) return rc;
  PKM_REQUIRE(dweight != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_rmsnorm_bwd: null dweight");
  hipStream_t st = (hipStream_t)stream;
  const int D = (int)dim;
  if (rows == 0) {  // dweight = 0 (a reduction over no partials)
    const dim3 rgrid((unsigned)((D + 63) / 64));
    if (dtype == PKM_DTYPE_BF16)
      hipLaunchKernelGGL((rmsnorm_bwd_dw_reduce_kernel<bf16_t>), rgrid, dim3(256), 0, st, (const float*)nullptr,
                         (int64_t)0, D, (bf16_t*)dweight);
    else
      hipLaunchKernelGGL((rmsnorm_bwd_dw_reduce_kernel<float>), rgrid, dim3(256), 0, st, (const float*)nullptr,
                         (int64_t)0, D, (float*)dweight);
    return pkm_check_launch("pkm_rmsnorm_bwd");
  }
  PKM_REQUIRE(dy && x && weight && rstd && dx && workspace, PKM_ERR_INVALID_ARGUMENT, "pkm_rmsnorm_bwd: null pointer");
  PKM_REQUIRE(((uintptr_t)dy | (uintptr_t)x | (uintptr_t)weight | (uintptr_t)dx | (uintptr_t)workspace) % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_rmsnorm_bwd: buffers must be 16-byte aligned");
  PKM_REQUIRE(workspace_bytes >= pkm_rmsnorm_bwd_workspace_size(rows, dim), PKM_ERR_WORKSPACE,
              "pkm_rmsnorm_bwd: workspace of %zu bytes, %zu needed", workspace_bytes,
              pkm_rmsnorm_bwd_workspace_size(rows, dim));
  const int epv = dtype == PKM_DTYPE_BF16 ? 8 : 4;
  const int nv = D / epv;
  const int64_t nrb = (rows + kNormRB - 1) / kNormRB;
  PKM_REQUIRE(nrb < 65536, PKM_ERR_UNSUPPORTED, "pkm_rmsnorm_bwd: %lld rows exceed the partial grid",
              (long long)rows);
  const dim3 grid((unsigned)((rows + 3) / 4));
  const dim3 pgrid((unsigned)((nv + 255) / 256), (unsigned)nrb);
  const dim3 rgrid((unsigned)((D + 63) / 64));
  float* part = (float*)workspace;
  if (nv <= 64 * 8) {  // dx and the dw partials in one pass, kFusedRB rows per partial
    const int64_t fnrb = (rows + kFusedRB - 1) / kFusedRB;
    const dim3 fgrid((unsigned)((fnrb + 3) / 4));
    if (dtype == PKM_DTYPE_BF16) {
      hipLaunchKernelGGL((rmsnorm_bwd_fused_kernel<bf16_t>), fgrid, dim3(256), 0, st, (const bf16_t*)dy,
                         (const bf16_t*)x, (const bf16_t*)weight, rstd, rows, D, (bf16_t*)dx, part);
      hipLaunchKernelGGL((rmsnorm_bwd_dw_reduce_kernel<bf16_t>), rgrid, dim3(256), 0, st, (const float*)part, fnrb,
                         D, (bf16_t*)dweight);
    } else {
      hipLaunchKernelGGL((rmsnorm_bwd_fused_kernel<float>), fgrid, dim3(256), 0, st, (const float*)dy,
                         (const float*)x, (const float*)weight, rstd, rows, D, (float*)dx, part);
      hipLaunchKernelGGL((rmsnorm_bwd_dw_reduce_kernel<float>), rgrid, dim3(256), 0, st, (const float*)part, fnrb, D,
                         (float*)dweight);
    }
  } else if (dtype == PKM_DTYPE_BF16) {
    hipLaunchKernelGGL((rmsnorm_bwd_dx_kernel<bf16_t, 0>), grid, dim3(256), 0, st, (const bf16_t*)dy,
                       (const bf16_t*)x, (const bf16_t*)weight, rstd, rows, D, (bf16_t*)dx);
    hipLaunchKernelGGL((rmsnorm_bwd_dw_partial_kernel<bf16_t>), pgrid, dim3(256), 0, st, (const bf16_t*)dy,
                       (const bf16_t*)x, rstd, rows, D, part);
    hipLaunchKernelGGL((rmsnorm_bwd_dw_reduce_kernel<bf16_t>), rgrid, dim3(256), 0, st, (const float*)part, nrb, D,
                       (bf16_t*)dweight);
  } else {
    hipLaunchKernelGGL((rmsnorm_bwd_dx_kernel<float, 0>), grid, dim3(256), 0, st, (const float*)dy,
                       (const float*)x, (const float*)weight, rstd, rows, D, (float*)dx);
    hipLaunchKernelGGL((rmsnorm_bwd_dw_partial_kernel<float>), pgrid, dim3(256), 0, st, (const float*)dy,
                       (const float*)x, rstd, rows, D, part);
    hipLaunchKernelGGL((rmsnorm_bwd_dw_reduce_kernel<float>), rgrid, dim3(256), 0, st, (const float*)part, nrb, D,
                       (float*)dweight);
  }
  return pkm_check_launch("pkm_rmsnorm_bwd");
}

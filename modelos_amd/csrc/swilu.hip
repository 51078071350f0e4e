// SwiLU gating of the PKM layer's value output, forward and backward, gfx950
// (pkm/memory.py:229: value_proj(output * F.silu(swilu_projection(input)))).
//
//   a[i]  = T(s[i] / (1 + exp(-s[i])))                 F.silu in T, float32 math
//   h[i]  = T(e[i] * a[i])
// and, given dh, the gradients autograd forms through the product and silu:
//   de[i] = T(dh[i] * a[i])
//   dm[i] = T(dh[i] * e[i])
//   ds[i] = T(dm[i] * sig * (1 + s[i] * (1 - sig)))    sig = 1 / (1 + exp(-s[i]))
// T is float32 or bfloat16 (all tensors alike). One pass each way
// over 16-byte vectors (grid-stride), the n % (elements per vector) tail
// element by element.
#include "pkm_common.h"

namespace pkm {

template <typename T>
__device__ __forceinline__ float sw_round(float v);
template <>
__device__ __forceinline__ float sw_round<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float sw_round<bf16_t>(float v) {
  return bf16_to_f32(f32_to_bf16_bits(v));
}

template <typename T>
struct SwDtype;
template <>
struct SwDtype<float> {
  static constexpr int code = PKM_DTYPE_F32;
};
template <>
struct SwDtype<bf16_t> {
  static constexpr int code = PKM_DTYPE_BF16;
};

__device__ __forceinline__ float sw_sigmoid(float s) { return 1.f / (1.f + expf(-s)); }

template <typename T>
__device__ __forceinline__ float sw_fwd(float e, float s) {
  const float a = sw_round<T>(s / (1.f + expf(-s)));
  return e * a;
}

template <typename T>
__device__ __forceinline__ void sw_bwd(float dh, float e, float s, float& de, float& ds) {
  const float a = sw_round<T>(s / (1.f + expf(-s)));
  de = dh * a;
  const float dm = sw_round<T>(dh * e);
  const float sig = sw_sigmoid(s);
  ds = dm * sig * (1.f + s * (1.f - sig));
}

template <typename T>
__global__ __launch_bounds__(256) void swilu_fwd_kernel(const T* __restrict__ e, const T* __restrict__ s, int64_t n,
                                                        T* __restrict__ h) {
  constexpr int EPV = VecTraits<T>::EPV;
  const int64_t nvec = n / EPV;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    float fe[EPV], fs[EPV], fh[EPV];
    VecTraits<T>::unpack(((const uint4*)e)[v], fe);
    VecTraits<T>::unpack(((const uint4*)s)[v], fs);
#pragma unroll
    for (int k = 0; k < EPV; ++k) fh[k] = sw_fwd<T>(fe[k], fs[k]);
    st16_nt((uint4*)h + v, VecTraits<T>::pack(fh));
  }
  const int64_t i = nvec * EPV + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    constexpr int dt = SwDtype<T>::code;
    store_scalar(h, dt, i, sw_fwd<T>(load_scalar(e, dt, i), load_scalar(s, dt, i)));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swilu_bwd_kernel(const T* __restrict__ dh, const T* __restrict__ e,
                                                        const T* __restrict__ s, int64_t n, T* __restrict__ de,
                                                        T* __restrict__ ds) {
  constexpr int EPV = VecTraits<T>::EPV;
  const int64_t nvec = n / EPV;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    float fdh[EPV], fe[EPV], fs[EPV], fde[EPV], fds[EPV];
    VecTraits<T>::unpack(((const uint4*)dh)[v], fdh);
    VecTraits<T>::unpack(((const uint4*)e)[v], fe);
    VecTraits<T>::unpack(((const uint4*)s)[v], fs);
#pragma unroll
    for (int k = 0; k < EPV; ++k) sw_bwd<T>(fdh[k], fe[k], fs[k], fde[k], fds[k]);
    st16_nt((uint4*)de + v, VecTraits<T>::pack(fde));
    st16_nt((uint4*)ds + v, VecTraits<T>::pack(fds));
  }
  const int64_t i = nvec * EPV + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    constexpr int dt = SwDtype<T>::code;
    float a, b;
    sw_bwd<T>(load_scalar(dh, dt, i), load_scalar(e, dt, i), load_scalar(s, dt, i), a, b);
    store_scalar(de, dt, i, a);
    store_scalar(ds, dt, i, b);
  }
}

// enough 256-thread blocks to cover the vectors (grid-stride above 16 per CU),
// and at least one for the tail
static unsigned sw_blocks(int64_t n, int epv) {
  const int64_t nvec = n / epv;
  int64_t b = (nvec + 255) / 256;
  if (b > 256 * 16) b = 256 * 16;
  return (unsigned)(b < 1 ? 1 : b);
}

static bool sw_aligned(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace pkm

using namespace pkm;

extern "C" int pkm_swilu_fwd(const void* e, const void* s, int64_t n, int dtype, void* h, void* stream) {
  PKM_REQUIRE(n >= 0, PKM_ERR_INVALID_ARGUMENT, "pkm_swilu_fwd: n %lld < 0", (long long)n);
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "pkm_swilu_fwd: dtype %d not supported (float32, bfloat16 are)", dtype);
  if (n == 0) return PKM_OK;
  PKM_REQUIRE(e && s && h, PKM_ERR_INVALID_ARGUMENT, "pkm_swilu_fwd: null pointer");
  PKM_REQUIRE(sw_aligned(e) && sw_aligned(s) && sw_aligned(h), PKM_ERR_INVALID_ARGUMENT,
              "pkm_swilu_fwd: e, s, h must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PKM_DTYPE_F32)
    hipLaunchKernelGGL(swilu_fwd_kernel<float>, dim3(sw_blocks(n, 4)), dim3(256), 0, st, (const float*)e,
                       (const float*)s, n, (float*)h);
  else
    hipLaunchKernelGGL(swilu_fwd_kernel<bf16_t>, dim3(sw_blocks(n, 8)), dim3(256), 0, st, (const bf16_t*)e,
                       (const bf16_t*)s, n, (bf16_t*)h);
  return pkm_check_launch("pkm_swilu_fwd");
}

extern "C" int pkm_swilu_bwd(const void* dh, const void* e, const void* s, int64_t n, int dtype, void* de, void* ds,
                             void* stream) {
  PKM_REQUIRE(n >= 0, PKM_ERR_INVALID_ARGUMENT, "pkm_swilu_bwd: n %lld < 0", (long long)n);
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "pkm_swilu_bwd: dtype %d not supported (float32, bfloat16 are)", dtype);
  if (n == 0) return PKM_OK;
  PKM_REQUIRE(dh && e && s && de && ds, PKM_ERR_INVALID_ARGUMENT, "pkm_swilu_bwd: null pointer");
  PKM_REQUIRE(sw_aligned(dh) && sw_aligned(e) && sw_aligned(s) && sw_aligned(de) && sw_aligned(ds),
              PKM_ERR_INVALID_ARGUMENT, "pkm_swilu_bwd: all tensors must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PKM_DTYPE_F32)
    hipLaunchKernelGGL(swilu_bwd_kernel<float>, dim3(sw_blocks(n, 4)), dim3(256), 0, st, (const float*)dh,
                       (const float*)e, (const float*)s, n, (float*)de, (float*)ds);
  else
    hipLaunchKernelGGL(swilu_bwd_kernel<bf16_t>, dim3(sw_blocks(n, 8)), dim3(256), 0, st, (const bf16_t*)dh,
                       (const bf16_t*)e, (const bf16_t*)s, n, (bf16_t*)de, (bf16_t*)ds);
  return pkm_check_launch("pkm_swilu_bwd");
}

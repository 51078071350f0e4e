// Fast-weight value update of FwPKM in one pass, gfx950
// (FastWeightProductKeyMemory.update_fw, fwpkm/fwpkm.py:334-365, values
// branch with the "sgd" optimizer, update_fw_param at 266-272):
//
//   gs[r, j] = T(T(g[r, j] * scale) / T(cnt[r]))        cnt[r] = occurrences of row r (1 where 0)
//   gc       = grad_clip ? min(max(gs, -1), 1) : gs
//   p'[r, j] = T(p - T(lr * T(gc + T(wd * p))))
// with every product, quotient and sum rounded to the tensor dtype T in the
// reference's order (ATen elementwise ops on T tensors with float scalars),
// and no contraction of a product into a following sum. Outputs: gs (the
// scaled, unclipped gradient the reference returns) and p'. T is float32,
// bfloat16 or float16; 16-byte vectors over rows of D elements.
#include "pkm_common.h"

namespace pkm {

template <typename T>
__device__ __forceinline__ float fw_round(float v) {
  return round_to<T>(v);
}

#pragma clang fp contract(off)
template <typename T>
__global__ __launch_bounds__(256) void fw_sgd_update_kernel(const T* __restrict__ p, const T* __restrict__ g,
                                                            const int64_t* __restrict__ cnt, int64_t K, int D,
                                                            float scale, float lr, float wd, int clip,
                                                            T* __restrict__ gs_out, T* __restrict__ p_out) {
  constexpr int EPV = VecTraits<T>::EPV;
  const uint32_t vpr = (uint32_t)(D / EPV);  // vectors per row
  const uint32_t nvec = (uint32_t)(K * vpr);  // < 2^32 (host check)
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const uint32_t r = v / vpr;
    const int64_t c = cnt[r];
    const float cs = fw_round<T>(c == 0 ? 1.f : (float)c);
    float fp[EPV], fg[EPV], o_g[EPV], o_p[EPV];
    VecTraits<T>::unpack(((const uint4*)p)[v], fp);
    VecTraits<T>::unpack(((const uint4*)g)[v], fg);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const float gs = fw_round<T>(fw_round<T>(fg[e] * scale) / cs);
      float gc = gs;
      if (clip) gc = gc < -1.f ? -1.f : (gc > 1.f ? 1.f : gc);
      const float wp = fw_round<T>(wd * fp[e]);
      const float dp = fw_round<T>(lr * fw_round<T>(gc + wp));
      o_g[e] = gs;
      o_p[e] = fw_round<T>(fp[e] - dp);
    }
    const uint4 wg = VecTraits<T>::pack(o_g), wpv = VecTraits<T>::pack(o_p);
    __builtin_nontemporal_store(u32x4_t{wg.x, wg.y, wg.z, wg.w}, (u32x4_t*)gs_out + v);  // streamed out
    __builtin_nontemporal_store(u32x4_t{wpv.x, wpv.y, wpv.z, wpv.w}, (u32x4_t*)p_out + v);
  }
}
// Backward of the update, the gradients autograd forms for the reference's
// p - lr * (clip(gs) + wd * p), gs = g * scale / cnt, op by op in T:
//   x   = T(lr * -dnew)                     (d of lr * (.))
//   dp  = T(dnew + T(wd * x))               (p - dp and wd * p)
//   dgs = (clip ? x * [-1 <= gs <= 1] : x) (+ dgs_in when given)
//   dg  = T(T(dgs / T(cnt)) * scale)
template <typename T>
__global__ __launch_bounds__(256) void fw_sgd_update_bwd_kernel(const T* __restrict__ dnew, const T* __restrict__ dgs_in,
                                                                const T* __restrict__ gs,
                                                                const int64_t* __restrict__ cnt, int64_t K, int D,
                                                                float scale, float lr, float wd, int clip,
                                                                T* __restrict__ dp_out, T* __restrict__ dg_out) {
  constexpr int EPV = VecTraits<T>::EPV;
  const uint32_t vpr = (uint32_t)(D / EPV);
  const uint32_t nvec = (uint32_t)(K * vpr);
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const uint32_t r = v / vpr;
    const int64_t c = cnt[r];
    const float cs = fw_round<T>(c == 0 ? 1.f : (float)c);
    float fd[EPV], fs[EPV], fi[EPV], o_p[EPV], o_g[EPV];
    VecTraits<T>::unpack(((const uint4*)dnew)[v], fd);
    VecTraits<T>::unpack(((const uint4*)gs)[v], fs);
    if (dgs_in != nullptr) VecTraits<T>::unpack(((const uint4*)dgs_in)[v], fi);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const float x = fw_round<T>(lr * -fd[e]);
      o_p[e] = fw_round<T>(fd[e] + fw_round<T>(wd * x));
      float d = clip ? ((fs[e] >= -1.f && fs[e] <= 1.f) ? x : 0.f) : x;
      if (dgs_in != nullptr) d = fw_round<T>(d + fi[e]);
      o_g[e] = fw_round<T>(fw_round<T>(d / cs) * scale);
    }
    ((uint4*)dp_out)[v] = VecTraits<T>::pack(o_p);
    if (dg_out != nullptr) ((uint4*)dg_out)[v] = VecTraits<T>::pack(o_g);
  }
}
#pragma clang fp contract(on)

}  // namespace pkm

using namespace pkm;

extern "C" int pkm_fw_sgd_update(const void* values, const void* grad, const int64_t* counts, int64_t num_rows,
                                 int64_t dim, int dtype, float scale, float lr, float weight_decay, int grad_clip,
                                 void* scaled_grad, void* new_values, void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16 || dtype == PKM_DTYPE_F16, PKM_ERR_UNSUPPORTED,
              "pkm_fw_sgd_update: dtype %d not supported (float32, bfloat16, float16 are)", dtype);
  const int epv = dtype == PKM_DTYPE_F32 ? 4 : 8;
  PKM_REQUIRE(num_rows >= 0 && dim >= 1 && dim % epv == 0 && dim < (1 << 30), PKM_ERR_UNSUPPORTED,
              "pkm_fw_sgd_update: rows of %lld elements (a positive multiple of %d) not supported", (long long)dim,
              epv);
  if (num_rows == 0) return PKM_OK;
  PKM_REQUIRE(values && grad && counts && scaled_grad && new_values, PKM_ERR_INVALID_ARGUMENT,
              "pkm_fw_sgd_update: null pointer");
  PKM_REQUIRE(((uintptr_t)values | (uintptr_t)grad | (uintptr_t)scaled_grad | (uintptr_t)new_values) % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_fw_sgd_update: values, grad and outputs must be 16-byte aligned");
  const int64_t nvec = num_rows * (dim / epv);
  PKM_REQUIRE(nvec < ((int64_t)1 << 32) - ((int64_t)256 << 12), PKM_ERR_UNSUPPORTED,
              "pkm_fw_sgd_update: table of %lld 16-byte vectors too large", (long long)nvec);
  int64_t blocks = (nvec + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PKM_DTYPE_BF16)
    hipLaunchKernelGGL(fw_sgd_update_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, st, (const bf16_t*)values,
                       (const bf16_t*)grad, counts, num_rows, (int)dim, scale, lr, weight_decay, grad_clip,
                       (bf16_t*)scaled_grad, (bf16_t*)new_values);
  else if (dtype == PKM_DTYPE_F16)
    hipLaunchKernelGGL(fw_sgd_update_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, st, (const f16_t*)values,
                       (const f16_t*)grad, counts, num_rows, (int)dim, scale, lr, weight_decay, grad_clip,
                       (f16_t*)scaled_grad, (f16_t*)new_values);
  else
    hipLaunchKernelGGL(fw_sgd_update_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)values,
                       (const float*)grad, counts, num_rows, (int)dim, scale, lr, weight_decay, grad_clip,
                       (float*)scaled_grad, (float*)new_values);
  return pkm_check_launch("pkm_fw_sgd_update");
}

extern "C" int pkm_fw_sgd_update_bwd(const void* d_new_values, const void* d_scaled_grad, const void* scaled_grad,
                                     const int64_t* counts, int64_t num_rows, int64_t dim, int dtype, float scale,
                                     float lr, float weight_decay, int grad_clip, void* d_values, void* d_grad,
                                     void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16 || dtype == PKM_DTYPE_F16, PKM_ERR_UNSUPPORTED,
              "pkm_fw_sgd_update_bwd: dtype %d not supported (float32, bfloat16, float16 are)", dtype);
  const int epv = dtype == PKM_DTYPE_F32 ? 4 : 8;
  PKM_REQUIRE(num_rows >= 0 && dim >= 1 && dim % epv == 0 && dim < (1 << 30), PKM_ERR_UNSUPPORTED,
              "pkm_fw_sgd_update_bwd: rows of %lld elements (a positive multiple of %d) not supported",
              (long long)dim, epv);
  if (num_rows == 0) return PKM_OK;
  PKM_REQUIRE(d_new_values && scaled_grad && counts && d_values, PKM_ERR_INVALID_ARGUMENT,
              "pkm_fw_sgd_update_bwd: null pointer");
  PKM_REQUIRE(((uintptr_t)d_new_values | (uintptr_t)d_scaled_grad | (uintptr_t)scaled_grad | (uintptr_t)d_values |
               (uintptr_t)d_grad) % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_fw_sgd_update_bwd: tensors must be 16-byte aligned");
  const int64_t nvec = num_rows * (dim / epv);
  PKM_REQUIRE(nvec < ((int64_t)1 << 32) - ((int64_t)256 << 12), PKM_ERR_UNSUPPORTED,
              "pkm_fw_sgd_update_bwd: table of %lld 16-byte vectors too large", (long long)nvec);
  int64_t blocks = (nvec + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PKM_DTYPE_BF16)
    hipLaunchKernelGGL(fw_sgd_update_bwd_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const bf16_t*)d_new_values, (const bf16_t*)d_scaled_grad, (const bf16_t*)scaled_grad, counts,
                       num_rows, (int)dim, scale, lr, weight_decay, grad_clip, (bf16_t*)d_values, (bf16_t*)d_grad);
  else if (dtype == PKM_DTYPE_F16)
    hipLaunchKernelGGL(fw_sgd_update_bwd_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const f16_t*)d_new_values, (const f16_t*)d_scaled_grad, (const f16_t*)scaled_grad, counts,
                       num_rows, (int)dim, scale, lr, weight_decay, grad_clip, (f16_t*)d_values, (f16_t*)d_grad);
  else
    hipLaunchKernelGGL(fw_sgd_update_bwd_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const float*)d_new_values, (const float*)d_scaled_grad, (const float*)scaled_grad, counts,
                       num_rows, (int)dim, scale, lr, weight_decay, grad_clip, (float*)d_values, (float*)d_grad);
  return pkm_check_launch("pkm_fw_sgd_update_bwd");
}

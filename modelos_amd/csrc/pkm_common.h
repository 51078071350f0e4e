// Shared device helpers for the PKM lookup kernels (gfx950 / CDNA4, wave64).
//
// Element types: the value tables, gradients and per-sample weights of the
// product-key memory are float32, bfloat16 or float16.  All arithmetic is
// done in float32; results are rounded to the storage type once, with
// round-to-nearest-even (the rounding ATen applies when it narrows a float32
// accumulator, e.g. pkm/xformer_embeddingbag.py:113 storing the fp32
// accumulator into a bf16 output).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pkm_hip.h"

namespace pkm {

struct bf16_t {
  uint16_t x;
};
typedef _Float16 f16_t;

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) {
  // v_cvt_pk_bf16_f32: round-to-nearest-even, NaN stays NaN.
  __bf16 h = (__bf16)v;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ uint32_t pack2_f16(float lo, float hi) {
  f16_t a = (f16_t)lo, b = (f16_t)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(f16_t, (uint16_t)bits);
}

// Runtime-typed scalar access, used for the small [B, L] tensors (per-sample
// weights and their gradients) whose dtype may differ from the table's.
__device__ __forceinline__ float load_scalar(const void* p, int dt, int64_t i) {
  if (dt == PKM_DTYPE_F32) return ((const float*)p)[i];
  if (dt == PKM_DTYPE_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return f16_bits_to_f32(((const uint16_t*)p)[i]);
}

__device__ __forceinline__ void store_scalar(void* p, int dt, int64_t i, float v) {
  if (dt == PKM_DTYPE_F32) {
    ((float*)p)[i] = v;
  } else if (dt == PKM_DTYPE_BF16) {
    ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
  } else {
    f16_t h = (f16_t)v;
    ((uint16_t*)p)[i] = __builtin_bit_cast(uint16_t, h);
  }
}

// ---------------------------------------------------------------------------
// 16-byte vector traits: EPV elements of type T per 16-byte (dwordx4) access.
// ---------------------------------------------------------------------------
template <typename T>
struct VecTraits;

template <>
struct VecTraits<float> {
  static constexpr int EPV = 4;
  static __device__ __forceinline__ void unpack(const uint4& v, float* f) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
  static __device__ __forceinline__ uint4 pack(const float* f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
  }
};

template <>
struct VecTraits<bf16_t> {
  static constexpr int EPV = 8;
  static __device__ __forceinline__ void unpack(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ uint4 pack(const float* f) {
    return make_uint4(pack2_bf16(f[0], f[1]), pack2_bf16(f[2], f[3]), pack2_bf16(f[4], f[5]), pack2_bf16(f[6], f[7]));
  }
};

template <>
struct VecTraits<f16_t> {
  static constexpr int EPV = 8;
  static __device__ __forceinline__ void unpack(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      f[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
  static __device__ __forceinline__ uint4 pack(const float* f) {
    return make_uint4(pack2_f16(f[0], f[1]), pack2_f16(f[2], f[3]), pack2_f16(f[4], f[5]), pack2_f16(f[6], f[7]));
  }
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *(const uint4*)p; }
__device__ __forceinline__ void st16(void* p, const uint4& v) { *(uint4*)p = v; }
// Streaming store for write-once outputs (dense weight gradient).
__device__ __forceinline__ void st16_nt(void* p, const uint4& v) {
  __builtin_nontemporal_store(v.x, (uint32_t*)p + 0);
  __builtin_nontemporal_store(v.y, (uint32_t*)p + 1);
  __builtin_nontemporal_store(v.z, (uint32_t*)p + 2);
  __builtin_nontemporal_store(v.w, (uint32_t*)p + 3);
}

// ---------------------------------------------------------------------------
// Lane-group broadcast and reduction. A "group" is LPG consecutive lanes of a
// wave64 (LPG a power of two); the source lane index is relative to the group.
// ---------------------------------------------------------------------------
template <int LPG>
__device__ __forceinline__ int bcast_i32(int v, int src) {
  if constexpr (LPG == 64) {
    return __builtin_amdgcn_readlane(v, src);
  } else {
    return __shfl(v, src, LPG);
  }
}

template <int LPG>
__device__ __forceinline__ float bcast_f32(float v, int src) {
  return __int_as_float(bcast_i32<LPG>(__float_as_int(v), src));
}

template <int LPG>
__device__ __forceinline__ int64_t bcast_i64(int64_t v, int src) {
  const uint64_t u = (uint64_t)v;
  const uint32_t lo = (uint32_t)bcast_i32<LPG>((int)(uint32_t)u, src);
  const uint32_t hi = (uint32_t)bcast_i32<LPG>((int)(uint32_t)(u >> 32), src);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Sum over the LPG lanes of a group; every lane of the group gets the total.
// The butterfly order is fixed, so the result is deterministic.
template <int LPG>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = LPG / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, LPG);
  return v;
}

// ---------------------------------------------------------------------------
// Row split over lane groups (host side, defined in eb_fwd.hip): a row of D
// elements is covered by `slices` slices of LPG lanes x VPL 16-byte vectors.
// ---------------------------------------------------------------------------
struct GroupCfg {
  int lpg;
  int vpl;
  int64_t slices;
};
bool choose_group_cfg(int64_t D, int epv, bool single_slice, GroupCfg* c);

// ---------------------------------------------------------------------------
// Error reporting (host side), defined in capi.hip.
// ---------------------------------------------------------------------------
}  // namespace pkm

int pkm_set_error(int code, const char* fmt, ...);
int pkm_check_launch(const char* what);

#define PKM_REQUIRE(cond, code, ...)             \
  do {                                           \
    if (!(cond)) return pkm_set_error((code), __VA_ARGS__); \
  } while (0)

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

#include "pkm_hip.h"

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

// Two floats to a packed bf16 pair in one v_cvt_pk_bf16_f32 (round to
// nearest even, as f32_to_bf16_bits).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
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

// Float32 dot product of two packed bf16 pairs accumulated into c
// (v_dot2_f32_bf16: the bf16 products are exact in float32).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// d + <a, b> over the elements of two 16-byte vectors, float32 accumulation
// (packed dot instructions for 16-bit types).
template <typename T>
__device__ __forceinline__ float vec_dot(const uint4& a, const uint4& b, float d);
template <>
__device__ __forceinline__ float vec_dot<float>(const uint4& a, const uint4& b, float d) {
  d = __builtin_fmaf(__uint_as_float(a.x), __uint_as_float(b.x), d);
  d = __builtin_fmaf(__uint_as_float(a.y), __uint_as_float(b.y), d);
  d = __builtin_fmaf(__uint_as_float(a.z), __uint_as_float(b.z), d);
  return __builtin_fmaf(__uint_as_float(a.w), __uint_as_float(b.w), d);
}
template <>
__device__ __forceinline__ float vec_dot<bf16_t>(const uint4& a, const uint4& b, float d) {
  d = dot2_bf16(a.x, b.x, d);
  d = dot2_bf16(a.y, b.y, d);
  d = dot2_bf16(a.z, b.z, d);
  return dot2_bf16(a.w, b.w, d);
}
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
}
template <>
__device__ __forceinline__ float vec_dot<f16_t>(const uint4& a, const uint4& b, float d) {
  d = dot2_f16(a.x, b.x, d);
  d = dot2_f16(a.y, b.y, d);
  d = dot2_f16(a.z, b.z, d);
  return dot2_f16(a.w, b.w, d);
}

// Rounding of a float32 value to T, returned as float32 (ATen's narrowing of
// a float32 result into a T tensor).
template <typename T>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float round_to<bf16_t>(float v) {
  return bf16_to_f32(f32_to_bf16_bits(v));
}
template <>
__device__ __forceinline__ float round_to<f16_t>(float v) {
  return (float)(f16_t)v;
}

// ---------------------------------------------------------------------------
// A gradient read in its own dtype TG beside a table of dtype TW: one slot
// holds the EPV elements that one 16-byte vector of the table holds, in NV
// 16-byte loads (1 when TG is TW, 2 for a float32 gradient of a 16-bit table).
// ---------------------------------------------------------------------------
template <typename TW, typename TG>
struct GradTraits {
  static constexpr int EPV = VecTraits<TW>::EPV;
  static constexpr int NV = EPV * (int)sizeof(TG) / 16;
  static_assert(NV == 1 || NV == 2, "a gradient slot is one or two 16-byte vectors");
  static __device__ __forceinline__ void unpack(const uint4* v, float* f) {
    if constexpr (NV == 1) {
      VecTraits<TG>::unpack(v[0], f);
    } else {
      VecTraits<float>::unpack(v[0], f);
      VecTraits<float>::unpack(v[1], f + 4);
    }
  }
  static __device__ __forceinline__ void pack(const float* f, uint4* v) {
    if constexpr (NV == 1) {
      v[0] = VecTraits<TG>::pack(f);
    } else {
      v[0] = VecTraits<float>::pack(f);
      v[1] = VecTraits<float>::pack(f + 4);
    }
  }
  // d + <w, g> over one slot: the packed dot instructions when both are of
  // one type, float32 products of the widened table elements otherwise
  static __device__ __forceinline__ float dot(const uint4& w, const uint4* g, float d) {
    if constexpr (NV == 1) {
      return vec_dot<TW>(w, g[0], d);
    } else {
      float wf[EPV], gf[EPV];
      VecTraits<TW>::unpack(w, wf);
      unpack(g, gf);
#pragma unroll
      for (int e = 0; e < EPV; ++e) d = __builtin_fmaf(wf[e], gf[e], d);
      return d;
    }
  }
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *(const uint4*)p; }
__device__ __forceinline__ void st16(void* p, const uint4& v) { *(uint4*)p = v; }
// Streaming store for write-once outputs (dense weight gradient).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// 16-byte load marked non-temporal (read once: streamed through the caches)
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
  const u32x4_t x = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ void st16_nt(void* p, const uint4& v) {
  const u32x4_t x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, (u32x4_t*)p);
}

// 16-byte loads through a buffer resource over one row (wave-uniform base and
// size): a row given size 0 reads zeros without a memory access, in the same
// instruction as a present row (the loads' count does not depend on the data,
// so the compiler's waits on them stay partial). AUX: cache policy (2 = nt).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* row, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(row), (short)0, (int)bytes, 0x00020000);
}
template <int AUX>
__device__ __forceinline__ uint4 ld16_rsrc(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
  return make_uint4(x[0], x[1], x[2], x[3]);
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

// v + (v moved by a DPP pattern); lanes whose row is masked off add 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the LPG lanes of a group; every lane of the group gets the total.
// DPP lane permutes (no LDS traffic) in a fixed order, so the result is
// deterministic: quad swaps, half-row and row mirrors (16-lane rows), then
// row broadcasts across the wave.
template <int LPG>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPG >= 2) v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (LPG >= 4) v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (LPG >= 8) v = dpp_add<0x141>(v);  // row_half_mirror
  if constexpr (LPG >= 16) v = dpp_add<0x140>(v); // row_mirror: every lane holds its row's sum
  if constexpr (LPG == 32) {
    v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    v = (threadIdx.x & 32) ? hi : lo;
  } else if constexpr (LPG == 64) {
    v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  }
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

// Kernel timing for measurement tools (pkm_kernel_timing_begin / _read /
// _end, defined in capi.hip): while timing is on (process-wide), a
// KernelSpan records a HIP event on its stream when it is constructed and
// another when it goes out of scope, so the pair brackets the launches made in
// its scope. Off (the default), it does nothing.
struct KernelSpan {
  KernelSpan(const char* name, hipStream_t st);
  ~KernelSpan();
  KernelSpan(const KernelSpan&) = delete;
  KernelSpan& operator=(const KernelSpan&) = delete;
  long slot;            // record index, -1 when timing is off
  uint64_t generation;  // of the record set the slot belongs to
  hipStream_t stream;
};

#define PKM_REQUIRE(cond, code, ...)             \
  do {                                           \
    if (!(cond)) return pkm_set_error((code), __VA_ARGS__); \
  } while (0)

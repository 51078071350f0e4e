// Weighted embedding-bag forward gather and its double-backward, gfx950.
//
//   out[b, :] = sum_{j<L} psw[b, j] * W[idx[b, j], :]
//
// Semantics follow the reference Triton kernel embedding_bag_k
// (pkm/xformer_embeddingbag.py:97-113): float32 accumulation over j in
// increasing order, one rounding to the table dtype at the end (:113, output
// allocated in weight.dtype at :123).
//
// Mapping (HBM-bound gather): a "lane group" of LPG lanes (LPG = 64: one
// wave) owns one (bag, column-slice) task. Each lane holds VPL 16-byte vectors
// of the slice, so one row read by the group is LPG*VPL*16 contiguous bytes
// (2 KB for a bf16 row of 1024 at LPG=64, VPL=2). The group loads LPG bag
// entries (index + weight) with one coalesced access, broadcasts them lane by
// lane (readlane -> SGPR row base when LPG = 64), and keeps U rows in flight
// before consuming them.
//
// DOT = true is the double backward (fwpkm/xformer_embeddingbag_grad_wrapper.py:55-74):
// the same gather over gbar, plus d_a[b, j] = <gbar[idx[b, j]], g[b]>, a dot
// product against the bag's upstream gradient that the group holds in registers.
// The upstream gradient g and the gathered sum (d_grad_out) are of type TG:
// the table's type, or float32 beside a 16-bit gbar (read in its own dtype,
// float32 arithmetic as the reference's type promotion gives).
#include "pkm_common.h"

namespace pkm {

// The double backward of the fast-weight values step (pkm_eb_bwd2_sgd): the
// gathered rows are not a stored table gradient but the gradient that
// autograd forms for it through the reference's step
// p' = p - lr * (clip(gs) + wd * p), gs = g * scale / cnt (fwpkm/fwpkm.py:351-365,
// 266-272), from the gradient of p' (dnew) and optionally of gs (dgs):
//   x  = T(lr * -dnew)
//   d  = clip ? (-1 <= gs <= 1 ? x : 0) : x      (+ dgs: d = T(d + dgs))
//   gb = T(T(d / T(max(cnt, 1))) * scale)
// computed row by row as the rows are gathered, so the dense [K, D] gradient
// of the table gradient is never written.
struct SgdBwdArgs {
  const void* gs;         // [K, D] scaled gradient (read when clip)
  const void* dgs;        // [K, D] its upstream gradient, or NULL
  const int32_t* counts;  // [K] lookups per row
  float scale, lr;
  int clip;
};

#pragma clang fp contract(off)
template <typename TW, int NE>
__device__ __forceinline__ void sgd_bwd_row(float* f, uint32_t cnt, const float* fs, const float* fi,
                                            const SgdBwdArgs& A) {
  const float cs = round_to<TW>(cnt == 0 ? 1.f : (float)cnt);
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const float x = round_to<TW>(A.lr * -f[e]);
    float d = A.clip ? ((fs[e] >= -1.f && fs[e] <= 1.f) ? x : 0.f) : x;
    if (A.dgs != nullptr) d = round_to<TW>(d + fi[e]);
    f[e] = round_to<TW>(round_to<TW>(d / cs) * A.scale);
  }
}
#pragma clang fp contract(on)

template <int VPL>
struct FwdUnroll {
  static constexpr int U = VPL >= 8 ? 2 : (VPL >= 4 ? 4 : 8);
};

template <typename TW, typename TG, int LPG, int VPL, bool DOT, bool SGDB = false>
__global__ __launch_bounds__(256) void eb_fwd_kernel(const TW* __restrict__ W, int64_t K, int64_t D,
                                                     const int64_t* __restrict__ idx,
                                                     const void* __restrict__ psw, int pdt, int64_t B,
                                                     int64_t L, int64_t S, TG* __restrict__ out,
                                                     const TG* __restrict__ g, void* __restrict__ dot_out,
                                                     int ddt, SgdBwdArgs A) {
  using GT = GradTraits<TW, TG>;
  constexpr int NV = GT::NV;
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int GPW = 64 / LPG;
  constexpr int NE = VPL * EPV;
  constexpr int U = FwdUnroll<VPL>::U;
  constexpr int VSTRIDE = LPG * EPV;  // element distance between a lane's vectors

  const int lane = threadIdx.x & 63;
  const int glane = lane & (LPG - 1);
  const int64_t task = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * GPW + (lane / LPG);
  if (task >= B * S) return;
  const int64_t b = task / S;
  const int64_t s = task - b * S;
  const int64_t col0 = s * (int64_t)(LPG * NE) + (int64_t)glane * EPV;

  float acc[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) acc[e] = 0.f;

  float gv[DOT ? NE : 1];
  if constexpr (DOT) {
    const TG* grow = g + b * D + col0;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      uint4 raw[NV];
#pragma unroll
      for (int h = 0; h < NV; ++h) raw[h] = ld16(grow + v * VSTRIDE + h * (EPV / NV));
      GT::unpack(raw, gv + v * EPV);
    }
  }

  const int64_t pbase = b * L;
  for (int64_t j0 = 0; j0 < L; j0 += LPG) {
    const int n = (int)((L - j0) < LPG ? (L - j0) : LPG);
    int64_t my_r = -1;
    float my_w = 0.f;
    if (glane < n) {
      my_r = idx[pbase + j0 + glane];
      my_w = psw ? load_scalar(psw, pdt, pbase + j0 + glane) : 1.f;
      if (my_r < 0 || my_r >= K) my_r = -1;
    }
    float my_dot = 0.f;
    for (int jj = 0; jj < n; jj += U) {
      uint4 rv[U][VPL];
      int64_t r[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int src = jj + u;
        r[u] = -1;
        w[u] = 0.f;
        if (src < n) {
          r[u] = bcast_i64<LPG>(my_r, src);
          w[u] = bcast_f32<LPG>(my_w, src);
        }
        if (r[u] >= 0) {
          const TW* row = W + r[u] * D + col0;
#pragma unroll
          for (int v = 0; v < VPL; ++v) rv[u][v] = ld16(row + v * VSTRIDE);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (r[u] >= 0) {
          float f[NE];
#pragma unroll
          for (int v = 0; v < VPL; ++v) VecTraits<TW>::unpack(rv[u][v], f + v * EPV);
          if constexpr (SGDB) {
            // the gathered row is dnew: turn it into the table gradient's gradient
            float fs[NE], fi[NE];
            const int64_t ro = r[u] * D + col0;
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
              if (A.clip) VecTraits<TW>::unpack(ld16((const TW*)A.gs + ro + v * VSTRIDE), fs + v * EPV);
              if (A.dgs != nullptr) VecTraits<TW>::unpack(ld16((const TW*)A.dgs + ro + v * VSTRIDE), fi + v * EPV);
            }
            sgd_bwd_row<TW, NE>(f, (uint32_t)A.counts[r[u]], fs, fi, A);
          }
#pragma unroll
          for (int e = 0; e < NE; ++e) acc[e] = __builtin_fmaf(f[e], w[u], acc[e]);
          if constexpr (DOT) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < NE; ++e) d = __builtin_fmaf(f[e], gv[e], d);
            d = group_sum<LPG>(d);
            if (glane == jj + u) my_dot = d;
          }
        }
      }
    }
    if constexpr (DOT) {
      if (dot_out != nullptr && glane < n) store_scalar(dot_out, ddt, pbase + j0 + glane, my_dot);
    }
  }

  TG* orow = out + b * D + col0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    uint4 raw[NV];
    GT::pack(acc + v * EPV, raw);
#pragma unroll
    for (int h = 0; h < NV; ++h) st16(orow + v * VSTRIDE + h * (EPV / NV), raw[h]);
  }
}

// Fallback for a row length that is not a multiple of the 16-byte vector:
// one thread per output element (forward only).
template <typename TW>
__device__ __forceinline__ float load_elem(const TW* p, int64_t i);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float load_elem<bf16_t>(const bf16_t* p, int64_t i) {
  return bf16_to_f32(p[i].x);
}
template <>
__device__ __forceinline__ float load_elem<f16_t>(const f16_t* p, int64_t i) {
  return (float)p[i];
}

template <typename TW>
__global__ __launch_bounds__(256) void eb_fwd_scalar_kernel(const TW* __restrict__ W, int64_t K, int64_t D,
                                                            const int64_t* __restrict__ idx,
                                                            const void* __restrict__ psw, int pdt, int64_t B,
                                                            int64_t L, TW* __restrict__ out, int odt) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= B * D) return;
  const int64_t b = t / D;
  const int64_t c = t - b * D;
  float acc = 0.f;
  for (int64_t j = 0; j < L; ++j) {
    const int64_t r = idx[b * L + j];
    if (r < 0 || r >= K) continue;
    const float w = psw ? load_scalar(psw, pdt, b * L + j) : 1.f;
    acc = __builtin_fmaf(load_elem<TW>(W, r * D + c), w, acc);
  }
  store_scalar(out, odt, t, acc);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Split a row of D elements over lane groups: LPG lanes x VPL vectors x EPV
// elements per slice. single_slice: the whole row must be one slice (needed
// when a kernel reduces over the row, e.g. a dot product).
bool choose_group_cfg(int64_t D, int epv, bool single_slice, GroupCfg* c) {
  if (D <= 0 || D % epv) return false;
  const int64_t nvec = D / epv;
  if (nvec % 64 == 0) {
    const int64_t per = nvec / 64;
    c->lpg = 64;
    if (per <= 8 && (per & (per - 1)) == 0) {
      c->vpl = (int)per;
      c->slices = 1;
      return true;
    }
    if (single_slice) return false;
    for (int vpl = 8; vpl >= 1; vpl >>= 1) {
      if (per % vpl == 0) {
        c->vpl = vpl;
        c->slices = per / vpl;
        return true;
      }
    }
    return false;
  }
  int lpg = 1;
  while (lpg < 32 && nvec % (2 * lpg) == 0) lpg *= 2;
  c->lpg = lpg;
  c->vpl = 1;
  c->slices = nvec / lpg;
  return !single_slice || c->slices == 1;
}

int elem_size(int dt) { return dt == PKM_DTYPE_F32 ? 4 : 2; }

template <typename TW, typename TG, int LPG, int VPL, bool DOT, bool SGDB>
static void launch_fwd(const void* W, int64_t K, int64_t D, const int64_t* idx, const void* psw, int pdt,
                       int64_t B, int64_t L, int64_t S, void* out, const void* g, void* dot_out, int ddt,
                       const SgdBwdArgs& A, hipStream_t stream) {
  constexpr int GPW = 64 / LPG;
  const int64_t tasks = B * S;
  const int64_t per_block = 4 * GPW;
  const unsigned blocks = (unsigned)((tasks + per_block - 1) / per_block);
  KernelSpan span(DOT ? "eb_bwd2" : "eb_fwd", stream);
  hipLaunchKernelGGL((eb_fwd_kernel<TW, TG, LPG, VPL, DOT, SGDB>), dim3(blocks), dim3(256), 0, stream, (const TW*)W, K,
                     D, idx, psw, pdt, B, L, S, (TG*)out, (const TG*)g, dot_out, ddt, A);
}

template <typename TW, bool DOT, typename TG = TW, bool SGDB = false>
static bool dispatch_fwd(const GroupCfg& c, const void* W, int64_t K, int64_t D, const int64_t* idx,
                         const void* psw, int pdt, int64_t B, int64_t L, void* out, const void* g,
                         void* dot_out, int ddt, hipStream_t stream, const SgdBwdArgs& A = SgdBwdArgs{}) {
#define PKM_FWD_CASE(LPG_, VPL_)                                                                      \
  if (c.lpg == LPG_ && c.vpl == VPL_) {                                                               \
    launch_fwd<TW, TG, LPG_, VPL_, DOT, SGDB>(W, K, D, idx, psw, pdt, B, L, c.slices, out, g, dot_out, ddt, A, stream); \
    return true;                                                                                      \
  }
  PKM_FWD_CASE(64, 1)
  PKM_FWD_CASE(64, 2)
  PKM_FWD_CASE(64, 4)
  PKM_FWD_CASE(64, 8)
  PKM_FWD_CASE(32, 1)
  PKM_FWD_CASE(16, 1)
  PKM_FWD_CASE(8, 1)
  PKM_FWD_CASE(4, 1)
  PKM_FWD_CASE(2, 1)
  PKM_FWD_CASE(1, 1)
#undef PKM_FWD_CASE
  return false;
}

static int epv_of(int dt) { return dt == PKM_DTYPE_F32 ? 4 : 8; }

static bool valid_dtype(int dt) { return dt == PKM_DTYPE_F32 || dt == PKM_DTYPE_BF16 || dt == PKM_DTYPE_F16; }

}  // namespace pkm

using namespace pkm;

extern "C" int pkm_eb_fwd(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                          const int64_t* indices, const void* psw, int psw_dtype, int64_t bags, int64_t bag_size,
                          void* out, void* stream) {
  PKM_REQUIRE(valid_dtype(weight_dtype), PKM_ERR_INVALID_ARGUMENT, "pkm_eb_fwd: bad weight dtype %d", weight_dtype);
  PKM_REQUIRE(psw_dtype == PKM_DTYPE_NONE ? psw == nullptr : (valid_dtype(psw_dtype) && (psw != nullptr || bags * bag_size == 0)), PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_fwd: psw pointer / dtype %d mismatch", psw_dtype);
  PKM_REQUIRE(num_rows >= 0 && dim > 0 && bags >= 0 && bag_size >= 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_fwd: bad sizes num_rows=%lld dim=%lld bags=%lld bag_size=%lld", (long long)num_rows,
              (long long)dim, (long long)bags, (long long)bag_size);
  if (bags == 0) return PKM_OK;
  PKM_REQUIRE(out != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_fwd: null output");
  PKM_REQUIRE(bag_size == 0 || (indices != nullptr && (weight != nullptr || num_rows == 0)),
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_fwd: null input");
  hipStream_t st = (hipStream_t)stream;
  GroupCfg c;
  bool ok = false;
  const bool aligned = ((uintptr_t)weight % 16 == 0) && ((uintptr_t)out % 16 == 0);
  if (aligned && choose_group_cfg(dim, epv_of(weight_dtype), false, &c)) {
    if (weight_dtype == PKM_DTYPE_F32)
      ok = dispatch_fwd<float, false>(c, weight, num_rows, dim, indices, psw, psw_dtype, bags, bag_size, out,
                                      nullptr, nullptr, 0, st);
    else if (weight_dtype == PKM_DTYPE_BF16)
      ok = dispatch_fwd<bf16_t, false>(c, weight, num_rows, dim, indices, psw, psw_dtype, bags, bag_size, out,
                                       nullptr, nullptr, 0, st);
    else
      ok = dispatch_fwd<f16_t, false>(c, weight, num_rows, dim, indices, psw, psw_dtype, bags, bag_size, out,
                                      nullptr, nullptr, 0, st);
  }
  if (!ok) {
    const int64_t n = bags * dim;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (weight_dtype == PKM_DTYPE_F32)
      hipLaunchKernelGGL(eb_fwd_scalar_kernel<float>, dim3(blocks), dim3(256), 0, st, (const float*)weight,
                         num_rows, dim, indices, psw, psw_dtype, bags, bag_size, (float*)out, weight_dtype);
    else if (weight_dtype == PKM_DTYPE_BF16)
      hipLaunchKernelGGL(eb_fwd_scalar_kernel<bf16_t>, dim3(blocks), dim3(256), 0, st, (const bf16_t*)weight,
                         num_rows, dim, indices, psw, psw_dtype, bags, bag_size, (bf16_t*)out, weight_dtype);
    else
      hipLaunchKernelGGL(eb_fwd_scalar_kernel<f16_t>, dim3(blocks), dim3(256), 0, st, (const f16_t*)weight,
                         num_rows, dim, indices, psw, psw_dtype, bags, bag_size, (f16_t*)out, weight_dtype);
  }
  return pkm_check_launch("pkm_eb_fwd");
}

extern "C" int pkm_eb_bwd2(const void* gbar, int64_t num_rows, int64_t dim, int gbar_dtype, const int64_t* indices,
                           const void* a, int a_dtype, const void* grad_out, int grad_dtype, int64_t bags,
                           int64_t bag_size, void* d_grad_out, void* d_a, void* stream) {
  PKM_REQUIRE(valid_dtype(gbar_dtype), PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2: bad gbar dtype %d", gbar_dtype);
  const bool wide_grad = grad_dtype == PKM_DTYPE_F32 && gbar_dtype != PKM_DTYPE_F32;
  PKM_REQUIRE(grad_dtype == gbar_dtype || wide_grad, PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd2: grad_out dtype %d with gbar dtype %d (supported: the same dtype, or a float32 "
              "grad_out for a 16-bit gbar)", grad_dtype, gbar_dtype);
  PKM_REQUIRE(a_dtype == PKM_DTYPE_NONE ? a == nullptr : (valid_dtype(a_dtype) && (a != nullptr || bags * bag_size == 0)), PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd2: a pointer / dtype %d mismatch", a_dtype);
  PKM_REQUIRE(num_rows >= 0 && dim > 0 && bags >= 0 && bag_size >= 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd2: bad sizes");
  if (bags == 0) return PKM_OK;
  PKM_REQUIRE(d_grad_out != nullptr && grad_out != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2: null pointer");
  PKM_REQUIRE(a == nullptr || d_a != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2: d_a is null");
  PKM_REQUIRE(bag_size == 0 || (indices != nullptr && (gbar != nullptr || num_rows == 0)),
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2: null input");
  PKM_REQUIRE((uintptr_t)gbar % 16 == 0 && (uintptr_t)grad_out % 16 == 0 && (uintptr_t)d_grad_out % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2: gbar, grad_out and d_grad_out must be 16-byte aligned");
  GroupCfg c;
  PKM_REQUIRE(choose_group_cfg(dim, epv_of(gbar_dtype), true, &c), PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd2: dim %lld not supported (need dim/%d = LPG*VPL with LPG<=64, VPL<=8)",
              (long long)dim, epv_of(gbar_dtype));
  hipStream_t st = (hipStream_t)stream;
  void* dot = a != nullptr ? d_a : nullptr;
#define PKM_BWD2(TW_, TG_)                                                                                        \
  dispatch_fwd<TW_, true, TG_>(c, gbar, num_rows, dim, indices, a, a_dtype, bags, bag_size, d_grad_out, grad_out, dot, \
                               a_dtype, st)
  if (gbar_dtype == PKM_DTYPE_F32)
    PKM_BWD2(float, float);
  else if (gbar_dtype == PKM_DTYPE_BF16)
    wide_grad ? PKM_BWD2(bf16_t, float) : PKM_BWD2(bf16_t, bf16_t);
  else
    wide_grad ? PKM_BWD2(f16_t, float) : PKM_BWD2(f16_t, f16_t);
#undef PKM_BWD2
  return pkm_check_launch("pkm_eb_bwd2");
}

extern "C" int pkm_eb_bwd2_sgd(const void* d_new_values, const void* d_scaled_grad, const void* scaled_grad,
                               const int32_t* counts, int64_t num_rows, int64_t dim, int dtype, float scale, float lr,
                               int grad_clip, const int64_t* indices, const void* a, int a_dtype,
                               const void* grad_out, int64_t bags, int64_t bag_size, void* d_grad_out, void* d_a,
                               void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd2_sgd: dtype %d not supported (float32, bfloat16 are)", dtype);
  PKM_REQUIRE(a_dtype == PKM_DTYPE_NONE ? a == nullptr : (valid_dtype(a_dtype) && (a != nullptr || bags * bag_size == 0)),
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2_sgd: a pointer / dtype %d mismatch", a_dtype);
  PKM_REQUIRE(num_rows >= 0 && dim > 0 && bags >= 0 && bag_size >= 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd2_sgd: bad sizes");
  if (bags == 0) return PKM_OK;
  PKM_REQUIRE(d_grad_out != nullptr && grad_out != nullptr, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd2_sgd: null pointer");
  PKM_REQUIRE(a == nullptr || d_a != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2_sgd: d_a is null");
  PKM_REQUIRE(bag_size == 0 || num_rows == 0 ||
                  (indices != nullptr && d_new_values != nullptr && counts != nullptr &&
                   (!grad_clip || scaled_grad != nullptr)),
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2_sgd: null input");
  PKM_REQUIRE(((uintptr_t)d_new_values | (uintptr_t)d_scaled_grad | (uintptr_t)scaled_grad | (uintptr_t)grad_out |
               (uintptr_t)d_grad_out) % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd2_sgd: tensors must be 16-byte aligned");
  GroupCfg c;
  PKM_REQUIRE(choose_group_cfg(dim, epv_of(dtype), true, &c), PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd2_sgd: dim %lld not supported (need dim/%d = LPG*VPL with LPG<=64, VPL<=8)",
              (long long)dim, epv_of(dtype));
  hipStream_t st = (hipStream_t)stream;
  void* dot = a != nullptr ? d_a : nullptr;
  const SgdBwdArgs A = {scaled_grad, d_scaled_grad, counts, scale, lr, grad_clip};
  if (dtype == PKM_DTYPE_F32)
    dispatch_fwd<float, true, float, true>(c, d_new_values, num_rows, dim, indices, a, a_dtype, bags, bag_size,
                                           d_grad_out, grad_out, dot, a_dtype, st, A);
  else
    dispatch_fwd<bf16_t, true, bf16_t, true>(c, d_new_values, num_rows, dim, indices, a, a_dtype, bags, bag_size,
                                             d_grad_out, grad_out, dot, a_dtype, st, A);
  return pkm_check_launch("pkm_eb_bwd2_sgd");
}

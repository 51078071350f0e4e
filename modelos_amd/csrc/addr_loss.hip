// Marginal-entropy address loss of the fast-weight product-key memory: the
// loss, its gradient with respect to the sub-scores and the key table, and
// the derivative of that key gradient along a direction (what the outer
// backward through an inner update step takes of it), gfx950.
//
// Reference: FastWeightProductKeyMemory.compute_marginal_entropy and
// compute_addr_loss (fwpkm/fwpkm.py:117-147, 233-264), differentiated with
// respect to the keys by update_fw with create_graph (fwpkm/fwpkm.py:274-367),
// on the sub-scores of compute_qk_scores (fwpkm/fwpkm.py:853-869).
//
// Per half c, over the sub-score matrix s [R = tokens x heads rows, n keys],
// row r = t * heads + h:
//   in_rj   = s_rj >= s_r[sel_r[topk - 1]]        (at least the row's topk best)
//   P_rj    = softmax of s_r over the j in the row's mask (0 elsewhere), float32
//   pbar_j  = (1/R) sum_r P_rj
//   H_c     = -sum_j pbar_j log(pbar_j + 1e-8)
//   loss    = w (-H_1 - H_2)
//   a_j     = d loss / d P_rj = w (log(pbar_j + eps) + pbar_j / (pbar_j + eps)) / R
//   dS_rj   = P_rj (a_j - sum_l P_rl a_l)         d loss / d s_rj, rounded to the scores' dtype
// Key gradient, batch b = 2h + c (head h, half c), key j, token t, q_t the
// token's half-query of head h:
//   idw: g_j = 2 sum_t U_tj (q_t - k_j), U_tj = dS_tj / (1e-3 + d2_tj) where d2_tj > 0, else 0,
//        d2_tj = |q_t|^2 + |k_j|^2 - 2 <q_t, k_j>
//   dot: g_j = sum_t dS_tj q_t
// The kernels write U (idw) or dS (dot) as dense rows [2 heads, tokens, n];
// the caller forms sum_t U_tj q_t as a batched GEMM, and hands in the dense
// products <q_t, k_j> (idw) as batched GEMM results too.
//
// Derivative of phi = <gbar, g> (gbar: the outer gradient of the key
// gradient), split the way autograd splits it:
//   through the sub-scores: sigma_tj = d phi / d dS_tj (idw: 2 u_tj e_tj with
//   u = 1 / (1e-3 + d2) where d2 > 0, else 0, e_tj = <q_t - k_j, gbar_j>;
//   dot: <q_t, gbar_j>), and rho = (Hessian of the loss in s) sigma:
//       Pdot_rj = P_rj (sigma_rj - sum_l P_rl sigma_rl)
//       adot_j  = w (1 / (pbar_j + eps) + eps / (pbar_j + eps)^2) ((1/R) sum_r Pdot_rj) / R
//       rho_rj  = Pdot_rj (a_j - sum_l P_rl a_l) + P_rj (adot_j - sum_l (Pdot_rl a_l + P_rl adot_l))
//     written as the sub-scores' gradient (the retrieval's backward carries
//     it on to the query and the keys);
//   directly, dS held fixed:
//     idw: d q_t = 2 (sum_j U_tj gbar_j + sum_j lam_tj (k_j - q_t)),
//          d k_j = 2 (sum_t lam_tj (q_t - k_j) - gbar_j sum_t U_tj),  lam = dS u sigma;
//     the lam terms have the form the retrieval's idw backward gives a
//     sub-score gradient D (2 sum D u (k - q), 2 sum D u (q - k)), so they
//     travel with rho as D = dS sigma: d_s = rho + dS sigma, and what stays
//     direct is 2 U gbar (query) and -2 gbar sum_t U (keys);
//     dot: d q_t = sum_j dS_tj gbar_j,  d k_j = 0;
//   the kernels write U (idw) or dS (dot) rows for the caller's batched GEMM
//   with gbar, from <q_t, gbar_j> handed in as a GEMM result.
//
// Every (t, j) entry is handled independently, so the cost does not depend
// on how many entries tie at a row's threshold (16-bit idw scores tie for
// most of a row). Work split: a wave takes G.rpw tokens of one batch b (1-8,
// chosen for about 16 K waves: the row loop is latency-bound),
// a row at a time; lane l holds the row's entries l, l + 64, ... (NPL of
// them, n <= 64 NPL). Column sums over rows (pbar, the Pdot sums) are
// per-wave register partials, added in wave order within a workgroup and in
// workgroup order by a finalize kernel: every result is deterministic. The
// column sums the key-side products need (sum_t U_tj, sum_t lam_tj) leave the
// row kernels the same way, as per-workgroup partials reduced in order.
//
// The same row layout serves the idw factor of the retrieval's dense
// backward (pkm_idw_grad_coef): with s = -log(1e-3 + d2) the products
// dq = 2 (U K - q rowsum U) and dK = 2 (U^T q - K colsum U) take
// U = dS / (1e-3 + d2) where d2 > 0 (cdist's autograd under
// compute_mode use_mm_for_euclid_dist, fwpkm/fwpkm.py:863-866).
#include <initializer_list>

#include "pkm_common.h"

namespace pkm {
namespace me {

constexpr int kWaves = 8;
constexpr int kMaxRowsPerWave = 8;
constexpr int64_t kTargetWaves = 16384;
constexpr float kEntEps = 1e-8f;
constexpr float kIdwEps = 1e-3f;

template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldf<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float ldf<bf16_t>(const bf16_t* p, int64_t i) {
  return bf16_to_f32(((const uint16_t*)p)[i]);
}
template <>
__device__ __forceinline__ float ldf<f16_t>(const f16_t* p, int64_t i) {
  return (float)p[i];
}

template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void stf<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ __forceinline__ void stf<bf16_t>(bf16_t* p, int64_t i, float v) {
  ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ void stf<f16_t>(f16_t* p, int64_t i, float v) {
  p[i] = (f16_t)v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

struct Geo {
  int64_t tokens;
  int heads, n, topk, wgb, rpw;  // rpw: tokens per wave
  int vec;  // rows read and written as 16-byte vectors (n % 8 == 0, aligned rows)
};

// The wave's batch and first token; workgroup g covers batch g / wgb.
struct WaveJob {
  int b, c, h;
  int64_t t0, t1;
};
__device__ __forceinline__ WaveJob wave_job(const Geo& G) {
  WaveJob J;
  const int g = blockIdx.x;
  J.b = g / G.wgb;
  J.c = J.b & 1;
  J.h = J.b >> 1;
  J.t0 = ((int64_t)(g % G.wgb) * kWaves + (threadIdx.x >> 6)) * G.rpw;
  J.t1 = J.t0 + G.rpw < G.tokens ? J.t0 + G.rpw : G.tokens;
  return J;
}

// Column of lane l's i-th entry of a row: 4 consecutive columns per 16-byte
// vector (entry 4v + e is column 256v + 4l + e) when the rows allow it, else
// column 64i + l.
template <int NPL>
__device__ __forceinline__ int col_of(const Geo& G, int lane, int i) {
  if constexpr (NPL >= 4) {
    if (G.vec) return 256 * (i >> 2) + 4 * lane + (i & 3);
  }
  return 64 * i + lane;
}

template <typename T>
__device__ __forceinline__ void ld4(const T* p, float* f);
template <>
__device__ __forceinline__ void ld4<float>(const float* p, float* f) {
  const float4 v = *(const float4*)p;
  f[0] = v.x;
  f[1] = v.y;
  f[2] = v.z;
  f[3] = v.w;
}
template <>
__device__ __forceinline__ void ld4<bf16_t>(const bf16_t* p, float* f) {
  const uint2 w = *(const uint2*)p;
  f[0] = __uint_as_float(w.x << 16);
  f[1] = __uint_as_float(w.x & 0xffff0000u);
  f[2] = __uint_as_float(w.y << 16);
  f[3] = __uint_as_float(w.y & 0xffff0000u);
}
template <>
__device__ __forceinline__ void ld4<f16_t>(const f16_t* p, float* f) {
  const uint2 w = *(const uint2*)p;
  f[0] = f16_bits_to_f32(w.x & 0xffffu);
  f[1] = f16_bits_to_f32(w.x >> 16);
  f[2] = f16_bits_to_f32(w.y & 0xffffu);
  f[3] = f16_bits_to_f32(w.y >> 16);
}

template <typename T>
__device__ __forceinline__ void st4(T* p, const float* f);
template <>
__device__ __forceinline__ void st4<float>(float* p, const float* f) {
  *(float4*)p = make_float4(f[0], f[1], f[2], f[3]);
}
template <>
__device__ __forceinline__ void st4<bf16_t>(bf16_t* p, const float* f) {
  *(uint2*)p = make_uint2(pack2_bf16(f[0], f[1]), pack2_bf16(f[2], f[3]));
}
template <>
__device__ __forceinline__ void st4<f16_t>(f16_t* p, const float* f) {
  *(uint2*)p = make_uint2(pack2_f16(f[0], f[1]), pack2_f16(f[2], f[3]));
}

// A lane's entries of a row of n (fill outside [0, n)).
template <typename T, int NPL>
__device__ __forceinline__ void load_row(const T* __restrict__ row, const Geo& G, int lane, float fill,
                                         float (&v)[NPL]) {
  if constexpr (NPL >= 4) {
    if (G.vec) {
#pragma unroll
      for (int q = 0; q < NPL / 4; ++q) {
        const int c0 = 256 * q + 4 * lane;
        if (c0 < G.n) {
          ld4<T>(row + c0, v + 4 * q);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * q + e] = fill;
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = 64 * i + lane;
    v[i] = j < G.n ? ldf<T>(row, j) : fill;
  }
}

template <typename T, int NPL>
__device__ __forceinline__ void store_row(T* __restrict__ row, const Geo& G, int lane, const float (&v)[NPL]) {
  if constexpr (NPL >= 4) {
    if (G.vec) {
#pragma unroll
      for (int q = 0; q < NPL / 4; ++q) {
        const int c0 = 256 * q + 4 * lane;
        if (c0 < G.n) st4<T>(row + c0, v + 4 * q);
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = 64 * i + lane;
    if (j < G.n) stf<T>(row, j, v[i]);
  }
}

// P of one row (0 outside its mask) and the mask.
template <typename T, int NPL>
__device__ __forceinline__ void row_probs(const T* __restrict__ srow, const int64_t* __restrict__ selrow,
                                          const Geo& G, int lane, float (&p)[NPL], bool (&on)[NPL]) {
  int64_t kj = selrow[G.topk - 1];
  kj = kj < 0 ? 0 : (kj >= G.n ? G.n - 1 : kj);  // a list entry outside the row reads inside it
  const float kth = ldf<T>(srow, kj);
  float v[NPL];
  load_row<T, NPL>(srow, G, lane, -__builtin_inff(), v);
  float mx = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    on[i] = col_of<NPL>(G, lane, i) < G.n && v[i] >= kth;
    if (on[i]) mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    p[i] = on[i] ? expf(v[i] - mx) : 0.f;
    z += p[i];
  }
  z = wave_sum(z);
#pragma unroll
  for (int i = 0; i < NPL; ++i) p[i] = p[i] / z;
}

// Per-lane column partials of the wave's rows, added in wave order, one row
// of `partial` per workgroup.
template <int NPL>
__device__ __forceinline__ void store_partial(const float (&acc)[NPL], const Geo& G, float* __restrict__ partial) {
  __shared__ float red[kWaves][64 * NPL];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < NPL; ++i) red[wv][col_of<NPL>(G, lane, i)] = acc[i];
  __syncthreads();
  for (int j = threadIdx.x; j < G.n; j += 64 * kWaves) {
    float s = red[0][j];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += red[w][j];
    partial[(int64_t)blockIdx.x * G.n + j] = s;
  }
}

// Pass 1 of the loss: column partials of P.
template <typename T, int NPL>
__global__ __launch_bounds__(64 * kWaves) void me_pbar_kernel(const T* __restrict__ s1, const T* __restrict__ s2,
                                                              const int64_t* __restrict__ sel1,
                                                              const int64_t* __restrict__ sel2, Geo G,
                                                              float* __restrict__ partial) {
  const int lane = threadIdx.x & 63;
  const WaveJob J = wave_job(G);
  const T* s = J.c ? s2 : s1;
  const int64_t* sel = J.c ? sel2 : sel1;
  float acc[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) acc[i] = 0.f;
  for (int64_t t = J.t0; t < J.t1; ++t) {
    const int64_t r = t * G.heads + J.h;
    float p[NPL];
    bool on[NPL];
    row_probs<T, NPL>(s + r * G.n, sel + r * G.topk, G, lane, p, on);
#pragma unroll
    for (int i = 0; i < NPL; ++i) acc[i] += p[i];
  }
  store_partial<NPL>(acc, G, partial);
}

// Sums the partials of each half: workgroup (column block, half c) of
// kFinCols columns x kFinGroups row groups; row group rg adds partial rows rg,
// rg + kFinGroups, ... (heads, then workgroups) and the groups are added in
// order.
//   mode 0: pbar, a, and the block's share of sum_j pbar_j log(pbar_j + eps)
//           (ent_part [2, column blocks]; me_coef_kernel adds the shares);
//   mode 1: adot from the Pdot partials.
constexpr int kFinCols = 16;
constexpr int kFinGroups = 64;
__global__ __launch_bounds__(kFinCols * kFinGroups) void me_finalize_kernel(const float* __restrict__ partial, Geo G,
                                                                            float weight, int mode,
                                                                            float* __restrict__ pbar,
                                                                            float* __restrict__ avec,
                                                                            float* __restrict__ ent_part) {
  const int c = blockIdx.y;
  const int col = threadIdx.x % kFinCols, rg = threadIdx.x / kFinCols;
  const int j = blockIdx.x * kFinCols + col;
  const int rows = G.heads * G.wgb;
  float S = 0.f;
  if (j < G.n) {
#pragma unroll 4
    for (int q = rg; q < rows; q += kFinGroups) {
      const int h = q / G.wgb, g = q - h * G.wgb;
      S += partial[((int64_t)(2 * h + c) * G.wgb + g) * G.n + j];
    }
  }
  __shared__ float red[kFinGroups][kFinCols];
  red[rg][col] = S;
  __syncthreads();
  if (threadIdx.x >= 64) return;  // wave 0 finishes (its first kFinCols lanes own the columns)
  float hs = 0.f;
  if (rg == 0 && j < G.n) {
    float T = red[0][col];
#pragma unroll 8
    for (int k = 1; k < kFinGroups; ++k) T += red[k][col];
    const float R = (float)(G.tokens * G.heads);
    if (mode == 0) {
      const float pb = T * (1.f / R);
      const float lg = logf(pb + kEntEps);
      pbar[c * G.n + j] = pb;
      avec[c * G.n + j] = weight * (lg + pb / (pb + kEntEps)) / R;
      hs = pb * lg;
    } else {
      const float d = pbar[c * G.n + j] + kEntEps;
      avec[c * G.n + j] = weight * (1.f / d + kEntEps / (d * d)) * (T * (1.f / R)) / R;
    }
  }
  if (mode == 0) {
    hs = wave_sum(hs);
    if (threadIdx.x == 0) ent_part[c * gridDim.x + blockIdx.x] = hs;
  }
}

// out[b, j] = sum over the batch's workgroups g, in order, of partial[b * wgb + g][j]
// (row groups rg, rg + kFinGroups, ... summed per thread, the groups added in order).
__global__ __launch_bounds__(kFinCols * kFinGroups) void me_colsum_kernel(const float* __restrict__ partial, Geo G,
                                                                          float* __restrict__ out) {
  const int b = blockIdx.y;
  const int col = threadIdx.x % kFinCols, rg = threadIdx.x / kFinCols;
  const int j = blockIdx.x * kFinCols + col;
  float S = 0.f;
  if (j < G.n) {
#pragma unroll 4
    for (int g = rg; g < G.wgb; g += kFinGroups) S += partial[((int64_t)b * G.wgb + g) * G.n + j];
  }
  __shared__ float red[kFinGroups][kFinCols];
  red[rg][col] = S;
  __syncthreads();
  if (rg == 0 && j < G.n) {
    float T = red[0][col];
#pragma unroll 8
    for (int k = 1; k < kFinGroups; ++k) T += red[k][col];
    out[(int64_t)b * G.n + j] = T;
  }
}

template <typename T, int NPL>
__device__ __forceinline__ void row_dS(const float (&p)[NPL], const float (&av)[NPL], float (&ds)[NPL], float* pa_out) {
  float pa = 0.f;
#pragma unroll
  for (int i = 0; i < NPL; ++i) pa += p[i] * av[i];
  pa = wave_sum(pa);
#pragma unroll
  for (int i = 0; i < NPL; ++i) ds[i] = round_to<T>(p[i] * (av[i] - pa));
  *pa_out = pa;
}

// Pass 2 of the loss: dense coefficient rows (U for idw, dS for dot) and, for
// idw, per-workgroup column partials of U. d2_tj = (|q_t|^2 + |k_j|^2) - 2
// dots_tj from qq [2 heads, tokens], kk [2 heads, n] and dots [2 heads,
// tokens, n] (the same expression and operands as the reference path's
// mm-based distances).
template <typename T, int NPL, bool IDW>
__global__ __launch_bounds__(64 * kWaves) void me_coef_kernel(const T* __restrict__ s1, const T* __restrict__ s2,
                                                              const int64_t* __restrict__ sel1,
                                                              const int64_t* __restrict__ sel2,
                                                              const float* __restrict__ qq,
                                                              const float* __restrict__ kk,
                                                              const float* __restrict__ dots, Geo G,
                                                              const float* __restrict__ avec,
                                                              const float* __restrict__ ent_part,
                                                              float* __restrict__ entropy, float* __restrict__ coef,
                                                              float* __restrict__ partial) {
  const int lane = threadIdx.x & 63;
  if (blockIdx.x == 0 && threadIdx.x < 2) {
    // H_c from the finalize kernel's column-block shares, in block order
    const int nb = (G.n + kFinCols - 1) / kFinCols;
    float h = 0.f;
    for (int k = 0; k < nb; ++k) h += ent_part[threadIdx.x * nb + k];
    entropy[threadIdx.x] = -h;
  }
  const WaveJob J = wave_job(G);
  const T* s = J.c ? s2 : s1;
  const int64_t* sel = J.c ? sel2 : sel1;
  float av[NPL], kv[NPL], csum[NPL];
  load_row<float, NPL>(avec + J.c * G.n, G, lane, 0.f, av);
  if constexpr (IDW) load_row<float, NPL>(kk + (int64_t)J.b * G.n, G, lane, 0.f, kv);
#pragma unroll
  for (int i = 0; i < NPL; ++i) csum[i] = 0.f;
  for (int64_t t = J.t0; t < J.t1; ++t) {
    const int64_t r = t * G.heads + J.h;
    const int64_t bt = (int64_t)J.b * G.tokens + t;
    float p[NPL], ds[NPL], cf[NPL], pa;
    bool on[NPL];
    row_probs<T, NPL>(s + r * G.n, sel + r * G.topk, G, lane, p, on);
    row_dS<T, NPL>(p, av, ds, &pa);
    if constexpr (IDW) {
      const float q2 = qq[bt];
      float dv[NPL];
      load_row<float, NPL>(dots + bt * G.n, G, lane, 0.f, dv);
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const float d2 = (q2 + kv[i]) - 2.f * dv[i];
        cf[i] = on[i] && d2 > 0.f ? ds[i] / (kIdwEps + d2) : 0.f;
        csum[i] += cf[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NPL; ++i) cf[i] = ds[i];
    }
    store_row<float, NPL>(coef + bt * G.n, G, lane, cf);
  }
  // idw: column sums of U (the key gradient's k_j sum_t U_tj term), per workgroup
  if constexpr (IDW) store_partial<NPL>(csum, G, partial);
}

// sigma and u of a row's entries (0 outside the mask): idw sigma = 2 u e with
// e = qg_tj - kg_j (qg = <q_t, gbar_j>, kg = <k_j, gbar_j>); dot sigma = qg_tj.
template <int NPL, bool IDW>
__device__ __forceinline__ void row_sigma(const bool (&on)[NPL], float q2, const float (&kv)[NPL],
                                          const float (&kg)[NPL], const float (&dv)[NPL], const float (&ev)[NPL],
                                          float (&sg)[NPL], float (&uu)[NPL], float (&d2v)[NPL]) {
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    sg[i] = uu[i] = d2v[i] = 0.f;
    if (!on[i]) continue;
    if constexpr (IDW) {
      const float d2 = (q2 + kv[i]) - 2.f * dv[i];
      d2v[i] = d2;
      if (d2 > 0.f) {
        uu[i] = 1.f / (kIdwEps + d2);
        sg[i] = 2.f * uu[i] * (ev[i] - kg[i]);
      }
    } else {
      sg[i] = ev[i];
    }
  }
}

// Pass 1 of the derivative: column partials of Pdot.
template <typename T, int NPL, bool IDW>
__global__ __launch_bounds__(64 * kWaves) void me_hvp1_kernel(const T* __restrict__ s1, const T* __restrict__ s2,
                                                              const int64_t* __restrict__ sel1,
                                                              const int64_t* __restrict__ sel2,
                                                              const float* __restrict__ qq,
                                                              const float* __restrict__ kk,
                                                              const float* __restrict__ kg,
                                                              const float* __restrict__ dots,
                                                              const float* __restrict__ qg, Geo G,
                                                              float* __restrict__ partial) {
  const int lane = threadIdx.x & 63;
  const WaveJob J = wave_job(G);
  const T* s = J.c ? s2 : s1;
  const int64_t* sel = J.c ? sel2 : sel1;
  float kv[NPL], kgv[NPL];
  if constexpr (IDW) {
    load_row<float, NPL>(kk + (int64_t)J.b * G.n, G, lane, 0.f, kv);
    load_row<float, NPL>(kg + (int64_t)J.b * G.n, G, lane, 0.f, kgv);
  }
  float acc[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) acc[i] = 0.f;
  for (int64_t t = J.t0; t < J.t1; ++t) {
    const int64_t r = t * G.heads + J.h;
    const int64_t bt = (int64_t)J.b * G.tokens + t;
    float p[NPL], sg[NPL], uu[NPL], d2v[NPL], dv[NPL], ev[NPL];
    bool on[NPL];
    row_probs<T, NPL>(s + r * G.n, sel + r * G.topk, G, lane, p, on);
    if constexpr (IDW) load_row<float, NPL>(dots + bt * G.n, G, lane, 0.f, dv);
    load_row<float, NPL>(qg + bt * G.n, G, lane, 0.f, ev);
    row_sigma<NPL, IDW>(on, IDW ? qq[bt] : 0.f, kv, kgv, dv, ev, sg, uu, d2v);
    float tau = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) tau += p[i] * sg[i];
    tau = wave_sum(tau);
#pragma unroll
    for (int i = 0; i < NPL; ++i) acc[i] += p[i] * (sg[i] - tau);
  }
  store_partial<NPL>(acc, G, partial);
}

// Pass 2 of the derivative: the sub-scores' gradient (rho, plus dS sigma for
// idw) and the direct term's coefficient rows (U for idw, dS for dot).
template <typename T, int NPL, bool IDW>
__global__ __launch_bounds__(64 * kWaves) void me_hvp2_kernel(const T* __restrict__ s1, const T* __restrict__ s2,
                                                              const int64_t* __restrict__ sel1,
                                                              const int64_t* __restrict__ sel2,
                                                              const float* __restrict__ qq,
                                                              const float* __restrict__ kk,
                                                              const float* __restrict__ kg,
                                                              const float* __restrict__ dots,
                                                              const float* __restrict__ qg, Geo G,
                                                              const float* __restrict__ avec,
                                                              const float* __restrict__ adot, T* __restrict__ d_s1,
                                                              T* __restrict__ d_s2, float* __restrict__ ul) {
  const int lane = threadIdx.x & 63;
  const WaveJob J = wave_job(G);
  const T* s = J.c ? s2 : s1;
  const int64_t* sel = J.c ? sel2 : sel1;
  T* d_s = J.c ? d_s2 : d_s1;
  float av[NPL], ad[NPL], kv[NPL], kgv[NPL];
  load_row<float, NPL>(avec + J.c * G.n, G, lane, 0.f, av);
  load_row<float, NPL>(adot + J.c * G.n, G, lane, 0.f, ad);
  if constexpr (IDW) {
    load_row<float, NPL>(kk + (int64_t)J.b * G.n, G, lane, 0.f, kv);
    load_row<float, NPL>(kg + (int64_t)J.b * G.n, G, lane, 0.f, kgv);
  }
  for (int64_t t = J.t0; t < J.t1; ++t) {
    const int64_t r = t * G.heads + J.h;
    const int64_t bt = (int64_t)J.b * G.tokens + t;
    float p[NPL], ds[NPL], sg[NPL], uu[NPL], d2v[NPL], dv[NPL], ev[NPL], pa;
    bool on[NPL];
    row_probs<T, NPL>(s + r * G.n, sel + r * G.topk, G, lane, p, on);
    row_dS<T, NPL>(p, av, ds, &pa);
    if constexpr (IDW) load_row<float, NPL>(dots + bt * G.n, G, lane, 0.f, dv);
    load_row<float, NPL>(qg + bt * G.n, G, lane, 0.f, ev);
    row_sigma<NPL, IDW>(on, IDW ? qq[bt] : 0.f, kv, kgv, dv, ev, sg, uu, d2v);
    float tau = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) tau += p[i] * sg[i];
    tau = wave_sum(tau);
    float pd[NPL], rho[NPL];
    float beta_dot = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      pd[i] = p[i] * (sg[i] - tau);
      beta_dot += pd[i] * av[i] + p[i] * ad[i];
    }
    beta_dot = wave_sum(beta_dot);
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      rho[i] = pd[i] * (av[i] - pa) + p[i] * (ad[i] - beta_dot);
      if constexpr (IDW) rho[i] += ds[i] * sg[i];  // the lam terms, as a sub-score gradient
    }
    store_row<T, NPL>(d_s + r * G.n, G, lane, rho);
    float* urow = ul + bt * G.n;
    if constexpr (IDW) {
      // U as the loss pass writes it (uu = 0 where d2 <= 0 or outside the mask)
      float U[NPL];
#pragma unroll
      for (int i = 0; i < NPL; ++i) U[i] = uu[i] != 0.f ? ds[i] / (kIdwEps + d2v[i]) : 0.f;
      store_row<float, NPL>(urow, G, lane, U);
    } else {
      store_row<float, NPL>(urow, G, lane, ds);
    }
  }
}

// The idw factor of a dense sub-score gradient dS [batches, tokens, n]:
// U = dS / (1e-3 + d2) where d2 = (qq + kk) - 2 dots > 0, else 0; row sums
// (lane entries in order, then a fixed DPP tree) and per-workgroup column
// partials.
template <typename T, int NPL>
__global__ __launch_bounds__(64 * kWaves) void me_idw_coef_kernel(const T* __restrict__ dS,
                                                                  const float* __restrict__ qq,
                                                                  const float* __restrict__ kk,
                                                                  const float* __restrict__ dots, Geo G,
                                                                  float* __restrict__ U, float* __restrict__ rowsum,
                                                                  float* __restrict__ partial) {
  const int lane = threadIdx.x & 63;
  const WaveJob J = wave_job(G);
  float kv[NPL], csum[NPL];
  load_row<float, NPL>(kk + (int64_t)J.b * G.n, G, lane, 0.f, kv);
#pragma unroll
  for (int i = 0; i < NPL; ++i) csum[i] = 0.f;
  for (int64_t t = J.t0; t < J.t1; ++t) {
    const int64_t bt = (int64_t)J.b * G.tokens + t;
    const float q2 = qq[bt];
    float gv[NPL], dv[NPL], u[NPL];
    load_row<T, NPL>(dS + bt * G.n, G, lane, 0.f, gv);
    load_row<float, NPL>(dots + bt * G.n, G, lane, 0.f, dv);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float d2 = (q2 + kv[i]) - 2.f * dv[i];
      u[i] = col_of<NPL>(G, lane, i) < G.n && d2 > 0.f ? gv[i] / (kIdwEps + d2) : 0.f;
      acc += u[i];
      csum[i] += u[i];
    }
    store_row<float, NPL>(U + bt * G.n, G, lane, u);
    acc = wave_sum(acc);
    if (lane == 0) rowsum[bt] = acc;
  }
  store_partial<NPL>(csum, G, partial);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int64_t kMaxN = 1024;

static int npl_of(int64_t n) {
  const int64_t v = (n + 63) / 64;
  return v <= 1 ? 1 : v <= 2 ? 2 : v <= 4 ? 4 : v <= 8 ? 8 : 16;
}

static int check(const char* fn, int64_t tokens, int64_t heads, int64_t n, int64_t topk, int dtype, int score_type,
                 Geo* G) {
  PKM_REQUIRE(tokens >= 1 && heads >= 1 && n >= 1 && topk >= 1 && topk <= n, PKM_ERR_INVALID_ARGUMENT,
              "%s: bad sizes (tokens %lld, heads %lld, n %lld, topk %lld)", fn, (long long)tokens, (long long)heads,
              (long long)n, (long long)topk);
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16 || dtype == PKM_DTYPE_F16,
              PKM_ERR_INVALID_ARGUMENT, "%s: dtype %d", fn, dtype);
  PKM_REQUIRE(score_type == PKM_SCORE_DOT || score_type == PKM_SCORE_IDW, PKM_ERR_INVALID_ARGUMENT,
              "%s: score type %d", fn, score_type);
  PKM_REQUIRE(n <= kMaxN && heads <= 4096, PKM_ERR_UNSUPPORTED, "%s: n_keys %lld > %lld or heads %lld > 4096", fn,
              (long long)n, (long long)kMaxN, (long long)heads);
  // tokens per wave: about kTargetWaves waves over the 2 heads x tokens rows
  int64_t rpw = 2 * heads * tokens / kTargetWaves;
  rpw = rpw < 1 ? 1 : (rpw > kMaxRowsPerWave ? kMaxRowsPerWave : rpw);
  const int64_t tblocks = (tokens + rpw - 1) / rpw;
  const int64_t wgb = (tblocks + kWaves - 1) / kWaves;
  PKM_REQUIRE(tokens < ((int64_t)1 << 40) && wgb * 2 * heads < ((int64_t)1 << 31), PKM_ERR_INVALID_ARGUMENT,
              "%s: %lld tokens too many", fn, (long long)tokens);
  G->tokens = tokens;
  G->heads = (int)heads;
  G->n = (int)n;
  G->topk = (int)topk;
  G->wgb = (int)wgb;
  G->rpw = (int)rpw;
  G->vec = 0;
  return PKM_OK;
}

// Rows as 16-byte vectors: 4 entries per lane and vector (NPL >= 4), rows of a
// multiple of 8 entries (16-byte row starts for float32, 8-byte for 16-bit),
// every row array 16-byte aligned.
static int vec_ok(int64_t n, std::initializer_list<const void*> rows) {
  if (n % 8 != 0 || npl_of(n) < 4) return 0;
  for (const void* p : rows)
    if (p != nullptr && (uintptr_t)p % 16 != 0) return 0;
  return 1;
}

// partials [2 heads x wgb, n], then the entropy shares [2, column blocks]
static size_t workspace_bytes(const Geo& G) {
  return ((size_t)(2 * G.heads) * (size_t)G.wgb * (size_t)G.n + 2 * (size_t)((G.n + kFinCols - 1) / kFinCols)) *
         sizeof(float);
}
static float* ent_part_of(const Geo& G, float* ws) { return ws + (size_t)(2 * G.heads) * G.wgb * G.n; }
static dim3 fin_grid(const Geo& G) { return dim3((unsigned)((G.n + kFinCols - 1) / kFinCols), 2); }

static dim3 colsum_grid(const Geo& G, int batches) {
  return dim3((unsigned)((G.n + kFinCols - 1) / kFinCols), (unsigned)batches);
}

template <typename T, int NPL>
static void launch_fwd(const Geo& G, int idw, const void* s1, const void* s2, const int64_t* sel1,
                       const int64_t* sel2, const float* qq, const float* kk, const float* dots, float weight,
                       float* entropy, float* coef, float* avec, float* pbar, float* colsum, float* partial,
                       hipStream_t st) {
  const dim3 grid((unsigned)(2 * G.heads * G.wgb)), block(64 * kWaves);
  hipLaunchKernelGGL((me_pbar_kernel<T, NPL>), grid, block, 0, st, (const T*)s1, (const T*)s2, sel1, sel2, G,
                     partial);
  float* ent = ent_part_of(G, partial);
  hipLaunchKernelGGL(me_finalize_kernel, fin_grid(G), dim3(kFinCols * kFinGroups), 0, st, (const float*)partial, G, weight,
                     0, pbar, avec, ent);
  // the coefficient kernel's column partials reuse the pbar partials' space (consumed by the finalize kernel)
  if (idw) {
    hipLaunchKernelGGL((me_coef_kernel<T, NPL, true>), grid, block, 0, st, (const T*)s1, (const T*)s2, sel1, sel2,
                       qq, kk, dots, G, (const float*)avec, (const float*)ent, entropy, coef, partial);
    if (colsum != nullptr)
      hipLaunchKernelGGL(me_colsum_kernel, colsum_grid(G, 2 * G.heads), dim3(kFinCols * kFinGroups), 0, st,
                         (const float*)partial, G, colsum);
  } else {
    hipLaunchKernelGGL((me_coef_kernel<T, NPL, false>), grid, block, 0, st, (const T*)s1, (const T*)s2, sel1, sel2,
                       qq, kk, dots, G, (const float*)avec, (const float*)ent, entropy, coef, partial);
  }
}

template <typename T, int NPL, bool IDW>
static void launch_hvp_t(const Geo& G, const void* s1, const void* s2, const int64_t* sel1, const int64_t* sel2,
                         const float* qq, const float* kk, const float* kg, const float* dots, const float* qg,
                         float weight, const float* avec, float* pbar, float* adot, void* d_s1, void* d_s2,
                         float* ul, float* partial, hipStream_t st) {
  const dim3 grid((unsigned)(2 * G.heads * G.wgb)), block(64 * kWaves);
  hipLaunchKernelGGL((me_hvp1_kernel<T, NPL, IDW>), grid, block, 0, st, (const T*)s1, (const T*)s2, sel1, sel2, qq,
                     kk, kg, dots, qg, G, partial);
  hipLaunchKernelGGL(me_finalize_kernel, fin_grid(G), dim3(kFinCols * kFinGroups), 0, st, (const float*)partial, G, weight,
                     1, pbar, adot, (float*)nullptr);
  hipLaunchKernelGGL((me_hvp2_kernel<T, NPL, IDW>), grid, block, 0, st, (const T*)s1, (const T*)s2, sel1, sel2, qq,
                     kk, kg, dots, qg, G, avec, (const float*)adot, (T*)d_s1, (T*)d_s2, ul);
}

template <typename T, int NPL>
static void launch_hvp(const Geo& G, int idw, const void* s1, const void* s2, const int64_t* sel1,
                       const int64_t* sel2, const float* qq, const float* kk, const float* kg, const float* dots,
                       const float* qg, float weight, const float* avec, float* pbar, float* adot, void* d_s1,
                       void* d_s2, float* ul, float* partial, hipStream_t st) {
  if (idw)
    launch_hvp_t<T, NPL, true>(G, s1, s2, sel1, sel2, qq, kk, kg, dots, qg, weight, avec, pbar, adot, d_s1, d_s2, ul,
                               partial, st);
  else
    launch_hvp_t<T, NPL, false>(G, s1, s2, sel1, sel2, qq, kk, kg, dots, qg, weight, avec, pbar, adot, d_s1, d_s2,
                                ul, partial, st);
}

template <typename T, int NPL>
static void launch_idw(const Geo& G, int batches, const void* dS, const float* qq, const float* kk,
                       const float* dots, float* U, float* rowsum, float* colsum, float* partial, hipStream_t st) {
  hipLaunchKernelGGL((me_idw_coef_kernel<T, NPL>), dim3((unsigned)(batches * G.wgb)), dim3(64 * kWaves), 0, st,
                     (const T*)dS, qq, kk, dots, G, U, rowsum, partial);
  hipLaunchKernelGGL(me_colsum_kernel, colsum_grid(G, batches), dim3(kFinCols * kFinGroups), 0, st, (const float*)partial,
                     G, colsum);
}

#define PKM_ME_DISPATCH(FN, dtype, npl, ...)                                          \
  do {                                                                                \
    if ((dtype) == PKM_DTYPE_F32) {                                                   \
      if (npl == 1) FN<float, 1>(__VA_ARGS__);                                        \
      else if (npl == 2) FN<float, 2>(__VA_ARGS__);                                   \
      else if (npl == 4) FN<float, 4>(__VA_ARGS__);                                   \
      else if (npl == 8) FN<float, 8>(__VA_ARGS__);                                   \
      else FN<float, 16>(__VA_ARGS__);                                                \
    } else if ((dtype) == PKM_DTYPE_BF16) {                                           \
      if (npl == 1) FN<bf16_t, 1>(__VA_ARGS__);                                       \
      else if (npl == 2) FN<bf16_t, 2>(__VA_ARGS__);                                  \
      else if (npl == 4) FN<bf16_t, 4>(__VA_ARGS__);                                  \
      else if (npl == 8) FN<bf16_t, 8>(__VA_ARGS__);                                  \
      else FN<bf16_t, 16>(__VA_ARGS__);                                               \
    } else {                                                                          \
      if (npl == 1) FN<f16_t, 1>(__VA_ARGS__);                                        \
      else if (npl == 2) FN<f16_t, 2>(__VA_ARGS__);                                   \
      else if (npl == 4) FN<f16_t, 4>(__VA_ARGS__);                                   \
      else if (npl == 8) FN<f16_t, 8>(__VA_ARGS__);                                   \
      else FN<f16_t, 16>(__VA_ARGS__);                                                \
    }                                                                                 \
  } while (0)

}  // namespace me
}  // namespace pkm

using namespace pkm;

extern "C" size_t pkm_me_grad_workspace_size(int64_t num_tokens, int64_t heads, int64_t n_keys) {
  me::Geo G;
  if (me::check("pkm_me_grad_workspace_size", num_tokens, heads, n_keys, 1, PKM_DTYPE_F32, PKM_SCORE_DOT, &G) !=
      PKM_OK)
    return 0;
  return me::workspace_bytes(G);
}

extern "C" int pkm_me_grad_fwd(const void* s1, const void* s2, const int64_t* sel1, const int64_t* sel2, int dtype,
                               int64_t num_tokens, int64_t heads, int64_t n_keys, int64_t topk, int score_type,
                               float weight, const float* qq, const float* kk, const float* dots, float* entropy,
                               float* coef, float* avec, float* pbar, float* colsum, void* workspace,
                               size_t workspace_bytes, void* stream) {
  me::Geo G;
  int rc = me::check("pkm_me_grad_fwd", num_tokens, heads, n_keys, topk, dtype, score_type, &G);
  if (rc != PKM_OK) return rc;
  const bool idw = score_type == PKM_SCORE_IDW;
  PKM_REQUIRE(s1 && s2 && sel1 && sel2 && entropy && coef && avec && pbar, PKM_ERR_INVALID_ARGUMENT,
              "pkm_me_grad_fwd: null pointer");
  PKM_REQUIRE(!idw || (qq && kk && dots), PKM_ERR_INVALID_ARGUMENT,
              "pkm_me_grad_fwd: idw scores need qq, kk and dots");
  PKM_REQUIRE(workspace && workspace_bytes >= me::workspace_bytes(G), PKM_ERR_WORKSPACE,
              "pkm_me_grad_fwd: workspace %zu bytes < %zu", workspace_bytes, me::workspace_bytes(G));
  G.vec = me::vec_ok(n_keys, {s1, s2, dots, coef, avec, kk});
  const int npl = me::npl_of(n_keys);
  PKM_ME_DISPATCH(me::launch_fwd, dtype, npl, G, idw ? 1 : 0, s1, s2, sel1, sel2, qq, kk, dots, weight, entropy,
                  coef, avec, pbar, colsum, (float*)workspace, (hipStream_t)stream);
  return pkm_check_launch("pkm_me_grad_fwd");
}

extern "C" int pkm_me_grad_hvp(const void* s1, const void* s2, const int64_t* sel1, const int64_t* sel2, int dtype,
                               int64_t num_tokens, int64_t heads, int64_t n_keys, int64_t topk, int score_type,
                               float weight, const float* qq, const float* kk, const float* kg, const float* dots,
                               const float* qg, const float* avec, const float* pbar, float* adot, void* d_s1,
                               void* d_s2, float* ul, void* workspace, size_t workspace_bytes, void* stream) {
  me::Geo G;
  int rc = me::check("pkm_me_grad_hvp", num_tokens, heads, n_keys, topk, dtype, score_type, &G);
  if (rc != PKM_OK) return rc;
  const bool idw = score_type == PKM_SCORE_IDW;
  PKM_REQUIRE(s1 && s2 && sel1 && sel2 && qg && avec && pbar && adot && d_s1 && d_s2 && ul,
              PKM_ERR_INVALID_ARGUMENT, "pkm_me_grad_hvp: null pointer");
  PKM_REQUIRE(!idw || (qq && kk && kg && dots), PKM_ERR_INVALID_ARGUMENT,
              "pkm_me_grad_hvp: idw scores need qq, kk, kg and dots");
  PKM_REQUIRE(workspace && workspace_bytes >= me::workspace_bytes(G), PKM_ERR_WORKSPACE,
              "pkm_me_grad_hvp: workspace %zu bytes < %zu", workspace_bytes, me::workspace_bytes(G));
  G.vec = me::vec_ok(n_keys, {s1, s2, dots, qg, kk, kg, avec, adot, d_s1, d_s2, ul});
  const int npl = me::npl_of(n_keys);
  PKM_ME_DISPATCH(me::launch_hvp, dtype, npl, G, idw ? 1 : 0, s1, s2, sel1, sel2, qq, kk, kg, dots, qg, weight, avec,
                  (float*)pbar, adot, d_s1, d_s2, ul, (float*)workspace, (hipStream_t)stream);
  return pkm_check_launch("pkm_me_grad_hvp");
}

extern "C" size_t pkm_idw_grad_coef_workspace_size(int64_t batches, int64_t tokens, int64_t n_keys) {
  me::Geo G;
  if (batches < 1 || batches % 2 ||
      me::check("pkm_idw_grad_coef_workspace_size", tokens, batches / 2, n_keys, 1, PKM_DTYPE_F32, PKM_SCORE_IDW,
                &G) != PKM_OK)
    return 0;
  return me::workspace_bytes(G);
}

extern "C" int pkm_idw_grad_coef(const void* dS, int dtype, const float* qq, const float* kk, const float* dots,
                                 int64_t batches, int64_t tokens, int64_t n_keys, float* U, float* rowsum,
                                 float* colsum, void* workspace, size_t workspace_bytes, void* stream) {
  PKM_REQUIRE(batches >= 2 && batches % 2 == 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_idw_grad_coef: batches %lld (2 per head)", (long long)batches);
  me::Geo G;
  const int rc = me::check("pkm_idw_grad_coef", tokens, batches / 2, n_keys, 1, dtype, PKM_SCORE_IDW, &G);
  if (rc != PKM_OK) return rc;
  PKM_REQUIRE(dS && qq && kk && dots && U && rowsum && colsum, PKM_ERR_INVALID_ARGUMENT,
              "pkm_idw_grad_coef: null pointer");
  PKM_REQUIRE(workspace && workspace_bytes >= me::workspace_bytes(G), PKM_ERR_WORKSPACE,
              "pkm_idw_grad_coef: workspace %zu bytes < %zu", workspace_bytes, me::workspace_bytes(G));
  G.vec = me::vec_ok(n_keys, {dS, dots, U, kk});
  const int npl = me::npl_of(n_keys);
  PKM_ME_DISPATCH(me::launch_idw, dtype, npl, G, (int)batches, dS, qq, kk, dots, U, rowsum, colsum,
                  (float*)workspace, (hipStream_t)stream);
  return pkm_check_launch("pkm_idw_grad_coef");
}

// Weighted embedding-bag backward, deterministic, gfx950.
//
//   gW[r, :]  = sum_{(b,j): idx[b,j]==r} psw[b,j] * g[b, :]   (dense, every row written once)
//   gpsw[b,j] = <W[idx[b,j], :], g[b, :]>
//
// Same outputs as the reference reverse-indices backward
// (pkm/xformer_embeddingbag.py:261-386): it histograms the rows (:261-274),
// builds a reverse mapping with an atomic counting-sort scatter (:277-288,
// order inside a row is nondeterministic) and reduces row by row (:291-328),
// reading W and writing gW for all K rows.
//
// This design (own):
//  1. count:   rows histogram with integer atomics (exact), indices outside
//              [0, K) go to a sentinel row K;
//  2. scan:    exclusive scan of the counts -> row offsets (K+2 entries);
//  3. sort:    stable LSD radix sort (8-bit digits) of (row, flat position)
//              pairs. The input is in position order and every pass is stable,
//              so each row's occurrences end up in increasing position order:
//              the float32 sums below have a fixed order, independent of the
//              launch (no float atomics anywhere);
//  4. heavy:   rows with more than T occurrences are cut into fixed chunks of
//              T sorted occurrences; each chunk writes a float32 partial sum
//              (2 slots per chunk: the row running in from the previous chunk
//              and the row starting inside this one);
//  5. rows:    one lane group per row, rows in order: untouched rows get zeros,
//              light rows are reduced in position order while the group holds
//              W[r] in registers for the psw-gradient dot products, heavy rows
//              add their chunk partials in chunk order.
// HBM traffic: W is read once per distinct row, gW written once per row, the
// upstream gradient g (B x D, tens of MB) is re-read per occurrence from
// L2 / Infinity Cache.
#include "pkm_common.h"

namespace pkm {

constexpr int kHeavyT = 256;  // chunk length and light/heavy row threshold

// ---------------------------------------------------------------------------
// Utilities
// ---------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__device__ __forceinline__ uint32_t row_key(int64_t r, int64_t K) {
  return (r >= 0 && r < K) ? (uint32_t)r : (uint32_t)K;
}

__global__ void count_rows_kernel(const int64_t* __restrict__ idx, int64_t N, int64_t K, uint32_t* __restrict__ counts) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < N; p += (int64_t)gridDim.x * blockDim.x)
    atomicAdd(&counts[row_key(idx[p], K)], 1u);
}

__global__ void count_invalid_kernel(const int64_t* __restrict__ idx, int64_t n, int64_t K,
                                     unsigned long long* __restrict__ out) {
  uint32_t c = 0;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < n; p += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx[p];
    c += (r < 0 || r >= K) ? 1u : 0u;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) c += __shfl_xor(c, m);
  if ((threadIdx.x & 63) == 0 && c) atomicAdd(out, (unsigned long long)c);
}

__global__ void zero_i64_kernel(unsigned long long* p) { *p = 0; }

// ---------------------------------------------------------------------------
// Device-wide exclusive scan of uint32 (tiles of 4096 = 256 threads x 16).
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

// Exclusive scan of one value per thread across a 256-thread block.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* total, uint32_t* lds4) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) lds4[w] = x;
  __syncthreads();
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = lds4[i];
    pre += (i < w) ? t : 0u;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return pre + x - v;
}

__global__ __launch_bounds__(256) void scan_reduce_kernel(const uint32_t* __restrict__ in, int64_t n,
                                                          uint32_t* __restrict__ parts) {
  __shared__ uint32_t lds4[4];
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t p = base + (int64_t)i * kScanThreads + threadIdx.x;
    s += p < n ? in[p] : 0u;
  }
  uint32_t tot;
  block_exclusive_scan(s, &tot, lds4);
  if (threadIdx.x == 0) parts[blockIdx.x] = tot;
}

// Single block: exclusive scan of the per-tile sums, in place.
__global__ __launch_bounds__(256) void scan_parts_kernel(uint32_t* __restrict__ parts, int64_t nparts) {
  __shared__ uint32_t lds4[4];
  uint32_t carry = 0;
  for (int64_t base = 0; base < nparts; base += kScanTile) {
    uint32_t v[kScanItems];
    uint32_t s = 0;
    const int64_t p0 = base + (int64_t)threadIdx.x * kScanItems;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      v[i] = (p0 + i < nparts) ? parts[p0 + i] : 0u;
      s += v[i];
    }
    uint32_t tot;
    uint32_t run = carry + block_exclusive_scan(s, &tot, lds4);
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      if (p0 + i < nparts) parts[p0 + i] = run;
      run += v[i];
    }
    carry += tot;
  }
}

// data[i] <- tile prefix + exclusive scan inside the tile; data[n] <- total.
__global__ __launch_bounds__(256) void scan_apply_kernel(uint32_t* __restrict__ data, int64_t n,
                                                         const uint32_t* __restrict__ parts) {
  __shared__ uint32_t lds4[4];
  const int64_t p0 = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    v[i] = (p0 + i < n) ? data[p0 + i] : 0u;
    s += v[i];
  }
  uint32_t tot;
  uint32_t run = parts[blockIdx.x] + block_exclusive_scan(s, &tot, lds4);
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    if (p0 + i < n) data[p0 + i] = run;
    run += v[i];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) data[n] = parts[blockIdx.x] + tot;
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort pass, 8-bit digit, tiles of 4096 (4 waves x 16 x 64).
// Item order inside a tile: wave-major, then round, then lane, so a wave's
// rounds cover consecutive 64-item runs and ranks stay stable.
// ---------------------------------------------------------------------------
constexpr int kRadix = 256;
constexpr int kRadixItems = 16;
constexpr int kRadixTile = 256 * kRadixItems;

template <bool FIRST>
__global__ __launch_bounds__(256) void radix_hist_kernel(const int64_t* __restrict__ idx,
                                                         const uint32_t* __restrict__ keys, int64_t N, int64_t K,
                                                         int shift, uint32_t* __restrict__ hist, int64_t ntiles) {
  __shared__ uint32_t h[kRadix];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kRadixTile;
#pragma unroll 4
  for (int i = 0; i < kRadixItems; ++i) {
    const int64_t p = base + (int64_t)i * 256 + threadIdx.x;
    if (p < N) {
      const uint32_t k = FIRST ? row_key(idx[p], K) : keys[p];
      atomicAdd(&h[(k >> shift) & (kRadix - 1)], 1u);
    }
  }
  __syncthreads();
  hist[(int64_t)threadIdx.x * ntiles + blockIdx.x] = h[threadIdx.x];
}

template <bool FIRST>
__global__ __launch_bounds__(256) void radix_scatter_kernel(const int64_t* __restrict__ idx,
                                                            const uint32_t* __restrict__ keys_in,
                                                            const uint32_t* __restrict__ vals_in, int64_t N,
                                                            int64_t K, int shift, const uint32_t* __restrict__ ofs,
                                                            int64_t ntiles, uint32_t* __restrict__ keys_out,
                                                            uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t wcnt[4][kRadix];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 4; ++i) wcnt[i][threadIdx.x] = 0;
  __syncthreads();

  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t base = (int64_t)blockIdx.x * kRadixTile + (int64_t)w * (kRadixItems * 64);
  uint32_t k[kRadixItems], v[kRadixItems], pre[kRadixItems];
#pragma unroll
  for (int i = 0; i < kRadixItems; ++i) {
    const int64_t p = base + (int64_t)i * 64 + lane;
    const bool valid = p < N;
    k[i] = valid ? (FIRST ? row_key(idx[p], K) : keys_in[p]) : 0u;
    v[i] = valid ? (FIRST ? (uint32_t)p : vals_in[p]) : 0u;
    const uint32_t d = (k[i] >> shift) & (kRadix - 1);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool on = (d >> bit) & 1u;
      const uint64_t bb = __ballot(on);
      peers &= on ? bb : ~bb;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & below);
    const uint32_t old = wcnt[w][d];
    if (valid && rank == 0) wcnt[w][d] = old + (uint32_t)__popcll(peers);
    pre[i] = old + rank;
  }
  __syncthreads();
  {
    const int d = threadIdx.x;
    uint32_t run = ofs[(int64_t)d * ntiles + blockIdx.x];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = wcnt[i][d];
      wcnt[i][d] = run;
      run += t;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kRadixItems; ++i) {
    const int64_t p = base + (int64_t)i * 64 + lane;
    if (p < N) {
      const uint32_t d = (k[i] >> shift) & (kRadix - 1);
      const uint32_t dst = wcnt[w][d] + pre[i];
      keys_out[dst] = k[i];
      vals_out[dst] = v[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Segmented reduction over sorted occurrences.
// ---------------------------------------------------------------------------
template <int VPL>
struct BwdUnroll {
  static constexpr int U = VPL >= 8 ? 2 : (VPL >= 4 ? 4 : 8);
};

// acc += sum over sorted occurrences [i_beg, i_end) (in order) of psw[p] * g[p / L];
// with want_dot, gpsw[p] = <wv, g[p / L]> for each of them.
template <typename TW, int LPG, int VPL>
__device__ __forceinline__ void reduce_occurrences(uint32_t i_beg, uint32_t i_end, const uint32_t* __restrict__ svals,
                                                   const void* __restrict__ psw, int pdt,
                                                   const TW* __restrict__ g, int64_t D, uint32_t L32,
                                                   int64_t col0, int glane, const float* wv, bool want_dot,
                                                   void* __restrict__ gpsw, float* acc) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int U = BwdUnroll<VPL>::U;
  constexpr int VSTRIDE = LPG * EPV;
  for (uint32_t i0 = i_beg; i0 < i_end; i0 += LPG) {
    const int n = (int)((i_end - i0) < (uint32_t)LPG ? (i_end - i0) : (uint32_t)LPG);
    uint32_t my_p = 0, my_b = 0;
    float my_w = 0.f;
    if (glane < n) {
      my_p = svals[i0 + glane];
      my_b = my_p / L32;
      my_w = psw ? load_scalar(psw, pdt, my_p) : 1.f;
    }
    float my_dot = 0.f;
    for (int jj = 0; jj < n; jj += U) {
      uint4 gvec[U][VPL];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        w[u] = 0.f;
        if (jj + u < n) {
          const uint32_t b = (uint32_t)bcast_i32<LPG>((int)my_b, jj + u);
          w[u] = bcast_f32<LPG>(my_w, jj + u);
          const TW* grow = g + (int64_t)b * D + col0;
#pragma unroll
          for (int v = 0; v < VPL; ++v) gvec[u][v] = ld16(grow + v * VSTRIDE);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (jj + u < n) {
          float f[NE];
#pragma unroll
          for (int v = 0; v < VPL; ++v) VecTraits<TW>::unpack(gvec[u][v], f + v * EPV);
#pragma unroll
          for (int e = 0; e < NE; ++e) acc[e] = __builtin_fmaf(f[e], w[u], acc[e]);
          if (want_dot) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < NE; ++e) d = __builtin_fmaf(wv[e], f[e], d);
            d = group_sum<LPG>(d);
            if (glane == jj + u) my_dot = d;
          }
        }
      }
    }
    if (want_dot && glane < n) store_scalar(gpsw, pdt, my_p, my_dot);
  }
}

template <typename TW, int LPG, int VPL>
__device__ __forceinline__ void load_row_f32(const TW* __restrict__ row, int64_t col0, float* f) {
  constexpr int EPV = VecTraits<TW>::EPV;
#pragma unroll
  for (int v = 0; v < VPL; ++v) VecTraits<TW>::unpack(ld16(row + col0 + v * LPG * EPV), f + v * EPV);
}

// Heavy rows: chunk c = sorted occurrences [c*T, (c+1)*T). A row with more
// than T occurrences always contains the chunk's first or last occurrence.
template <typename TW, int LPG, int VPL>
__global__ __launch_bounds__(256) void eb_bwd_heavy_kernel(const TW* __restrict__ W, int64_t K, int64_t D,
                                                           const void* __restrict__ psw, int pdt,
                                                           const TW* __restrict__ g, uint32_t L32,
                                                           const uint32_t* __restrict__ offs,
                                                           const uint32_t* __restrict__ skeys,
                                                           const uint32_t* __restrict__ svals, uint32_t N,
                                                           int64_t nchunks, float* __restrict__ partials,
                                                           void* __restrict__ gpsw) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int GPW = 64 / LPG;
  const int lane = threadIdx.x & 63;
  const int glane = lane & (LPG - 1);
  const int64_t c = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * GPW + (lane / LPG);
  if (c >= nchunks) return;
  const uint32_t i_beg = (uint32_t)(c * kHeavyT);
  const uint32_t i_end = (uint32_t)((int64_t)i_beg + kHeavyT < (int64_t)N ? i_beg + kHeavyT : N);
  const int64_t col0 = (int64_t)glane * EPV;
  const bool want_dot = psw != nullptr;
  const uint32_t cand[2] = {skeys[i_beg], skeys[i_end - 1]};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t r = cand[t];
    if (t == 1 && r == cand[0]) break;
    if (r >= (uint32_t)K) continue;  // sentinel row: handled by the rows kernel
    const uint32_t rb = offs[r], re = offs[r + 1];
    if (re - rb <= (uint32_t)kHeavyT) continue;
    const uint32_t s_beg = rb > i_beg ? rb : i_beg;
    const uint32_t s_end = re < i_end ? re : i_end;
    const int slot = rb > i_beg ? 1 : 0;
    float wv[NE];
    if (want_dot) load_row_f32<TW, LPG, VPL>(W + (int64_t)r * D, col0, wv);
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    reduce_occurrences<TW, LPG, VPL>(s_beg, s_end, svals, psw, pdt, g, D, L32, col0, glane, wv, want_dot, gpsw, acc);
    float* prow = partials + (2 * c + slot) * D + col0;
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int h = 0; h < EPV; h += 4) st16(prow + v * LPG * EPV + h, VecTraits<float>::pack(acc + v * EPV + h));
  }
}

template <typename TW, int LPG, int VPL>
__global__ __launch_bounds__(256) void eb_bwd_rows_kernel(const TW* __restrict__ W, int64_t K, int64_t D,
                                                          const void* __restrict__ psw, int pdt,
                                                          const TW* __restrict__ g, uint32_t L32,
                                                          const uint32_t* __restrict__ offs,
                                                          const uint32_t* __restrict__ svals,
                                                          const float* __restrict__ partials, int rows_per_group,
                                                          TW* __restrict__ gW, void* __restrict__ gpsw) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int GPW = 64 / LPG;
  constexpr int VSTRIDE = LPG * EPV;
  const int lane = threadIdx.x & 63;
  const int glane = lane & (LPG - 1);
  const int64_t grp = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * GPW + (lane / LPG);
  const int64_t r0 = grp * rows_per_group;
  if (r0 > K) return;
  const int64_t r1 = (r0 + rows_per_group < K + 1) ? r0 + rows_per_group : K + 1;
  const int64_t col0 = (int64_t)glane * EPV;
  const bool want_dot = psw != nullptr;

  for (int64_t r = r0; r < r1; ++r) {
    const uint32_t beg = offs[r], end = offs[r + 1];
    const uint32_t cnt = end - beg;
    if (r == K) {
      // occurrences whose index was out of range: zero psw-gradient
      if (want_dot)
        for (uint32_t i = beg + glane; i < end; i += LPG) store_scalar(gpsw, pdt, svals[i], 0.f);
      continue;
    }
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    if (cnt > (uint32_t)kHeavyT) {
      const uint32_t c_first = beg / kHeavyT, c_last = (end - 1) / kHeavyT;
      for (uint32_t c = c_first; c <= c_last; ++c) {
        const int slot = (c == c_first && beg != c * (uint32_t)kHeavyT) ? 1 : 0;
        const float* prow = partials + (2 * (int64_t)c + slot) * D + col0;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
#pragma unroll
          for (int h = 0; h < EPV; h += 4) {
            float f[4];
            VecTraits<float>::unpack(ld16(prow + v * VSTRIDE + h), f);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[v * EPV + h + e] += f[e];
          }
        }
      }
    } else if (cnt > 0) {
      float wv[NE];
      if (want_dot) load_row_f32<TW, LPG, VPL>(W + r * D, col0, wv);
      reduce_occurrences<TW, LPG, VPL>(beg, end, svals, psw, pdt, g, D, L32, col0, glane, wv, want_dot, gpsw, acc);
    }
    TW* orow = gW + r * D + col0;
#pragma unroll
    for (int v = 0; v < VPL; ++v) st16_nt(orow + v * VSTRIDE, VecTraits<TW>::pack(acc + v * EPV));
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct BwdLayout {
  size_t counts, keys0, vals0, keys1, vals1, hist, parts, partials, total;
  int64_t ntiles, nchunks;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

static BwdLayout bwd_layout(int64_t K, int64_t D, int64_t N) {
  BwdLayout l;
  size_t off = 0;
  l.counts = off;
  off += align256((size_t)(K + 2) * 4);
  l.keys0 = off;
  off += align256((size_t)N * 4);
  l.vals0 = off;
  off += align256((size_t)N * 4);
  l.keys1 = off;
  off += align256((size_t)N * 4);
  l.vals1 = off;
  off += align256((size_t)N * 4);
  l.ntiles = cdiv(N, kRadixTile);
  l.hist = off;
  off += align256((size_t)(kRadix * l.ntiles + 1) * 4);
  const int64_t scan_n = (K + 1) > kRadix * l.ntiles ? (K + 1) : kRadix * l.ntiles;
  l.parts = off;
  off += align256((size_t)(cdiv(scan_n, kScanTile) + 1) * 4);
  l.nchunks = cdiv(N, kHeavyT);
  l.partials = off;
  off += align256((size_t)(2 * l.nchunks) * (size_t)D * 4);
  l.total = off;
  return l;
}

// In-place exclusive scan of data[0..n) with data[n] <- total.
static void device_exclusive_scan(uint32_t* data, int64_t n, uint32_t* parts, hipStream_t st) {
  const int64_t tiles = cdiv(n, kScanTile);
  hipLaunchKernelGGL(scan_reduce_kernel, dim3((unsigned)tiles), dim3(kScanThreads), 0, st, data, n, parts);
  hipLaunchKernelGGL(scan_parts_kernel, dim3(1), dim3(kScanThreads), 0, st, parts, tiles);
  hipLaunchKernelGGL(scan_apply_kernel, dim3((unsigned)tiles), dim3(kScanThreads), 0, st, data, n, parts);
}

static unsigned grid_for(int64_t n, int threads, int64_t cap = 65536) {
  int64_t b = cdiv(n, threads);
  if (b < 1) b = 1;
  return (unsigned)(b < cap ? b : cap);
}

template <typename TW, int LPG, int VPL>
static void launch_reduce(const void* W, int64_t K, int64_t D, const void* psw, int pdt, const void* g, int64_t L,
                          const uint32_t* offs, const uint32_t* skeys, const uint32_t* svals, int64_t N,
                          const BwdLayout& l, float* partials, void* gW, void* gpsw, hipStream_t st) {
  constexpr int GPW = 64 / LPG;
  const int64_t groups_per_block = 4 * GPW;
  if (N > 0) {
    const unsigned hb = (unsigned)cdiv(l.nchunks, groups_per_block);
    hipLaunchKernelGGL((eb_bwd_heavy_kernel<TW, LPG, VPL>), dim3(hb), dim3(256), 0, st, (const TW*)W, K, D, psw, pdt,
                       (const TW*)g, (uint32_t)L, offs, skeys, svals, (uint32_t)N, l.nchunks, partials, gpsw);
  }
  const int rows_per_group = 4;
  const int64_t groups = cdiv(K + 1, rows_per_group);
  const unsigned rb = (unsigned)cdiv(groups, groups_per_block);
  hipLaunchKernelGGL((eb_bwd_rows_kernel<TW, LPG, VPL>), dim3(rb), dim3(256), 0, st, (const TW*)W, K, D, psw, pdt,
                     (const TW*)g, (uint32_t)L, offs, svals, (const float*)partials, rows_per_group, (TW*)gW, gpsw);
}

template <typename TW>
static bool dispatch_reduce(const GroupCfg& c, const void* W, int64_t K, int64_t D, const void* psw, int pdt,
                            const void* g, int64_t L, const uint32_t* offs, const uint32_t* skeys,
                            const uint32_t* svals, int64_t N, const BwdLayout& l, float* partials, void* gW,
                            void* gpsw, hipStream_t st) {
#define PKM_RED_CASE(LPG_, VPL_)                                                                           \
  if (c.lpg == LPG_ && c.vpl == VPL_) {                                                                    \
    launch_reduce<TW, LPG_, VPL_>(W, K, D, psw, pdt, g, L, offs, skeys, svals, N, l, partials, gW, gpsw, st); \
    return true;                                                                                           \
  }
  PKM_RED_CASE(64, 1)
  PKM_RED_CASE(64, 2)
  PKM_RED_CASE(64, 4)
  PKM_RED_CASE(64, 8)
  PKM_RED_CASE(32, 1)
  PKM_RED_CASE(16, 1)
  PKM_RED_CASE(8, 1)
  PKM_RED_CASE(4, 1)
  PKM_RED_CASE(2, 1)
  PKM_RED_CASE(1, 1)
#undef PKM_RED_CASE
  return false;
}

static bool valid_dt(int dt) { return dt == PKM_DTYPE_F32 || dt == PKM_DTYPE_BF16 || dt == PKM_DTYPE_F16; }

}  // namespace pkm

using namespace pkm;

extern "C" size_t pkm_eb_bwd_workspace_size(int64_t num_rows, int64_t dim, int64_t bags, int64_t bag_size) {
  if (num_rows < 0 || dim <= 0 || bags < 0 || bag_size < 0) return 0;
  return bwd_layout(num_rows, dim, bags * bag_size).total;
}

extern "C" int pkm_eb_bwd(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype, const int64_t* indices,
                          const void* psw, int psw_dtype, const void* grad_out, int grad_dtype, int64_t bags,
                          int64_t bag_size, void* grad_weight, void* grad_psw, void* workspace,
                          size_t workspace_bytes, void* stream) {
  PKM_REQUIRE(valid_dt(weight_dtype), PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: bad weight dtype %d", weight_dtype);
  PKM_REQUIRE(grad_dtype == weight_dtype, PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd: grad_out dtype %d differs from weight dtype %d", grad_dtype, weight_dtype);
  PKM_REQUIRE(psw == nullptr ? psw_dtype == PKM_DTYPE_NONE : valid_dt(psw_dtype), PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd: psw pointer / dtype %d mismatch", psw_dtype);
  PKM_REQUIRE(num_rows >= 0 && dim > 0 && bags >= 0 && bag_size >= 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd: bad sizes num_rows=%lld dim=%lld bags=%lld bag_size=%lld", (long long)num_rows,
              (long long)dim, (long long)bags, (long long)bag_size);
  const int64_t N = bags * bag_size;
  PKM_REQUIRE(N < ((int64_t)1 << 32) - 1 && num_rows < ((int64_t)1 << 31) - 1, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd: bags*bag_size=%lld or num_rows=%lld too large", (long long)N, (long long)num_rows);
  if (num_rows == 0) {
    // nothing to write for the weight; every lookup is out of range
    PKM_REQUIRE(psw == nullptr || N == 0 || grad_psw != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: null grad_psw");
  }
  PKM_REQUIRE(grad_weight != nullptr || num_rows == 0, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: null grad_weight");
  PKM_REQUIRE(N == 0 || (indices != nullptr && grad_out != nullptr), PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd: null indices / grad_out");
  PKM_REQUIRE(psw == nullptr || N == 0 || (grad_psw != nullptr && (weight != nullptr || num_rows == 0)),
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: null weight / grad_psw");
  const int epv = weight_dtype == PKM_DTYPE_F32 ? 4 : 8;
  GroupCfg c;
  PKM_REQUIRE(choose_group_cfg(dim, epv, true, &c), PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd: dim %lld not supported (need dim/%d = LPG*VPL with LPG<=64, VPL<=8)", (long long)dim, epv);
  const BwdLayout l = bwd_layout(num_rows, dim, N);
  PKM_REQUIRE(workspace != nullptr && workspace_bytes >= l.total, PKM_ERR_WORKSPACE,
              "pkm_eb_bwd: workspace of %zu bytes given, %zu needed", workspace_bytes, l.total);
  PKM_REQUIRE((uintptr_t)weight % 16 == 0 && (uintptr_t)grad_out % 16 == 0 && (uintptr_t)grad_weight % 16 == 0 &&
                  (uintptr_t)workspace % 256 == 0,
              PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd: weight, grad_out, grad_weight must be 16-byte and workspace 256-byte aligned");

  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint32_t* counts = (uint32_t*)(ws + l.counts);
  uint32_t* keys[2] = {(uint32_t*)(ws + l.keys0), (uint32_t*)(ws + l.keys1)};
  uint32_t* vals[2] = {(uint32_t*)(ws + l.vals0), (uint32_t*)(ws + l.vals1)};
  uint32_t* hist = (uint32_t*)(ws + l.hist);
  uint32_t* parts = (uint32_t*)(ws + l.parts);
  float* partials = (float*)(ws + l.partials);
  const int64_t K = num_rows;

  // 1-2. row counts -> offsets[0..K+1]
  hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(K + 2, 256, 4096)), dim3(256), 0, st, counts, 0u, K + 2);
  if (N > 0)
    hipLaunchKernelGGL(count_rows_kernel, dim3(grid_for(N, 256, 16384)), dim3(256), 0, st, indices, N, K, counts);
  device_exclusive_scan(counts, K + 1, parts, st);

  // 3. stable LSD radix sort of (row, position)
  int cur = 0;
  if (N > 0) {
    int bits = 0;
    while (bits < 32 && ((uint64_t)K >> bits) != 0) ++bits;  // keys are in [0, K]
    const int passes = bits == 0 ? 1 : (bits + 7) / 8;
    for (int pass = 0; pass < passes; ++pass) {
      const int shift = pass * 8;
      const int nxt = pass == 0 ? 0 : 1 - cur;
      if (pass == 0) {
        hipLaunchKernelGGL(radix_hist_kernel<true>, dim3((unsigned)l.ntiles), dim3(256), 0, st, indices,
                           (const uint32_t*)nullptr, N, K, shift, hist, l.ntiles);
        device_exclusive_scan(hist, kRadix * l.ntiles, parts, st);
        hipLaunchKernelGGL(radix_scatter_kernel<true>, dim3((unsigned)l.ntiles), dim3(256), 0, st, indices,
                           (const uint32_t*)nullptr, (const uint32_t*)nullptr, N, K, shift, (const uint32_t*)hist,
                           l.ntiles, keys[0], vals[0]);
        cur = 0;
      } else {
        hipLaunchKernelGGL(radix_hist_kernel<false>, dim3((unsigned)l.ntiles), dim3(256), 0, st,
                           (const int64_t*)nullptr, (const uint32_t*)keys[cur], N, K, shift, hist, l.ntiles);
        device_exclusive_scan(hist, kRadix * l.ntiles, parts, st);
        hipLaunchKernelGGL(radix_scatter_kernel<false>, dim3((unsigned)l.ntiles), dim3(256), 0, st,
                           (const int64_t*)nullptr, (const uint32_t*)keys[cur], (const uint32_t*)vals[cur], N, K,
                           shift, (const uint32_t*)hist, l.ntiles, keys[nxt], vals[nxt]);
        cur = nxt;
      }
    }
  }

  // 4-5. heavy-row chunk partials, then every row once
  bool ok;
  if (weight_dtype == PKM_DTYPE_F32)
    ok = dispatch_reduce<float>(c, weight, K, dim, psw, psw_dtype, grad_out, bag_size, counts, keys[cur], vals[cur], N,
                                l, partials, grad_weight, grad_psw, st);
  else if (weight_dtype == PKM_DTYPE_BF16)
    ok = dispatch_reduce<bf16_t>(c, weight, K, dim, psw, psw_dtype, grad_out, bag_size, counts, keys[cur], vals[cur],
                                 N, l, partials, grad_weight, grad_psw, st);
  else
    ok = dispatch_reduce<f16_t>(c, weight, K, dim, psw, psw_dtype, grad_out, bag_size, counts, keys[cur], vals[cur],
                                N, l, partials, grad_weight, grad_psw, st);
  PKM_REQUIRE(ok, PKM_ERR_UNSUPPORTED, "pkm_eb_bwd: no kernel for lpg=%d vpl=%d", c.lpg, c.vpl);
  return pkm_check_launch("pkm_eb_bwd");
}

extern "C" int pkm_count_invalid_indices(const int64_t* indices, int64_t n, int64_t num_rows, int64_t* count_out,
                                         void* stream) {
  PKM_REQUIRE(count_out != nullptr && n >= 0 && num_rows >= 0 && (n == 0 || indices != nullptr),
              PKM_ERR_INVALID_ARGUMENT, "pkm_count_invalid_indices: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(1), 0, st, (unsigned long long*)count_out);
  if (n > 0)
    hipLaunchKernelGGL(count_invalid_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, st, indices, n, num_rows,
                       (unsigned long long*)count_out);
  return pkm_check_launch("pkm_count_invalid_indices");
}

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
//  1. sort:    stable sort of (row, flat position) pairs. Up to 2^22 rows: a
//              radix pass buckets the lookups by the high 8/10/11-bit digit of
//              the row, then a local pass sorts each bucket (2^B consecutive
//              rows) by the low digit, segment by segment, and writes the row
//              offsets and the occurrence metadata on the way. Other row
//              counts: LSD radix passes. Lookups whose index is out of [0, K)
//              are dropped here (their psw-gradient is written as 0). The input
//              is in position order and every pass is stable, so each row's
//              occurrences end up in increasing position order: the float32
//              sums below have a fixed order, independent of the launch (no
//              float atomics anywhere).
//  2. offsets: row r starts at its bucket's start plus the counts of the
//              bucket's lower rows (the local pass), or at the first sorted
//              position whose key is >= r (a binary search per row, after LSD
//              passes).
//  3. heavy:   rows with more than T occurrences are cut into fixed chunks of
//              T sorted occurrences; each chunk writes a float32 partial sum
//              (2 slots per chunk: the row running in from the previous chunk
//              and the row starting inside this one).
//  4. rows:    a wave reduces one row at a time, in position order, with the
//              next row's loads in flight; rows are handed out in chunks of 4
//              through per-XCD ticket counters so that the waves of one XCD
//              work on the same block of 1024 rows at once (PKM's lookups of a
//              bag share sub-key blocks: their gradient rows are re-read from
//              that XCD's L2). Untouched rows get zeros, light rows are reduced
//              while the wave holds W[r] in registers for the psw-gradient dot
//              products, heavy rows add their chunk partials in chunk order,
//              rows longer than the prefetch go to a one-row-per-wave kernel.
// HBM traffic: W is read once per distinct row, gW written once per row, the
// upstream gradient g (B x D, tens of MB) is re-read per occurrence from
// L2 / Infinity Cache.
#include <mutex>
#include <type_traits>

#include "pkm_common.h"

namespace pkm {

constexpr int kHeavyT = 256;  // chunk length and light/heavy row threshold

// ---------------------------------------------------------------------------
// The fast-weight SGD step in the reduction's epilogue (pkm_eb_bwd_sgd): a
// row's float32 gradient sums become, instead of a table-gradient row, the
// scaled gradient and the updated table row of FwPKM's values step
// (fwpkm/fwpkm.py:351-365 with update_fw_param at 266-272, "sgd"):
//   g   = T(acc)                                  (the table gradient's rounding)
//   gs  = T(T(g * scale) / T(max(cnt, 1)))        cnt = the row's lookups (bincount)
//   gc  = clip ? min(max(gs, -1), 1) : gs
//   p'  = T(p - T(lr * T(gc + T(wd * p))))
// every step rounded to T in the reference's order, no contraction. The row
// of p is the table row the reduction reads anyway (for the psw-gradient
// dots), so the step costs no extra table read and no gradient round trip.
// ---------------------------------------------------------------------------
struct SgdArgs {
  void* new_values;   // [K, D], table dtype
  void* scaled_grad;  // [K, D], table dtype
  int32_t* counts;    // [K]: lookups per row, or NULL
  float* row_sumsq;   // [K]: sum over the row of gs^2 (float32), or NULL
  float scale, lr, wd;
  int clip;
};

#pragma clang fp contract(off)
// o_g = gs and o_p = p' of NE elements (acc: float32 sums, p: table
// elements); returns the sum of gs^2 over them.
template <typename TW, int NE>
__device__ __forceinline__ float sgd_step(const float* acc, const float* p, uint32_t cnt, const SgdArgs& S,
                                          float* o_g, float* o_p) {
  const float cs = round_to<TW>(cnt == 0 ? 1.f : (float)cnt);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const float g = round_to<TW>(acc[e]);
    const float gs = round_to<TW>(round_to<TW>(g * S.scale) / cs);
    float gc = gs;
    if (S.clip) gc = gc < -1.f ? -1.f : (gc > 1.f ? 1.f : gc);
    const float wp = round_to<TW>(S.wd * p[e]);
    const float dp = round_to<TW>(S.lr * round_to<TW>(gc + wp));
    o_g[e] = gs;
    o_p[e] = round_to<TW>(p[e] - dp);
    ss = ss + gs * gs;
  }
  return ss;
}
#pragma clang fp contract(on)

// The SGD epilogue of one row held by LPG lanes (the lane's VPL vectors at
// element col0 + v * LPG * EPV): stores gs (unless S.scaled_grad is NULL) and
// p', and from the group's first lane the row's count and sum of gs^2.
template <typename TW, int LPG, int VPL>
__device__ __forceinline__ void sgd_store_row(const float* acc, const float* p, uint32_t cnt, int64_t row, int64_t D,
                                              int64_t col0, int glane, const SgdArgs& S) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  float o_g[NE], o_p[NE];
  float ss = sgd_step<TW, NE>(acc, p, cnt, S, o_g, o_p);
  TW* grow = (TW*)S.scaled_grad + row * D + col0;
  TW* prow = (TW*)S.new_values + row * D + col0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    if (S.scaled_grad != nullptr) st16_nt(grow + v * LPG * EPV, VecTraits<TW>::pack(o_g + v * EPV));
    st16_nt(prow + v * LPG * EPV, VecTraits<TW>::pack(o_p + v * EPV));
  }
  ss = group_sum<LPG>(ss);
  if (glane == 0) {
    if (S.row_sumsq != nullptr) S.row_sumsq[row] = ss;
    if (S.counts != nullptr) S.counts[row] = (int32_t)cnt;
  }
}

// ---------------------------------------------------------------------------
// Utilities
// ---------------------------------------------------------------------------
// The prepare phase's zeroed state in one launch: the out-of-range lookup
// count, the long-row count, the hot-row count and lo flag (2 words) and the
// zero row (n_zrow u32 words), each when not null.
__global__ void prep_fill_kernel(uint32_t* __restrict__ invalid, uint32_t* __restrict__ long_count,
                                 uint32_t* __restrict__ hot_state, uint32_t* __restrict__ zrow, int64_t n_zrow) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    invalid[0] = 0u;
    if (long_count != nullptr) long_count[0] = 0u;
    if (hot_state != nullptr) {
      hot_state[0] = 0u;
      hot_state[1] = 0u;
    }
  }
  if (zrow == nullptr) return;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_zrow; i += (int64_t)gridDim.x * blockDim.x)
    zrow[i] = 0u;
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
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
// Device-wide exclusive prefix sum of uint32 (tiles of 4096 = 256 threads x
// 16): the radix digit offsets.
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

// Exclusive prefix sum of one value per thread across a 256-thread block.
__device__ __forceinline__ uint32_t block_exclusive_sum(uint32_t v, uint32_t* total, uint32_t* lds4) {
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
  block_exclusive_sum(s, &tot, lds4);
  if (threadIdx.x == 0) parts[blockIdx.x] = tot;
}

// Single block: exclusive prefix sum of the per-tile sums, in place.
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
    uint32_t run = carry + block_exclusive_sum(s, &tot, lds4);
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      if (p0 + i < nparts) parts[p0 + i] = run;
      run += v[i];
    }
    carry += tot;
  }
}

// data[i] <- tile prefix + exclusive sum inside the tile; data[n] <- total.
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
  uint32_t run = parts[blockIdx.x] + block_exclusive_sum(s, &tot, lds4);
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    if (p0 + i < n) data[p0 + i] = run;
    run += v[i];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) data[n] = parts[blockIdx.x] + tot;
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort pass with BITS-bit digits over tiles of kRadixSubs
// sub-tiles of 4096 items (4 waves x 16 rounds x 64 lanes), taken in order.
// Item order inside a sub-tile: wave-major, then round, then lane, so ranks
// stay stable. The first pass reads the int64 indices (dropping out-of-range
// ones); later passes read nvalid items. (Tiles of 4 sub-tiles shrink the
// per-tile digit histogram 4x but leave a quarter of the blocks: measured
// slower at 4 M lookups.)
// ---------------------------------------------------------------------------
constexpr int kRadixItems = 16;
constexpr int kRadixSub = 256 * kRadixItems;
constexpr int kRadixSubs = 1;
constexpr int kRadixTile = kRadixSub * kRadixSubs;

template <bool FIRST>
__device__ __forceinline__ bool radix_item(int64_t p, int64_t N, uint32_t nv, const int64_t* __restrict__ idx,
                                           const uint32_t* __restrict__ keys, int64_t K, uint32_t* k) {
  if (FIRST) {
    if (p >= N) return false;
    const int64_t r = idx[p];
    *k = (uint32_t)r;
    return r >= 0 && r < K;
  }
  if (p >= (int64_t)nv) return false;
  *k = keys[p];
  return true;
}

// FIRST pass: lookups whose index is outside [0, K) are dropped from the sort
// and their positions listed (invalid[0] = count, then the positions; one
// atomic per wave that holds any), so the reduction can zero their
// psw-gradients.
template <bool FIRST, int BITS>
__global__ __launch_bounds__(256) void radix_hist_kernel(const int64_t* __restrict__ idx,
                                                         const uint32_t* __restrict__ keys, int64_t N,
                                                         const uint32_t* __restrict__ nvalid, int64_t K, int shift,
                                                         uint32_t* __restrict__ hist, int64_t ntiles,
                                                         uint32_t* __restrict__ invalid) {
  constexpr int R = 1 << BITS;
  __shared__ uint32_t h[R];
  for (int d = threadIdx.x; d < R; d += 256) h[d] = 0;
  __syncthreads();
  const uint32_t nv = FIRST ? 0u : *nvalid;
  const int64_t base = (int64_t)blockIdx.x * kRadixTile;
#pragma unroll 4
  for (int i = 0; i < kRadixItems * kRadixSubs; ++i) {
    const int64_t p = base + (int64_t)i * 256 + threadIdx.x;
    uint32_t k;
    const bool valid = radix_item<FIRST>(p, N, nv, idx, keys, K, &k);
    if (valid) atomicAdd(&h[(k >> shift) & (R - 1)], 1u);
    if (FIRST) {
      const bool bad = !valid && p < N;
      const uint64_t m = __ballot(bad);
      if (m != 0ull) {
        const int lane = threadIdx.x & 63;
        uint32_t at = 0;
        if (lane == 0) at = atomicAdd(invalid, (uint32_t)__popcll(m));
        at = (uint32_t)__builtin_amdgcn_readlane((int)at, 0);
        if (bad) invalid[1 + at + (uint32_t)__popcll(lane == 0 ? 0ull : (m & (~0ull >> (64 - lane))))] = (uint32_t)p;
      }
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < R; d += 256) hist[(int64_t)d * ntiles + blockIdx.x] = h[d];
}

// Segments of the local pass (LOCAL scatter): per segment its first item and
// one past its last, then the segment count at [2 * max_segs].
struct SegTab {
  const uint32_t* tab;
  int64_t max_segs;
};

// Stable scatter of one tile by digit, sub-tile by sub-tile. Each sub-tile is
// first ordered by digit in LDS (per digit in item order), then written out in
// that order, so each digit's run of the sub-tile goes to consecutive
// addresses, right after the previous sub-tile's run of that digit: keys first,
// then values, through one LDS buffer.
// LOCAL: the block is one segment of the local pass (items [begin, end) of one
// high-digit bucket, in order), its per-digit destinations given in ofs
// [segment][digit]; the occurrence metadata {position / L, psw as float32
// bits} of each item is written beside it when meta is not null.
template <bool FIRST, int BITS, bool LOCAL = false>
__global__ __launch_bounds__(256) void radix_scatter_kernel(const int64_t* __restrict__ idx,
                                                            const uint32_t* __restrict__ keys_in,
                                                            const uint32_t* __restrict__ vals_in, int64_t N,
                                                            const uint32_t* __restrict__ nvalid, int64_t K,
                                                            int shift, const uint32_t* __restrict__ ofs,
                                                            int64_t ntiles, uint32_t* __restrict__ keys_out,
                                                            uint32_t* __restrict__ vals_out, SegTab seg = SegTab{},
                                                            uint2* __restrict__ meta = nullptr,
                                                            const void* __restrict__ psw = nullptr, int pdt = 0,
                                                            uint32_t L32 = 1) {
  static_assert(!(FIRST && LOCAL), "the local pass reads the bucketed keys");
  constexpr int R = 1 << BITS;
  constexpr int DPT = R / 256;  // digits per thread in the digit scan
  static_assert(R % 256 == 0, "digit count per thread");
  __shared__ uint32_t wcnt[4][R];        // per-wave digit counts, then their starts inside the sub-tile
  __shared__ uint32_t gofs[R];           // per digit: global start - start inside the sub-tile
  __shared__ uint32_t stage[kRadixSub];  // the sub-tile in digit order (keys, then values)
  __shared__ uint32_t wsum[4];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int64_t first = (int64_t)blockIdx.x * kRadixTile;  // the block's first item
  uint32_t lim;                                      // items below lim (non-first passes) are valid
  int nsub = kRadixSubs;
  // per owned digit (thread t: digits DPT t .. DPT t + DPT - 1): the global
  // position of its next item in this tile
  uint32_t running[DPT];
  if constexpr (LOCAL) {
    const uint32_t nseg = seg.tab[2 * seg.max_segs];
    if (blockIdx.x >= nseg) return;
    const uint32_t b = seg.tab[2 * blockIdx.x], e = seg.tab[2 * blockIdx.x + 1];
    first = b;
    lim = e;
    nsub = (int)((e - b + kRadixSub - 1) / kRadixSub);
#pragma unroll
    for (int j = 0; j < DPT; ++j) running[j] = ofs[(int64_t)blockIdx.x * R + threadIdx.x * DPT + j];
  } else {
    lim = FIRST ? 0u : *nvalid;
#pragma unroll
    for (int j = 0; j < DPT; ++j) running[j] = ofs[(int64_t)(threadIdx.x * DPT + j) * ntiles + blockIdx.x];
  }
  const uint32_t nv = lim;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

#pragma unroll 1
  for (int sub = 0; sub < nsub; ++sub) {
    for (int d = threadIdx.x; d < R; d += 256) {
#pragma unroll
      for (int i = 0; i < 4; ++i) wcnt[i][d] = 0;
    }
    __syncthreads();
    const int64_t base = first + (int64_t)sub * kRadixSub + (int64_t)w * (kRadixItems * 64);
    uint32_t k[kRadixItems], v[kRadixItems], pre[kRadixItems];
    uint32_t validmask = 0;
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i) {
      const int64_t p = base + (int64_t)i * 64 + lane;
      k[i] = 0;
      const bool valid = radix_item<FIRST>(p, N, nv, idx, keys_in, K, &k[i]);
      v[i] = valid ? (FIRST ? (uint32_t)p : vals_in[p]) : 0u;
      validmask |= valid ? (1u << i) : 0u;
      const uint32_t d = (k[i] >> shift) & (R - 1);
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int bit = 0; bit < BITS; ++bit) {
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
    // digit starts inside the sub-tile: exclusive scan over the digits (thread
    // t owns digits DPT t .. DPT t + DPT - 1) of the sub-tile's digit counts
    uint32_t tot[DPT], mine = 0;
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = threadIdx.x * DPT + j;
      tot[j] = wcnt[0][d] + wcnt[1][d] + wcnt[2][d] + wcnt[3][d];
      mine += tot[j];
    }
    uint32_t incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = (uint32_t)__shfl_up((int)incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint32_t run = incl - mine;
    for (int i = 0; i < w; ++i) run += wsum[i];
    const uint32_t nloc = wsum[0] + wsum[1] + wsum[2] + wsum[3];  // valid items of the sub-tile
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = threadIdx.x * DPT + j;
      gofs[d] = running[j] - run;
      running[j] += tot[j];
      uint32_t r2 = run;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t t = wcnt[i][d];
        wcnt[i][d] = r2;
        r2 += t;
      }
      run += tot[j];
    }
    __syncthreads();
    uint32_t lp[kRadixItems];  // position of item i inside the sub-tile's digit order
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i) {
      lp[i] = wcnt[w][(k[i] >> shift) & (R - 1)] + pre[i];
      if (validmask & (1u << i)) stage[lp[i]] = k[i];
    }
    __syncthreads();
    // keys out in digit order (consecutive positions of a digit: consecutive
    // addresses); the destinations are kept for the values
    uint32_t dst[kRadixItems];
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i) {
      const uint32_t q = (uint32_t)(i * 256 + threadIdx.x);
      dst[i] = 0;
      if (q < nloc) {
        const uint32_t key = stage[q];
        dst[i] = gofs[(key >> shift) & (R - 1)] + q;
        keys_out[dst[i]] = key;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i)
      if (validmask & (1u << i)) stage[lp[i]] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRadixItems; ++i) {
      const uint32_t q = (uint32_t)(i * 256 + threadIdx.x);
      if (q < nloc) {
        const uint32_t val = stage[q];
        vals_out[dst[i]] = val;
        if (LOCAL && meta != nullptr)
          meta[dst[i]] = make_uint2(val / L32, __float_as_uint(psw ? load_scalar(psw, pdt, val) : 1.f));
      }
    }
    __syncthreads();  // stage and wcnt are reused by the next sub-tile
  }
}

// ---------------------------------------------------------------------------
// Local pass of the two-level sort. The first pass buckets the lookups stably
// by the high digit of the row (bits [B, 2 B)); each bucket holds the rows
// b 2^B .. b 2^B + 2^B - 1 and its lookups in position order, so a stable
// sort of each bucket by the low digit completes the sort by (row, position),
// the order the single-digit passes give. Buckets are cut into segments of
// at most kSegItems lookups (one workgroup each): per-segment digit counts,
// then per bucket the digits' starts (the rows' offsets) and each segment's
// share, then the segments' stable scatters, which also write the occurrence
// metadata. A bucket's writes stay inside its own range of the outputs.
// ---------------------------------------------------------------------------
constexpr int kSegItems = kRadixSub;  // one sub-tile per segment: a hot bucket spreads over many workgroups

// One block: the segment table from the first pass's scanned digit offsets
// (bucket b starts at ofs[b * ntiles], the next bucket's start or the valid
// count ends it), and per bucket {first segment, one past its last, start};
// also offs[K] <- the valid count and, with meta, the metadata entries past it
// (the padding and the dropped lookups' share) <- 0.
__global__ __launch_bounds__(256) void seg_plan_kernel(const uint32_t* __restrict__ ofs, int64_t ntiles,
                                                       int nbuckets, int R, const uint32_t* __restrict__ nvalid,
                                                       uint32_t* __restrict__ tab, int64_t max_segs,
                                                       uint32_t* __restrict__ bseg, int64_t K,
                                                       uint32_t* __restrict__ offs, uint2* __restrict__ meta,
                                                       int64_t n_meta) {
  __shared__ uint32_t lds4[4];
  const uint32_t nv = *nvalid;
  if (threadIdx.x == 0) offs[K] = nv;
  if (meta != nullptr)
    for (int64_t i = (int64_t)nv + threadIdx.x; i < n_meta; i += 256) meta[i] = make_uint2(0u, 0u);
  uint32_t carry = 0;
  for (int b0 = 0; b0 < nbuckets; b0 += 256) {
    const int b = b0 + (int)threadIdx.x;
    uint32_t beg = 0, end = 0, ns = 0;
    if (b < nbuckets) {
      beg = ofs[(int64_t)b * ntiles];
      end = b + 1 < R ? ofs[(int64_t)(b + 1) * ntiles] : nv;
      if (b + 1 == nbuckets) end = nv;  // digits past the last bucket hold no lookups
      ns = (end - beg + kSegItems - 1) / kSegItems;
    }
    uint32_t tot;
    const uint32_t s0 = carry + block_exclusive_sum(ns, &tot, lds4);
    if (b < nbuckets) {
      bseg[3 * b] = s0;
      bseg[3 * b + 1] = s0 + ns;
      bseg[3 * b + 2] = beg;
      for (uint32_t j = 0; j < ns; ++j) {
        const uint32_t sb = beg + j * (uint32_t)kSegItems;
        tab[2 * (s0 + j)] = sb;
        tab[2 * (s0 + j) + 1] = end - sb < (uint32_t)kSegItems ? end : sb + (uint32_t)kSegItems;
      }
    }
    carry += tot;
  }
  if (threadIdx.x == 0) tab[2 * max_segs] = carry;
}

// Per segment: counts of the low digit (keys & (2^BITS - 1)).
template <int BITS>
__global__ __launch_bounds__(256) void seg_hist_kernel(const uint32_t* __restrict__ keys, SegTab seg,
                                                       uint32_t* __restrict__ hist) {
  constexpr int R = 1 << BITS;
  __shared__ uint32_t h[R];
  if (blockIdx.x >= seg.tab[2 * seg.max_segs]) return;
  for (int d = threadIdx.x; d < R; d += 256) h[d] = 0;
  __syncthreads();
  const uint32_t b = seg.tab[2 * blockIdx.x], e = seg.tab[2 * blockIdx.x + 1];
  for (uint32_t i = b + threadIdx.x; i < e; i += 256) atomicAdd(&h[keys[i] & (R - 1)], 1u);
  __syncthreads();
  for (int d = threadIdx.x; d < R; d += 256) hist[(int64_t)blockIdx.x * R + d] = h[d];
}

// Append the rows r = base_row + DPT t + j (j < DPT, r < K) whose flag is set
// to list (count at *count): one atomic per block for the block's range; the
// list's order does not matter to the kernels that read it.
template <int DPT>
__device__ __forceinline__ void append_rows(const bool (&flag)[DPT], int64_t base_row, uint32_t* __restrict__ list,
                                            uint32_t* __restrict__ count, uint32_t* lds4, uint32_t* base) {
  uint32_t nl = 0;
#pragma unroll
  for (int j = 0; j < DPT; ++j) nl += flag[j] ? 1u : 0u;
  uint32_t nall;
  uint32_t at = block_exclusive_sum(nl, &nall, lds4);
  if (nall == 0) return;
  if (threadIdx.x == 0) *base = atomicAdd(count, nall);
  __syncthreads();
  at += *base;
#pragma unroll
  for (int j = 0; j < DPT; ++j)
    if (flag[j]) list[at++] = (uint32_t)(base_row + threadIdx.x * DPT + j);
  __syncthreads();  // *base is reused
}

// Per bucket: the digits' starts (row r = b 2^BITS + d starts at offs[r]) and
// each segment's per-digit destination, in place of its counts. With
// long_rows: the bucket's rows of more than T and at most kHeavyT lookups are
// appended to the long-row list; with hot_bcnt: the number of its rows of at
// least H lookups (hot rows, listed in row order by hot_order_kernel).
template <int BITS>
__global__ __launch_bounds__(256) void seg_base_kernel(const uint32_t* __restrict__ bseg, int64_t K,
                                                       uint32_t* __restrict__ hist, uint32_t* __restrict__ offs,
                                                       uint32_t T, uint32_t* __restrict__ long_rows,
                                                       uint32_t* __restrict__ long_count, uint32_t H,
                                                       uint32_t* __restrict__ hot_bcnt) {
  constexpr int R = 1 << BITS;
  constexpr int DPT = R / 256;
  __shared__ uint32_t lds4[4];
  const int b = blockIdx.x;
  const uint32_t s0 = bseg[3 * b], s1 = bseg[3 * b + 1], start = bseg[3 * b + 2];
  // the thread's DPT consecutive digits of a segment: one or two 16-byte vectors (one word for DPT = 1); each
  // pass walks the bucket's segments once
  static_assert(DPT == 1 || DPT % 4 == 0, "digits per thread: 1 or a multiple of 4");
  auto seg_row = [&](uint32_t s) { return hist + (int64_t)s * R + threadIdx.x * DPT; };
  auto load_row = [&](uint32_t s, uint32_t (&v)[DPT]) {
    if constexpr (DPT == 1) {
      v[0] = *seg_row(s);
    } else {
#pragma unroll
      for (int q = 0; q < DPT / 4; ++q) {
        const uint4 x = *(const uint4*)(seg_row(s) + 4 * q);
        v[4 * q] = x.x;
        v[4 * q + 1] = x.y;
        v[4 * q + 2] = x.z;
        v[4 * q + 3] = x.w;
      }
    }
  };
  auto store_row = [&](uint32_t s, const uint32_t (&v)[DPT]) {
    if constexpr (DPT == 1) {
      *seg_row(s) = v[0];
    } else {
#pragma unroll
      for (int q = 0; q < DPT / 4; ++q)
        *(uint4*)(seg_row(s) + 4 * q) = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
  };
  uint32_t tot[DPT], mine = 0;
#pragma unroll
  for (int j = 0; j < DPT; ++j) tot[j] = 0;
#pragma unroll 4
  for (uint32_t s = s0; s < s1; ++s) {
    uint32_t v[DPT];
    load_row(s, v);
#pragma unroll
    for (int j = 0; j < DPT; ++j) tot[j] += v[j];
  }
#pragma unroll
  for (int j = 0; j < DPT; ++j) mine += tot[j];
  uint32_t all;
  uint32_t run = block_exclusive_sum(mine, &all, lds4);
  uint32_t at[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = threadIdx.x * DPT + j;
    const int64_t r = ((int64_t)b << BITS) + d;
    if (r < K) offs[r] = start + run;
    at[j] = start + run;
    run += tot[j];
  }
#pragma unroll 4
  for (uint32_t s = s0; s < s1; ++s) {
    uint32_t v[DPT];
    load_row(s, v);
    store_row(s, at);
#pragma unroll
    for (int j = 0; j < DPT; ++j) at[j] += v[j];
  }
  __shared__ uint32_t base;
  const int64_t row0 = (int64_t)b << BITS;
  if (long_rows != nullptr) {
    bool fl[DPT];
#pragma unroll
    for (int j = 0; j < DPT; ++j)
      fl[j] = row0 + threadIdx.x * DPT + j < K && tot[j] > T && tot[j] <= (uint32_t)kHeavyT;
    append_rows<DPT>(fl, row0, long_rows, long_count, lds4, &base);
  }
  if (hot_bcnt != nullptr) {
    uint32_t nh = 0;
#pragma unroll
    for (int j = 0; j < DPT; ++j) nh += (row0 + threadIdx.x * DPT + j < K && tot[j] >= H) ? 1u : 0u;
    uint32_t nall;
    block_exclusive_sum(nh, &nall, lds4);
    if (threadIdx.x == 0) hot_bcnt[b] = nall;
  }
}

// The hot rows (at least H lookups) in row order: bucket b (rows
// [b 2^BITS, (b + 1) 2^BITS)) writes its rows after the hot rows of the
// buckets before it (hot_bcnt: per-bucket counts); the last bucket writes the
// count at hot[hr_max]. Rows in order keep a tile's hot rows, and their
// merged entries, close together in memory.
template <int BITS>
__global__ __launch_bounds__(256) void hot_order_kernel(const uint32_t* __restrict__ hot_bcnt, int64_t nbuckets,
                                                        const uint32_t* __restrict__ offs, int64_t K, uint32_t H,
                                                        uint32_t* __restrict__ hot, int64_t hr_max) {
  constexpr int DPT = (1 << BITS) / 256;
  __shared__ uint32_t lds4[4];
  const int64_t b = blockIdx.x;
  uint32_t pre = 0;
  for (int64_t x = threadIdx.x; x < b; x += 256) pre += hot_bcnt[x];
  uint32_t prefix;
  block_exclusive_sum(pre, &prefix, lds4);
  const int64_t row0 = (b << BITS) + (int64_t)threadIdx.x * DPT;
  bool fl[DPT];
  uint32_t nh = 0;
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int64_t r = row0 + j;
    fl[j] = r < K && offs[r + 1] - offs[r] >= H;
    nh += fl[j] ? 1u : 0u;
  }
  uint32_t total;
  uint32_t at = prefix + block_exclusive_sum(nh, &total, lds4);
#pragma unroll
  for (int j = 0; j < DPT; ++j)
    if (fl[j]) hot[at++] = (uint32_t)(row0 + j);
  if (b == nbuckets - 1 && threadIdx.x == 0) hot[hr_max] = prefix + total;
}

// offs[r] <- the first sorted position whose key is >= r (a binary search of
// the nvalid sorted keys per row; the searches of neighbouring rows follow the
// same path, so a wave's loads mostly share cache lines); offs[K] <- nvalid.
__global__ void row_offsets_kernel(const uint32_t* __restrict__ skeys, const uint32_t* __restrict__ nvalid, int64_t K,
                                   uint32_t* __restrict__ offs) {
  const uint32_t nv = *nvalid;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r <= K; r += (int64_t)gridDim.x * blockDim.x) {
    uint32_t lo = 0, hi = nv;
    if (r == K) {
      lo = nv;
    } else {
      while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (skeys[mid] < (uint32_t)r)
          lo = mid + 1;
        else
          hi = mid;
      }
    }
    offs[r] = lo;
  }
}

// ---------------------------------------------------------------------------
// Segmented reduction over sorted occurrences (generic lane groups).
// ---------------------------------------------------------------------------
template <int VPL>
struct BwdUnroll {
  static constexpr int U = VPL >= 8 ? 2 : (VPL >= 4 ? 4 : 8);
};

// acc += sum over sorted occurrences [i_beg, i_end) (in order) of psw[p] * g[p / L];
// with want_dot, gpsw[p] = <wv, g[p / L]> for each of them.
template <typename TW, typename TG, int LPG, int VPL>
__device__ __forceinline__ void reduce_occurrences(uint32_t i_beg, uint32_t i_end, const uint32_t* __restrict__ svals,
                                                   const void* __restrict__ psw, int pdt,
                                                   const TG* __restrict__ g, int64_t D, uint32_t L32,
                                                   int64_t col0, int glane, const float* wv, bool want_dot,
                                                   void* __restrict__ gpsw, float* acc,
                                                   float* __restrict__ dsorted = nullptr) {
  using GT = GradTraits<TW, TG>;
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int NV = GT::NV;
  constexpr int U = BwdUnroll<VPL * NV>::U;
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
      uint4 gvec[U][VPL * NV];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        w[u] = 0.f;
        if (jj + u < n) {
          const uint32_t b = (uint32_t)bcast_i32<LPG>((int)my_b, jj + u);
          w[u] = bcast_f32<LPG>(my_w, jj + u);
          const TG* grow = g + (int64_t)b * D + col0;
#pragma unroll
          for (int v = 0; v < VPL; ++v)
#pragma unroll
            for (int h = 0; h < NV; ++h) gvec[u][v * NV + h] = ld16(grow + v * VSTRIDE + h * (EPV / NV));
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (jj + u < n) {
          float f[NE];
#pragma unroll
          for (int v = 0; v < VPL; ++v) GT::unpack(&gvec[u][v * NV], f + v * EPV);
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
    if (want_dot && glane < n) {
      if (dsorted != nullptr)
        dsorted[i0 + glane] = my_dot;  // sorted order, scattered by position later
      else
        store_scalar(gpsw, pdt, my_p, my_dot);
    }
  }
}

template <typename TW, int LPG, int VPL>
__device__ __forceinline__ void load_row_f32(const TW* __restrict__ row, int64_t col0, float* f) {
  constexpr int EPV = VecTraits<TW>::EPV;
#pragma unroll
  for (int v = 0; v < VPL; ++v) VecTraits<TW>::unpack(ld16(row + col0 + v * LPG * EPV), f + v * EPV);
}

// acc += partial sums of a heavy row [beg, end) in chunk order.
template <int LPG, int VPL, int EPV>
__device__ __forceinline__ void add_heavy_partials(uint32_t beg, uint32_t end, const float* __restrict__ partials,
                                                   int64_t D, int64_t col0, float* acc) {
  constexpr int VSTRIDE = LPG * EPV;
  const uint32_t c_first = beg / kHeavyT, c_last = (end - 1) / kHeavyT;
#pragma unroll 4
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
}

// Heavy rows: chunk c = sorted occurrences [c*T, (c+1)*T). A row with more
// than T occurrences always contains the chunk's first or last occurrence.
template <typename TW, typename TG, int LPG, int VPL>
__global__ __launch_bounds__(256) void eb_bwd_heavy_kernel(const TW* __restrict__ W, int64_t K, int64_t D,
                                                           const void* __restrict__ psw, int pdt,
                                                           const TG* __restrict__ g, uint32_t L32,
                                                           const uint32_t* __restrict__ offs,
                                                           const uint32_t* __restrict__ skeys,
                                                           const uint32_t* __restrict__ svals,
                                                           const uint32_t* __restrict__ nvalid, int64_t nchunks,
                                                           float* __restrict__ partials, void* __restrict__ gpsw,
                                                           float* __restrict__ dsorted, uint32_t hot_min) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int GPW = 64 / LPG;
  const int lane = threadIdx.x & 63;
  const int glane = lane & (LPG - 1);
  const int64_t c = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * GPW + (lane / LPG);
  if (c >= nchunks) return;
  const uint32_t nv = *nvalid;
  const uint32_t i_beg = (uint32_t)(c * kHeavyT);
  if (i_beg >= nv) return;
  const uint32_t i_end = (uint32_t)((int64_t)i_beg + kHeavyT < (int64_t)nv ? i_beg + kHeavyT : nv);
  const int64_t col0 = (int64_t)glane * EPV;
  const bool want_dot = psw != nullptr && (gpsw != nullptr || dsorted != nullptr);
  const uint32_t cand[2] = {skeys[i_beg], skeys[i_end - 1]};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t r = cand[t];
    if (t == 1 && r == cand[0]) break;
    const uint32_t rb = offs[r], re = offs[r + 1];
    if (re - rb <= (uint32_t)kHeavyT || re - rb >= hot_min) continue;  // light, or reduced on the matrix cores
    const uint32_t s_beg = rb > i_beg ? rb : i_beg;
    const uint32_t s_end = re < i_end ? re : i_end;
    const int slot = rb > i_beg ? 1 : 0;
    float wv[NE];
    if (want_dot) load_row_f32<TW, LPG, VPL>(W + (int64_t)r * D, col0, wv);
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    reduce_occurrences<TW, TG, LPG, VPL>(s_beg, s_end, svals, psw, pdt, g, D, L32, col0, glane, wv, want_dot, gpsw,
                                         acc, dsorted);
    float* prow = partials + (2 * c + slot) * D + col0;
#pragma unroll
    for (int v = 0; v < VPL; ++v)
#pragma unroll
      for (int h = 0; h < EPV; h += 4) st16(prow + v * LPG * EPV + h, VecTraits<float>::pack(acc + v * EPV + h));
  }
}

// Generic rows kernel (lane groups smaller than a wave, small rows).
template <typename TW, typename TG, int LPG, int VPL, bool SGD>
__global__ __launch_bounds__(256) void eb_bwd_rows_kernel(const TW* __restrict__ W, int64_t K, int64_t D,
                                                          const void* __restrict__ psw, int pdt,
                                                          const TG* __restrict__ g, uint32_t L32,
                                                          const uint32_t* __restrict__ offs,
                                                          const uint32_t* __restrict__ svals,
                                                          const float* __restrict__ partials, int rows_per_group,
                                                          TW* __restrict__ gW, void* __restrict__ gpsw,
                                                          SgdArgs S) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int GPW = 64 / LPG;
  constexpr int VSTRIDE = LPG * EPV;
  const int lane = threadIdx.x & 63;
  const int glane = lane & (LPG - 1);
  const int64_t grp = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * GPW + (lane / LPG);
  const int64_t r0 = grp * rows_per_group;
  if (r0 >= K) return;
  const int64_t r1 = (r0 + rows_per_group < K) ? r0 + rows_per_group : K;
  const int64_t col0 = (int64_t)glane * EPV;
  const bool want_dot = gpsw != nullptr;

  for (int64_t r = r0; r < r1; ++r) {
    const uint32_t beg = offs[r], end = offs[r + 1];
    const uint32_t cnt = end - beg;
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    if (cnt > (uint32_t)kHeavyT) {
      add_heavy_partials<LPG, VPL, EPV>(beg, end, partials, D, col0, acc);
    } else if (cnt > 0) {
      float wv[NE];
      if (want_dot) load_row_f32<TW, LPG, VPL>(W + r * D, col0, wv);
      reduce_occurrences<TW, TG, LPG, VPL>(beg, end, svals, psw, pdt, g, D, L32, col0, glane, wv, want_dot, gpsw, acc);
    }
    if constexpr (SGD) {
      float p[NE];
      load_row_f32<TW, LPG, VPL>(W + r * D, col0, p);
      sgd_store_row<TW, LPG, VPL>(acc, p, cnt, r, D, col0, glane, S);
    } else {
      TW* orow = gW + r * D + col0;
#pragma unroll
      for (int v = 0; v < VPL; ++v) st16_nt(orow + v * VSTRIDE, VecTraits<TW>::pack(acc + v * EPV));
    }
  }
}

// Row kernel (a wave per row; rows of 64*VPL 16-byte vectors), software-pipelined.
//
// Row i+1's W row and its first U gradient rows are in flight while row i is
// reduced and stored. gfx9 counts loads and stores in one in-order vmcnt, so
// the loads must be issued before the current row's stores, and every row
// issues the same number of vector loads (unused slots read a zero row, tail
// rows past K write a dummy row) so the compiler's waits stay partial. The
// psw-gradient dots of a row leave in one store into sorted order and are
// scattered by position afterwards.
constexpr int kMetaPad = 16;  // metadata entries past the last lookup (a row's U-slot reads stay in bounds)

// Sums of 8 per-lane partials over the 64 lanes of a wave, one butterfly for
// all 8 (18 lane operations instead of 8 full-wave reductions): lane l gets the
// total of slot 4 b5 + 2 b4 + b3 (bits 5, 4, 3 of l). Exchanges: the 32-lane
// halves (v_permlane32_swap), lane ^ 16, lane ^ 8 (DPP row_ror:8), then the 8
// lanes of a group. Fixed order, so the sums are deterministic.
__device__ __forceinline__ float reduce8_slots(const float (&d)[8], int lane) {
  float e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // lanes 0-31: d[j] of lanes l and l + 32; lanes 32-63: d[j + 4] of lanes l - 32 and l
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(d[j]), __float_as_uint(d[j + 4]), false, false);
    e[j] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
  const bool b4 = (lane & 16) != 0;
  float f[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) f[j] = (b4 ? e[j + 2] : e[j]) + __shfl_xor(b4 ? e[j] : e[j + 2], 16);
  const bool b3 = (lane & 8) != 0;
  const float send = b3 ? f[0] : f[1];
  const float t = (b3 ? f[1] : f[0]) +
                  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x128, 0xF, 0xF, false));
  return group_sum<8>(t);
}

template <int VPL, int U, int NV>
struct RowData {
  uint4 wraw[VPL];
  uint4 gvec[U][VPL * NV];  // NV 16-byte loads per table vector (GradTraits)
};
template <int U>
struct RowMeta {
  uint32_t beg, end, nh;  // nh: occurrences served by the prefetch (0 for empty / heavy rows)
  uint32_t b[U];
  float w[U];
};

// acc += sum_{u < nh} w[u] * gvec[u] over a row's U prefetch slots; the
// returned value holds, on lane dot_slot_of<U>(lane), the psw-gradient dot
// <wraw, gvec[slot]> (slots u >= nh, wave-uniform, are skipped).
template <int U>
__device__ __forceinline__ int dot_slot_of(int lane) {
  return U == 8 ? 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1) : lane;
}
// whether this lane stores its slot's dot (one lane per slot)
template <int U>
__device__ __forceinline__ bool dot_store_of(int lane) {
  return U == 8 ? (lane & 7) == 0 : true;
}
template <typename TW, typename TG, int VPL, int U>
__device__ __forceinline__ float accumulate_slots(const RowData<VPL, U, GradTraits<TW, TG>::NV>& R, const float* w,
                                                  uint32_t nh, float* acc, bool want_dot, int lane) {
  using GT = GradTraits<TW, TG>;
  constexpr int NV = GT::NV;
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  float d[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    d[u] = 0.f;
    if ((uint32_t)u < nh) {
      float f[NE];
#pragma unroll
      for (int v = 0; v < VPL; ++v) GT::unpack(&R.gvec[u][v * NV], f + v * EPV);
#pragma unroll
      for (int e = 0; e < NE; ++e) acc[e] = __builtin_fmaf(f[e], w[u], acc[e]);
      if (want_dot) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) d[u] = GT::dot(R.wraw[v], &R.gvec[u][v * NV], d[u]);
      }
    }
  }
  float mydot = 0.f;
  if (want_dot) {
    if constexpr (U == 8) {
      mydot = reduce8_slots(d, lane);  // the total of slot dot_slot_of<8>(lane) (slots >= nh hold 0)
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if ((uint32_t)u < nh) {
          const float t = group_sum<64>(d[u]);
          mydot = lane == u ? t : mydot;
        }
      }
    }
  }
  return mydot;
}

// Accumulating reduction (pkm_eb_bwd_accumulate): the row's gradient is added
// to the one already in gW, as autograd adds two gradients of one tensor:
// acc = pending + T(sum), rounded to T once more by the store.
template <typename TW, int VPL>
__device__ __forceinline__ void unpack_add_pending(const uint4* P, float* acc) {
  constexpr int EPV = VecTraits<TW>::EPV;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    float pv[EPV];
    VecTraits<TW>::unpack(P[v], pv);
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[v * EPV + e] = pv[e] + round_to<TW>(acc[v * EPV + e]);
  }
}
template <typename TW, int VPL>
__device__ __forceinline__ void add_pending_row(const char* orow, uint32_t lane_byte, float* acc) {
  uint4 P[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) P[v] = ld16(orow + lane_byte + v * 1024u);
  unpack_add_pending<TW, VPL>(P, acc);
}

// The long light rows list_long_rows_kernel listed: each wave takes one row at a time
// (grid-stride over the list, whose length every wave reads, so every wave
// ends) and reduces it U occurrences at a time, in order, the next chunk's
// metadata and gradient rows in flight while the current chunk is reduced.
// One wave per row keeps each row's sums in position order.
template <typename TW, typename TG, int VPL, int U, bool SGD, bool ACC>
__global__ __launch_bounds__(256) void eb_bwd_long_rows_kernel(
    const TW* __restrict__ W, int64_t D, int want_dot, const TG* __restrict__ g, const uint32_t* __restrict__ offs,
    const uint2* __restrict__ meta, const TW* __restrict__ zrow, TW* __restrict__ gW, float* __restrict__ dsorted,
    uint32_t dummy_slot, const uint32_t* __restrict__ long_rows, const uint32_t* __restrict__ long_count,
    SgdArgs S) {
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  constexpr int NV = GradTraits<TW, TG>::NV;
  const int lane = threadIdx.x & 63;
  const uint32_t lane_byte = (uint32_t)lane * 16u;
  const uint32_t glane_byte = lane_byte * NV;  // the lane's gradient elements (NV 16-byte pieces each)
  const uint64_t rowbytes = (uint64_t)D * sizeof(TW);
  const uint64_t growbytes = (uint64_t)D * sizeof(TG);
  const char* Wb = (const char*)W;
  const char* gb = (const char*)g;
  const char* zb = (const char*)zrow;
  const int dot_slot = dot_slot_of<U>(lane);
  const bool dot_store = dot_store_of<U>(lane);
  const uint32_t n = *long_count;
  const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
  auto fetch = [&](uint32_t s, uint32_t end, RowData<VPL, U, NV>& R, float* w) {
    const uint32_t nh = (end - s) < (uint32_t)U ? (end - s) : (uint32_t)U;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint2 m = meta[(uint32_t)u < nh ? s + (uint32_t)u : s];  // uniform: scalar loads
      w[u] = (uint32_t)u < nh ? __uint_as_float(m.y) : 0.f;
      const char* grow = (uint32_t)u < nh ? gb + (uint64_t)m.x * growbytes : zb;
#pragma unroll
      for (int v = 0; v < VPL * NV; ++v) R.gvec[u][v] = ld16(grow + glane_byte + (v / NV) * 1024u * NV + (v % NV) * 16u);
    }
    return nh;
  };
  for (uint32_t t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); t < n; t += nwaves) {
    const uint32_t r = (uint32_t)__builtin_amdgcn_readfirstlane((int)long_rows[t]);
    const uint32_t beg = offs[r], end = offs[r + 1];
    const char* wrow = (want_dot || SGD) ? Wb + (uint64_t)r * rowbytes : zb;
    RowData<VPL, U, NV> DA, DB;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      DA.wraw[v] = ld16(wrow + lane_byte + v * 1024u);
      DB.wraw[v] = ld16(wrow + lane_byte + v * 1024u);
    }
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    float wA[U], wB[U];
    uint32_t nA = fetch(beg, end, DA, wA), nB = 0;
    for (uint32_t s = beg;;) {
      const uint32_t s2 = s + U;
      if (s2 < end) nB = fetch(s2, end, DB, wB);
      float d = accumulate_slots<TW, TG, VPL, U>(DA, wA, nA, acc, want_dot, lane);
      if (want_dot && dot_store) dsorted[(uint32_t)dot_slot < nA ? s + dot_slot : dummy_slot] = d;
      if (s2 >= end) break;
      const uint32_t s3 = s2 + U;
      if (s3 < end) nA = fetch(s3, end, DA, wA);
      d = accumulate_slots<TW, TG, VPL, U>(DB, wB, nB, acc, want_dot, lane);
      if (want_dot && dot_store) dsorted[(uint32_t)dot_slot < nB ? s2 + dot_slot : dummy_slot] = d;
      if (s3 >= end) break;
      s = s3;
    }
    if constexpr (SGD) {
      float p[NE];
#pragma unroll
      for (int v = 0; v < VPL; ++v) VecTraits<TW>::unpack(DA.wraw[v], p + v * EPV);
      sgd_store_row<TW, 64, VPL>(acc, p, end - beg, r, D, (int64_t)lane * EPV, lane, S);
    } else {
      char* orow = (char*)gW + (uint64_t)r * rowbytes;
      if constexpr (ACC) add_pending_row<TW, VPL>(orow, lane_byte, acc);
#pragma unroll
      for (int v = 0; v < VPL; ++v) st16_nt(orow + lane_byte + v * 1024u, VecTraits<TW>::pack(acc + v * EPV));
    }
  }
}

// ---------------------------------------------------------------------------
// Row reduction scheduled for L2 reuse of the upstream gradient.
//
// PKM lookups are not uniform over the table: a bag's lookups for one head
// are the best pairs (i1, i2) of two short sub-key lists, so they share a few
// i1 values, and row i1 * n + i2 lies in the block of n consecutive rows of
// its i1. A block of 1024 rows is touched by ~1500 distinct bags at the
// layer shape, most of them ~2.7 times. If the waves of one XCD (one L2)
// reduce the same block at the same time, those re-reads of a bag's gradient
// row hit that L2 instead of going out to the Infinity Cache.
//
// Rows are split into blocks of `blk` rows; block k belongs to row group
// k % 8, and workgroup w works for group w % 8 (the XCD that round-robin
// dispatch places it on). Each group hands out its rows in chunks of kDynRC
// consecutive rows, block after block, through kDynSub ticket counters
// (counter s serves chunks s, s + kDynSub, ... of every block; workgroup w
// uses counter (w / 8) % kDynSub, each counter on its own cache line): a
// wave takes the next ticket when it needs work, so the XCD's waves stay on
// one or two blocks at a time (a static split drifts apart over a kernel's
// length). Tickets are taken two chunks ahead and each chunk's row offsets
// and metadata are loaded one chunk ahead, so their latency hides under the
// current chunk's rows. Each row is still reduced by one wave in position
// order, so the sums are those of the per-64-rows kernel, bit for bit.
// Rows of U + 1 .. long_min lookups are reduced in place U lookups at a time;
// longer light rows are listed beforehand by list_long_rows_kernel, skipped
// here and reduced by eb_bwd_long_rows_kernel.
// ---------------------------------------------------------------------------
constexpr int kDynRC = 4;       // rows per ticket
constexpr int kDynGroups = 8;   // row groups: one per XCD
constexpr int kDynSub = 4;      // ticket counters per group (one counter serves ~70 M tickets/s)
constexpr int kCtrStride = 64;  // u32 entries between counters: one 256-byte line each

struct DynChunk {
  uint32_t row0;  // first row (wave-uniform); K for a chunk past the group's end
  uint32_t off;   // lane i <= kDynRC: offs[min(row0 + i, K)]
  uint32_t mb;    // lane l < kDynRC * U: bag of row l / U, slot l % U
  uint32_t mw;    // ... its weight (float32 bits)
};

// Rows with offs[r + 1] - offs[r] in (T, kHeavyT] (T = 2 U), listed for
// eb_bwd_long_rows_kernel. A workgroup owns rows_per_wg consecutive rows: it
// counts its long rows, takes its range of the list with one atomic (atomics
// on one address serialise, ~15 ns each), then writes them.
__global__ __launch_bounds__(256) void list_long_rows_kernel(const uint32_t* __restrict__ offs, int64_t K,
                                                             uint32_t T, int64_t rows_per_wg,
                                                             uint32_t* __restrict__ long_rows,
                                                             uint32_t* __restrict__ long_count) {
  __shared__ uint32_t wave_cnt[4];
  __shared__ uint32_t wg_base;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t r_beg = (int64_t)blockIdx.x * rows_per_wg;
  const int64_t r_end = r_beg + rows_per_wg < K ? r_beg + rows_per_wg : K;
  auto is_long = [&](int64_t r) {
    const uint32_t cnt = r < r_end ? offs[r + 1] - offs[r] : 0u;
    return cnt > T && cnt <= (uint32_t)kHeavyT;
  };
  uint32_t n = 0;
  for (int64_t r0 = r_beg + wv * 64; r0 < r_end; r0 += 256) n += (uint32_t)__popcll(__ballot(is_long(r0 + lane)));
  if (lane == 0) wave_cnt[wv] = n;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t total = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    wg_base = total ? atomicAdd(long_count, total) : 0u;
  }
  __syncthreads();
  uint32_t at = wg_base;
  for (int w = 0; w < wv; ++w) at += wave_cnt[w];
  if (n == 0) return;
  for (int64_t r0 = r_beg + wv * 64; r0 < r_end; r0 += 256) {
    const bool lng = is_long(r0 + lane);
    const uint64_t mask = __ballot(lng);
    if (lng) {
      const uint64_t below = lane == 0 ? 0ull : (mask & (~0ull >> (64 - lane)));
      long_rows[at + (uint32_t)__popcll(below)] = (uint32_t)(r0 + lane);
    }
    at += (uint32_t)__popcll(mask);
  }
}

// Register footprint of a row's loads in 16-byte vectors per lane: the table
// row plus, per prefetch slot, the gradient row in its own dtype.
template <typename TW, typename TG, int VPL>
constexpr int kRowVecs = VPL * GradTraits<TW, TG>::NV;

template <typename TW, typename TG, int VPL, int U, bool SGD, bool ACC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((kRowVecs<TW, TG, VPL> == 1 && U <= 4) ? 5 : ((kRowVecs<TW, TG, VPL> == 1 || (kRowVecs<TW, TG, VPL> == 2 && U <= 4)) ? 3 : 2)))) void eb_bwd_rows_dyn_kernel(
    const TW* __restrict__ W, int64_t K, int64_t D, int want_dot, const TG* __restrict__ g,
    const uint32_t* __restrict__ offs, const uint2* __restrict__ meta, const float* __restrict__ partials,
    const TW* __restrict__ zrow, TW* __restrict__ dummy_row, TW* __restrict__ gW, float* __restrict__ dsorted,
    uint32_t dummy_slot, uint32_t* __restrict__ tickets, uint32_t blk, uint32_t long_min, uint32_t hot_min,
    SgdArgs S) {
  static_assert(kDynRC * U <= 64, "a chunk's metadata must fit one load per lane");
  constexpr int EPV = VecTraits<TW>::EPV;
  constexpr int NE = VPL * EPV;
  const int lane = threadIdx.x & 63;
  const uint32_t grp = blockIdx.x % kDynGroups;
  const uint32_t sub = (blockIdx.x / kDynGroups) % kDynSub;
  const uint32_t nblk = (uint32_t)((K + blk - 1) / blk);
  const uint32_t grp_blocks = nblk > grp ? (nblk - grp + kDynGroups - 1) / kDynGroups : 0u;
  const uint32_t cpb = blk / (kDynRC * kDynSub);  // chunks per block and counter
  const uint32_t nchunks = grp_blocks * cpb;
  const uint32_t K32 = (uint32_t)K;
  constexpr int NV = GradTraits<TW, TG>::NV;
  const uint32_t lane_byte = (uint32_t)lane * 16u;
  const uint32_t glane_byte = lane_byte * NV;  // the lane's gradient elements (NV 16-byte pieces each)
  const uint64_t rowbytes = (uint64_t)D * sizeof(TW);
  const uint64_t growbytes = (uint64_t)D * sizeof(TG);
  const char* Wb = (const char*)W;
  const char* gb = (const char*)g;
  const char* zb = (const char*)zrow;
  uint32_t* ticket_ctr = tickets + (grp * kDynSub + sub) * kCtrStride;

  auto take_ticket = [&]() {
    uint32_t t = 0;
    if (lane == 0) t = atomicAdd(ticket_ctr, 1u);
    return t;  // lane 0's value; read with readlane when used
  };
  auto fetch_offs = [&](uint32_t t_lane0, DynChunk& C) {
    const uint32_t t = (uint32_t)__builtin_amdgcn_readlane((int)t_lane0, 0);
    C.row0 = K32;
    if (t < nchunks) C.row0 = (grp + kDynGroups * (t / cpb)) * blk + ((t % cpb) * kDynSub + sub) * kDynRC;
    const uint32_t i = (uint32_t)(lane < kDynRC ? lane : kDynRC);
    const uint32_t r = C.row0 + i < K32 ? C.row0 + i : K32;
    C.off = offs[r];
  };
  auto fetch_meta = [&](DynChunk& C) {
    const int ri = (lane / U) & (kDynRC - 1);
    const uint32_t beg = (uint32_t)__shfl((int)C.off, ri);
    const uint2 m = meta[beg + (uint32_t)(lane % U)];  // in bounds: meta is padded past every row start
    C.mb = m.x;
    C.mw = m.y;
  };
  auto get_meta = [&](const DynChunk& C, int i, RowMeta<U>& M, uint32_t& row, bool& skip) {
    M.beg = (uint32_t)__builtin_amdgcn_readlane((int)C.off, i);
    M.end = (uint32_t)__builtin_amdgcn_readlane((int)C.off, i + 1);
    const uint32_t cnt = M.end - M.beg;
    // listed for the long-row kernel, or a hot row (the matrix-core products write it)
    skip = (cnt > long_min && cnt <= (uint32_t)kHeavyT) || cnt >= hot_min;
    M.nh = cnt <= (uint32_t)U ? cnt : 0u;
    row = C.row0 + (uint32_t)i;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      M.b[u] = (uint32_t)__builtin_amdgcn_readlane((int)C.mb, i * U + u);
      M.w[u] = (uint32_t)u < M.nh ? __int_as_float(__builtin_amdgcn_readlane((int)C.mw, i * U + u)) : 0.f;
    }
  };
  // Rows and slots with nothing to read (tail rows past K, unused prefetch slots, W of a row without dots)
  // load through a size-0 buffer resource: zeros, no memory access, same instructions.
  auto issue = [&](const RowMeta<U>& M, uint32_t row, RowData<VPL, U, NV>& R, uint4* P) {
    // the SGD epilogue reads every table row (empty ones included)
    const bool read_w = SGD ? row < K32 : (want_dot && M.nh);
    const auto wr = row_rsrc(Wb + (uint64_t)(read_w ? row : 0u) * rowbytes, read_w ? (uint32_t)rowbytes : 0u);
#pragma unroll
    for (int v = 0; v < VPL; ++v) R.wraw[v] = ld16_rsrc<2>(wr, lane_byte + v * 1024u);  // nt: keep L2 for g
    if constexpr (ACC) {
      // the pending gradient of a row this kernel writes (one with lookups, not left to the long-row kernel)
      const uint32_t cnt = M.end - M.beg;
      const bool mine = row < K32 && cnt > 0 && !(cnt > long_min && cnt <= (uint32_t)kHeavyT) && cnt < hot_min;
      const auto pr = row_rsrc((const char*)gW + (uint64_t)(mine ? row : 0u) * rowbytes, mine ? (uint32_t)rowbytes : 0u);
#pragma unroll
      for (int v = 0; v < VPL; ++v) P[v] = ld16_rsrc<0>(pr, lane_byte + v * 1024u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool used = (uint32_t)u < M.nh;
      const auto gr = row_rsrc(gb + (uint64_t)(used ? M.b[u] : 0u) * growbytes, used ? (uint32_t)growbytes : 0u);
#pragma unroll
      for (int v = 0; v < VPL * NV; ++v) R.gvec[u][v] = ld16_rsrc<0>(gr, glane_byte + (v / NV) * 1024u * NV + (v % NV) * 16u);
    }
  };
  const int dot_slot = dot_slot_of<U>(lane);
  const bool dot_store = dot_store_of<U>(lane);
  const int64_t col0 = (int64_t)lane * EPV;
  // A row of U + 1 .. 2 U lookups is reduced in place, U lookups at a time,
  // in R's registers (its prefetch slots hold nothing for it); the next row's
  // loads stay in flight meanwhile. Longer light rows (rare at uniform-ish
  // lookups, crowded when lookups pile onto few rows) go to the long-row
  // kernel, which spreads them over all XCDs.
  auto reduce_long = [&](const RowMeta<U>& M, uint32_t row, RowData<VPL, U, NV>& R, float* acc) {
    const char* wrow = (want_dot || SGD) ? Wb + (uint64_t)row * rowbytes : zb;
#pragma unroll
    for (int v = 0; v < VPL; ++v) R.wraw[v] = ld16_nt(wrow + lane_byte + v * 1024u);
    for (uint32_t s = M.beg; s < M.end; s += U) {
      const uint32_t nh = (M.end - s) < (uint32_t)U ? (M.end - s) : (uint32_t)U;
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint2 m = meta[s + (uint32_t)u];  // uniform; in bounds: meta is padded past every row start
        w[u] = (uint32_t)u < nh ? __uint_as_float(m.y) : 0.f;
        const char* grow = (uint32_t)u < nh ? gb + (uint64_t)m.x * growbytes : zb;
#pragma unroll
        for (int v = 0; v < VPL * NV; ++v) R.gvec[u][v] = ld16(grow + glane_byte + (v / NV) * 1024u * NV + (v % NV) * 16u);
      }
      const float d = accumulate_slots<TW, TG, VPL, U>(R, w, nh, acc, want_dot != 0, lane);
      if (want_dot && dot_store) dsorted[(uint32_t)dot_slot < nh ? s + dot_slot : dummy_slot] = d;
    }
  };
  auto process = [&](const RowMeta<U>& M, uint32_t row, bool skip, RowData<VPL, U, NV>& R, const uint4* P) {
    if (skip) return;  // longer than 2 U (and light): reduced by the long-row kernel; or hot
    float acc[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.f;
    const uint32_t cnt = M.end - M.beg;
    if (cnt > (uint32_t)U && cnt <= (uint32_t)kHeavyT) {
      reduce_long(M, row, R, acc);
    } else {
      const float mydot = accumulate_slots<TW, TG, VPL, U>(R, M.w, M.nh, acc, want_dot != 0, lane);
      if (want_dot && dot_store) dsorted[(uint32_t)dot_slot < M.nh ? M.beg + dot_slot : dummy_slot] = mydot;
    }
    if (M.end - M.beg > (uint32_t)kHeavyT) add_heavy_partials<64, VPL, EPV>(M.beg, M.end, partials, D, col0, acc);
    if constexpr (SGD) {
      if (row < K32) {
        float p[NE];
#pragma unroll
        for (int v = 0; v < VPL; ++v) VecTraits<TW>::unpack(R.wraw[v], p + v * EPV);
        sgd_store_row<TW, 64, VPL>(acc, p, cnt, row, D, col0, lane, S);
      }
    } else {
      if constexpr (ACC) {
        if (cnt == 0) return;  // no lookups: the row keeps its pending gradient
        unpack_add_pending<TW, VPL>(P, acc);
      }
      char* orow = row < K32 ? (char*)gW + (uint64_t)row * rowbytes : (char*)dummy_row;
#pragma unroll
      for (int v = 0; v < VPL; ++v) st16_nt(orow + lane_byte + v * 1024u, VecTraits<TW>::pack(acc + v * EPV));
    }
  };

  // prologue: chunk 0's offsets and metadata, chunk 1's offsets, chunk 2's ticket
  DynChunk cur, nxt, nn;
  const uint32_t t0 = take_ticket();
  const uint32_t t1 = take_ticket();
  uint32_t tk = take_ticket();
  fetch_offs(t0, cur);
  if (cur.row0 >= K32) return;  // nothing left for this group
  fetch_meta(cur);
  fetch_offs(t1, nxt);

  RowMeta<U> MA, MB;
  RowData<VPL, U, NV> DA, DB;
  uint4 PA[ACC ? VPL : 1], PB[ACC ? VPL : 1];  // pending gradient rows (accumulating reduction)
  uint32_t rowA, rowB;
  bool skA, skB;
  get_meta(cur, 0, MA, rowA, skA);
  issue(MA, rowA, DA, PA);
  get_meta(cur, 1, MB, rowB, skB);
  // One chunk's 4 rows per trip, rows i and i + 1 in flight across chunk
  // boundaries. The order keeps every wait partial: each load is first used
  // after a row whose gradient loads were issued after it (gfx9's vmcnt is
  // in order), so no use waits for loads still needed in flight, and the
  // chunk states are copied only once their loads have landed.
  static_assert(kDynRC == 4, "the loop body walks 4 rows per chunk");
  while (true) {
    fetch_offs(tk, nn);   // the chunk after next (its ticket was taken one trip ago)
    tk = take_ticket();
    issue(MB, rowB, DB, PB);  // row 1
    fetch_meta(nxt);          // its offsets were loaded one trip ago
    process(MA, rowA, skA, DA, PA);  // row 0
    get_meta(cur, 2, MA, rowA, skA);
    issue(MA, rowA, DA, PA);  // row 2
    process(MB, rowB, skB, DB, PB);  // row 1
    get_meta(cur, 3, MB, rowB, skB);
    issue(MB, rowB, DB, PB);  // row 3
    process(MA, rowA, skA, DA, PA);  // row 2 (its wait covers nxt's metadata)
    const bool more = nxt.row0 < K32;
    if (more) {
      get_meta(nxt, 0, MA, rowA, skA);
      issue(MA, rowA, DA, PA);  // next chunk's row 0
    }
    process(MB, rowB, skB, DB, PB);  // row 3
    if (!more) break;
    get_meta(nxt, 1, MB, rowB, skB);
    cur = nxt;
    nxt = nn;
  }
}

// meta[i] = {bag, weight as float32 bits} of sorted occurrence i;
// entries past the valid count (padding included) are zero.
__global__ void occ_meta_kernel(const uint32_t* __restrict__ svals, const uint32_t* __restrict__ nvalid,
                                int64_t n_total, uint32_t L32, const void* __restrict__ psw, int pdt,
                                uint2* __restrict__ meta) {
  const uint32_t nv = *nvalid;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_total; i += (int64_t)gridDim.x * blockDim.x) {
    uint2 m = make_uint2(0u, 0u);
    if (i < (int64_t)nv) {
      const uint32_t p = svals[i];
      m.x = p / L32;
      m.y = __float_as_uint(psw ? load_scalar(psw, pdt, p) : 1.f);
    }
    meta[i] = m;
  }
}


// gpsw[position] <- psw-gradient dots computed in sorted order; gpsw <- 0 at
// the positions the sort listed as out-of-range lookups (invalid: count, then
// positions).
__global__ void gpsw_scatter_kernel(const uint32_t* __restrict__ svals, const float* __restrict__ dsorted,
                                    const uint32_t* __restrict__ nvalid, int64_t N, void* __restrict__ gpsw, int pdt,
                                    const uint32_t* __restrict__ invalid) {
  const uint32_t nv = *nvalid;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < N; i += (int64_t)gridDim.x * blockDim.x) {
    if (i >= (int64_t)nv) break;
    store_scalar(gpsw, pdt, svals[i], dsorted[i]);
  }
  const uint32_t nbad = invalid[0];
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < nbad; i += gridDim.x * blockDim.x)
    store_scalar(gpsw, pdt, invalid[1 + i], 0.f);
}

// gpsw[p] <- 0 for the positions the sort listed as out-of-range lookups.
__global__ void zero_invalid_gpsw_kernel(const uint32_t* __restrict__ invalid, void* __restrict__ gpsw, int pdt) {
  const uint32_t n = invalid[0];
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    store_scalar(gpsw, pdt, invalid[1 + i], 0.f);
}

// ---------------------------------------------------------------------------
// Hot rows on the matrix cores. A row with at least hot_min lookups (a
// sizeable share of the bags: hot_min >= bags / 16) is reduced as a row of
// two dense products instead of one gradient-row read per lookup:
//   gW[hot[i]] = sum_b C[i, b] G[b]     C[i, b] = sum of psw over the row's lookups in bag b
//   E[i, b]    = <W[hot[i]], G[b]>      psw-gradient of each lookup of the row in bag b
// with G the upstream gradient [bags, D]: bf16 operands, float32 sums, on
// v_mfma_f32_16x16x32_bf16. C is never materialised. The row's lookups,
// sorted by position and hence by bag, are merged per bag into entries (the
// weights of one bag summed in float32, in position order), split into chunks
// of 32 bags, and each MFMA tile of C is built in LDS from the entries. A
// merged weight that bf16 does not hold exactly (a bag holding the row twice,
// float32 weights) is carried as hi + lo, both bf16; lo entries are read, and
// lo tiles multiplied, only in the chunks that have one. The sums run in a
// fixed order (deterministic), but not in position order, so they may differ
// from the light rows' in the last float32 bits.
// ---------------------------------------------------------------------------
constexpr int kHotKC = 32;         // bags per chunk (one MFMA k-step)
constexpr int kHotM = 64;          // hot rows per gradient-product tile
constexpr int kHotN = 512;         // table columns per gradient-product tile
constexpr int kHotGradThreads = 512;  // gradient product: 8 waves of 64 rows x 64 columns
constexpr int kHotDM = 128;        // hot rows per dot-product tile
constexpr int kHotDN = 128;        // bags per dot-product tile
constexpr int kHotDK = 64;         // dims per chunk of the dot product
constexpr int kHotThreads = 256;   // 4 waves of 64 x 64
constexpr uint32_t kHotLo = 0x80000000u;  // chunk-pointer flag: the row's chunk holds a lo entry
constexpr int kHotLoList = 256;    // lo chunks one row lists before it flags all of its chunks

// For each listed row i (row r = hot[i], count at hot[hr_max]; sorted
// occurrences [offs[r], offs[r+1])): the row's entries, one per distinct bag
// in bag order, written over the start of the row's own occurrence range of
// ent (bag % 32 | hi << 16) and ent_lo (lo); chunk pointers, chunk-major
// (index c * hr_max + i), pc (first entry, | kHotLo if the chunk holds a lo)
// and po (first occurrence) of the row's first bag >= 32 c, for c = 0..nc (c =
// nc: the row's ends); any_lo <- 1 if some lo is nonzero. A block per row,
// grid-stride over the list (every block reads the count).
__global__ __launch_bounds__(256) void hot_list_kernel(const uint32_t* __restrict__ hot, int64_t hr_max,
                                                       const uint32_t* __restrict__ offs,
                                                       const uint2* __restrict__ meta, uint32_t nc,
                                                       uint32_t* __restrict__ pc, uint32_t* __restrict__ po,
                                                       uint32_t* __restrict__ ent, uint16_t* __restrict__ ent_lo,
                                                       uint32_t* __restrict__ any_lo) {
  __shared__ uint32_t lds4[4];
  __shared__ uint32_t lo_chunks[kHotLoList];
  __shared__ uint32_t n_lo;
  const uint32_t n = hot[hr_max];
  const size_t H = (size_t)hr_max;
  for (uint32_t i = blockIdx.x; i < n; i += gridDim.x) {
    const uint32_t r = hot[i];
    const uint32_t beg = offs[r], end = offs[r + 1];
    if (threadIdx.x == 0) n_lo = 0u;
    __syncthreads();
    uint32_t carry = 0;  // entries of the row's earlier occurrence tiles
    for (uint32_t j0 = beg; j0 < end; j0 += 256) {
      const uint32_t j = j0 + threadIdx.x;
      uint32_t bag = 0, prev = 0;
      bool start = false;
      if (j < end) {
        bag = meta[j].x;
        prev = j > beg ? meta[j - 1].x : 0u;
        start = j == beg || bag != prev;
      }
      uint32_t tot;
      const uint32_t k = carry + block_exclusive_sum(start ? 1u : 0u, &tot, lds4);
      if (start) {
        // chunks (chunk of the previous occurrence, chunk of this one] start here
        const uint32_t c = bag / kHotKC;
        for (uint32_t cc = j == beg ? 0u : prev / kHotKC + 1u; cc <= c; ++cc) {
          pc[cc * H + i] = beg + k;
          po[cc * H + i] = j;
        }
        float s = __uint_as_float(meta[j].y);
        for (uint32_t t = j + 1; t < end && meta[t].x == bag; ++t) s += __uint_as_float(meta[t].y);
        const uint32_t hi = f32_to_bf16_bits(s);
        const uint32_t lo = f32_to_bf16_bits(s - bf16_to_f32(hi));
        ent[beg + k] = (bag % kHotKC) | (hi << 16);
        ent_lo[beg + k] = (uint16_t)lo;
        if ((lo & 0x7FFFu) != 0u) {
          *any_lo = 1u;
          const uint32_t at = atomicAdd(&n_lo, 1u);
          if (at < (uint32_t)kHotLoList) lo_chunks[at] = c;
        }
      }
      carry += tot;
    }
    const uint32_t c_end = end > beg ? meta[end - 1].x / kHotKC + 1u : 0u;
    for (uint32_t cc = c_end + threadIdx.x; cc <= nc; cc += 256) {
      pc[cc * H + i] = beg + carry;
      po[cc * H + i] = end;
    }
    __syncthreads();  // every pointer of the row written, n_lo final
    const uint32_t nl = n_lo;
    if (nl > (uint32_t)kHotLoList) {
      for (uint32_t cc = threadIdx.x; cc < nc; cc += 256) pc[cc * H + i] |= kHotLo;
    } else {
      for (uint32_t t = threadIdx.x; t < nl; t += 256) atomicOr(&pc[lo_chunks[t] * H + i], kHotLo);
    }
    __syncthreads();  // n_lo and lo_chunks before the next row
  }
}

// [rows][32] and [rows][64] bf16 LDS tiles: the 16-byte slots of a row are
// rotated by the row (eight consecutive rows read at one slot cover all banks).
__device__ __forceinline__ int hot_swz32(int row, int col) {
  return row * 32 + ((((col >> 3) ^ (row >> 1)) & 3) << 3) + (col & 7);
}
__device__ __forceinline__ int hot_swz64(int row, int col) {
  return row * 64 + ((((col >> 3) ^ row) & 7) << 3) + (col & 7);
}

// Tile t of mt x nt -> (m, n), m fastest. With 8 | nt, the tiles of
// workgroups on XCD x (t % 8 = x for a grid of a multiple of 8) take the
// n-tiles [x nt / 8, (x + 1) nt / 8): one XCD's L2 serves each operand column.
__device__ __forceinline__ void hot_tile(uint32_t t, uint32_t mt, uint32_t nt, uint32_t& m, uint32_t& n) {
  if ((nt & 7u) == 0u) {
    const uint32_t per = nt >> 3, x = t & 7u, j = t >> 3;
    m = j % mt;
    n = x * per + j / mt;
  } else {
    m = t % mt;
    n = t / mt;
  }
}

typedef __bf16 hot_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float hot_f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void hot_mma(const uint4& a, const uint4& b, hot_f32x4_t& c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(hot_bf16x8_t, a),
                                              __builtin_bit_cast(hot_bf16x8_t, b), c, 0, 0, 0);
}

// Gt[d][b] = G[b][d] for b < bags, 0 for bags <= b < 32 nc (the gradient
// product's bag operand, bag-contiguous), and with Wh != NULL, Wh[i] =
// W[hot[i]] (the dot product's row operand, contiguous); nothing without hot
// rows. Tiles of 32 bags x 64 columns through LDS, grid-stride.
__global__ __launch_bounds__(256) void hot_operands_kernel(const uint32_t* __restrict__ hot, int64_t hr_max,
                                                           const bf16_t* __restrict__ G, int64_t B, uint32_t nc,
                                                           int64_t D, uint16_t* __restrict__ Gt,
                                                           const bf16_t* __restrict__ W, uint16_t* __restrict__ Wh) {
  __shared__ uint16_t tile[32][64 + 2];
  const uint32_t count = hot[hr_max];
  if (count == 0) return;
  const int tid = threadIdx.x;
  const int64_t Bp = (int64_t)nc * kHotKC;
  const int64_t ncol = D / 64;
  const int64_t tiles = (int64_t)nc * ncol;
  const uint16_t* g16 = (const uint16_t*)G;
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int64_t b0 = (t / ncol) * kHotKC, d0 = (t % ncol) * 64;
    {
      const int bl = tid >> 3, part = tid & 7;  // bag b0 + bl, columns d0 + 8 part
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (b0 + bl < B) v = ld16(g16 + (b0 + bl) * D + d0 + 8 * part);
      const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tile[bl][8 * part + 2 * e] = (uint16_t)(x[e] & 0xFFFFu);
        tile[bl][8 * part + 2 * e + 1] = (uint16_t)(x[e] >> 16);
      }
    }
    __syncthreads();
    {
      const int col = tid >> 2, grp = tid & 3;  // column d0 + col, bags b0 + 8 grp .. + 7
      uint32_t x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        x[e] = (uint32_t)tile[8 * grp + 2 * e][col] | ((uint32_t)tile[8 * grp + 2 * e + 1][col] << 16);
      *(uint4*)(Gt + (d0 + col) * Bp + b0 + 8 * grp) = make_uint4(x[0], x[1], x[2], x[3]);
    }
    __syncthreads();
  }
  if (Wh == nullptr) return;
  const int64_t per_row = D / 8;  // 16-byte pieces
  const int64_t n16 = (int64_t)count * per_row;
  for (int64_t k = (int64_t)blockIdx.x * 256 + tid; k < n16; k += (int64_t)gridDim.x * 256) {
    const int64_t i = k / per_row, c = k % per_row;
    *(uint4*)(Wh + i * D + 8 * c) = ld16((const uint16_t*)W + (int64_t)hot[i] * D + 8 * c);
  }
}

// Bag splits of the gradient product (split-K): the largest power of two S
// that keeps S x (row tiles) x (column tiles) <= kHotTiles workgroup tiles, at
// least 8 chunks per split and the S partial row blocks within part_rows.
// S = 1: the product writes gW itself; else float32 partials, summed in split
// order by hot_finish_kernel.
constexpr uint32_t kHotTiles = 1024;
__device__ __forceinline__ uint32_t hot_splits(uint32_t count, int64_t D, uint32_t nc, int64_t part_rows) {
  const uint32_t mt = (count + kHotM - 1) / kHotM, nt = (uint32_t)(D / kHotN);
  uint32_t S = 1;
  while (S < 64 && 2 * S * mt * nt <= kHotTiles && nc >= 16 * S && (int64_t)(2 * S * mt) * kHotM <= part_rows) S *= 2;
  return S;
}

// gW[hot[i], n0 + col] for a tile of 64 hot rows x 512 columns: the sum over
// the bags' chunks of C-tile x Gt-tile. Wave w of 8 builds the C tile's rows
// 8 w .. 8 w + 7 from their entries, two rows per load (32 lanes a row: a
// chunk holds at most 32 distinct bags), and multiplies all 64 rows by its
// 64 columns of the Gt tile (each C tile serves 512 columns). C tiles triple-buffered and Gt tiles
// double-buffered in LDS, one barrier per chunk; a chunk's entries and Gt
// rows are loaded two chunks ahead, into alternating register stages (every
// load issued on every path, at clamped addresses, so the waits stay
// partial); each stage carries the chunk pointers of its next chunk. With S >
// 1 bag splits, tile (m, n, s) sums the chunks [s nc / S, (s + 1) nc / S) into
// the float32 partial rows s mt 64 + (hot row index). ACC: the sum is added to
// the gradient gW already holds (rounded to bf16 first, as the light rows do).
template <bool ACC>
__global__ __launch_bounds__(kHotGradThreads) __attribute__((amdgpu_waves_per_eu(2))) void hot_grad_kernel(
    const uint32_t* __restrict__ hot, int64_t hr_max, const uint32_t* __restrict__ pc, uint32_t nc,
    const uint32_t* __restrict__ ent, const uint16_t* __restrict__ ent_lo, const uint16_t* __restrict__ Gt,
    int64_t D, bf16_t* __restrict__ gW, float* __restrict__ part, int64_t part_rows) {
  constexpr int AT = kHotM * kHotKC;  // bf16 per C tile (4 KB)
  constexpr int BT = kHotN * kHotKC;  // bf16 per Gt tile (16 KB)
  __shared__ __align__(16) uint16_t Ah[3 * AT];
  __shared__ __align__(16) uint16_t Al[3 * AT];
  __shared__ __align__(16) uint16_t Bt[2 * BT];
  __shared__ uint32_t rows[kHotM];
  __shared__ uint32_t lo_tag[3];  // chunk + 1 of the last chunk that put a lo entry into the slot
  const uint32_t count = hot[hr_max];
  const bool any_lo = hot[hr_max + 1] != 0u;
  const uint32_t mt = (count + kHotM - 1) / kHotM, nt = (uint32_t)(D / kHotN);
  const uint32_t NS = hot_splits(count, D, nc, part_rows);
  const size_t H = (size_t)hr_max;
  const int64_t Bp = (int64_t)nc * kHotKC;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int eh = lane >> 5, el = lane & 31;  // entries: row 8 w + 2 s + eh of slot s, entry el of its chunk
  const int gcol = tid >> 2, gpart = tid & 3;  // Gt: columns gcol + 128 u, bags 8 gpart .. + 7 of the chunk
  // loaded values are kept as loaded (a select on one would wait for it); okm / flm: slots with an entry /
  // with a lo flag, from the pointers
  struct Stage {
    uint32_t p0, p1;  // chunk pointers (flagged) of the stage's next chunk, for the lane's row 8 w + (lane & 7)
    uint32_t okm, flm;
    uint32_t e[4];
    uint32_t lo[4];
    uint4 g[4];
  };
  for (uint32_t t = blockIdx.x; t < mt * NS * nt; t += gridDim.x) {
    uint32_t ms, n;
    hot_tile(t, mt * NS, nt, ms, n);
    const uint32_t m = ms % mt, sp = ms / mt;
    const uint32_t cb = (uint32_t)((uint64_t)sp * nc / NS), ce = (uint32_t)((uint64_t)(sp + 1) * nc / NS);
    const uint32_t i0 = m * kHotM;
    const int64_t n0 = (int64_t)n * kHotN;
    if (tid < kHotM) rows[tid] = i0 + tid < count ? hot[i0 + tid] : 0u;
    if (tid < 3) lo_tag[tid] = 0u;
    // the lane's row for the chunk pointers; a row past the count reads row 0's (its sums are never stored)
    const uint32_t prow = i0 + 8 * w + (lane & 7);
    const size_t prow_c = prow < count ? prow : 0u;
    const uint16_t* gbase = Gt + (n0 + gcol) * Bp + 8 * gpart;
    // load chunk c (pointers S.p0 / S.p1 = its own), then S.p0 / S.p1 <- chunk c + 2's
    auto load = [&](Stage& S, uint32_t c) {
      uint32_t k[4];
      S.okm = S.flm = 0u;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        // rows 2 s (lanes 0-31) and 2 s + 1 (lanes 32-63) of the wave: lane reads, no LDS round trips
        const uint32_t a0 = (uint32_t)__builtin_amdgcn_readlane((int)S.p0, 2 * s);
        const uint32_t b0 = (uint32_t)__builtin_amdgcn_readlane((int)S.p0, 2 * s + 1);
        const uint32_t a1 = (uint32_t)__builtin_amdgcn_readlane((int)S.p1, 2 * s);
        const uint32_t b1 = (uint32_t)__builtin_amdgcn_readlane((int)S.p1, 2 * s + 1);
        const uint32_t p0f = eh ? b0 : a0;
        const uint32_t p1 = (eh ? b1 : a1) & ~kHotLo;
        const uint32_t p0 = p0f & ~kHotLo;
        const uint32_t kk = p0 + (uint32_t)el;
        const bool ok = kk < p1;
        // a lane past the chunk reads the entry before the row's chunk (in bounds, the lanes' own lines;
        // one index shared by every such lane of the grid would make one hot cache line)
        k[s] = ok ? kk : (p0 > 0u ? p0 - 1u : 0u);
        S.okm |= ok ? 1u << s : 0u;
        S.flm |= (ok && (p0f & kHotLo) != 0u) ? 1u << s : 0u;
      }
      const uint32_t c2 = c + 2 < ce ? c + 2 : ce, c3 = c + 3 < ce ? c + 3 : ce;
      S.p0 = pc[c2 * H + prow_c];
      S.p1 = pc[c3 * H + prow_c];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        S.e[s] = ent[k[s]];
        S.lo[s] = ent_lo[k[s]];
      }
      const int64_t bc = (int64_t)(c < ce ? c : ce - 1) * kHotKC;
#pragma unroll
      for (int u = 0; u < 4; ++u) S.g[u] = ld16(gbase + 128 * u * Bp + bc);
    };
    auto put = [&](const Stage& S, int slot, uint32_t c, uint16_t* Bs) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if ((S.okm >> s) & 1u) {
          const int at = slot * AT + hot_swz32(8 * w + 2 * s + eh, (int)(S.e[s] % kHotKC));
          Ah[at] = (uint16_t)(S.e[s] >> 16);
          if (((S.flm >> s) & 1u) && (S.lo[s] & 0x7FFFu) != 0u) {
            Al[at] = (uint16_t)S.lo[s];
            lo_tag[slot] = c + 1u;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) *(uint4*)(Bs + hot_swz32(gcol + 128 * u, 8 * gpart)) = S.g[u];
    };
    auto zero = [&](uint16_t* T) {
      if (tid < AT / 8) *(uint4*)(T + 8 * tid) = make_uint4(0u, 0u, 0u, 0u);
    };
    hot_f32x4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = hot_f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](int slot, uint32_t c, const uint16_t* Bs) {
      uint4 a[4], b[4];
#pragma unroll
      for (int mt_ = 0; mt_ < 4; ++mt_) a[mt_] = *(const uint4*)(Ah + slot * AT + hot_swz32(16 * mt_ + r, 8 * q));
#pragma unroll
      for (int nt_ = 0; nt_ < 4; ++nt_) b[nt_] = *(const uint4*)(Bs + hot_swz32(64 * w + 16 * nt_ + r, 8 * q));
#pragma unroll
      for (int nt_ = 0; nt_ < 4; ++nt_)
#pragma unroll
        for (int mt_ = 0; mt_ < 4; ++mt_) hot_mma(a[mt_], b[nt_], acc[mt_][nt_]);
      if (lo_tag[slot] == c + 1u) {  // uniform
#pragma unroll
        for (int mt_ = 0; mt_ < 4; ++mt_) a[mt_] = *(const uint4*)(Al + slot * AT + hot_swz32(16 * mt_ + r, 8 * q));
#pragma unroll
        for (int nt_ = 0; nt_ < 4; ++nt_)
#pragma unroll
          for (int mt_ = 0; mt_ < 4; ++mt_) hot_mma(a[mt_], b[nt_], acc[mt_][nt_]);
      }
    };
    // stage (c - cb) & 1 holds chunk c; chunk pointers of chunks cb and cb + 1 to start with
    Stage s0, s1;
    s0.p0 = pc[cb * H + prow_c];
    s0.p1 = pc[(cb + 1) * H + prow_c];
    s1.p0 = s0.p1;
    s1.p1 = pc[(cb + 2 < ce ? cb + 2 : ce) * H + prow_c];
    zero(Ah);
    zero(Ah + AT);
    if (any_lo) {
      zero(Al);
      zero(Al + AT);
      zero(Al + 2 * AT);
    }
    load(s0, cb);
    load(s1, cb + 1);
    __syncthreads();
    put(s0, 0, cb, Bt + (cb & 1) * BT);
    load(s0, cb + 2);
    __syncthreads();
    // iteration c: put chunk c + 1 (its stage), reload that stage with chunk c + 3, multiply chunk c. Both
    // bodies of a trip run on every path (an odd count ends with an empty one) and every load is issued in
    // each: the waits for a stage's loads stay partial.
    auto body = [&](uint32_t c, int ia, Stage& S) {
      const int ia1 = ia == 2 ? 0 : ia + 1, ia2 = ia1 == 2 ? 0 : ia1 + 1;
      // slot ia2 held chunk c - 1 (multiplied before the last barrier); its lo tile was put to only if
      // its tag says so (the tags start at 0 and the lo tiles zeroed)
      zero(Ah + ia2 * AT);
      if (any_lo && lo_tag[ia2] == c) zero(Al + ia2 * AT);
      if (c + 1 < ce) put(S, ia1, c + 1, Bt + ((c + 1) & 1) * BT);
      load(S, c + 3);
      if (c < ce) mma(ia, c, Bt + (c & 1) * BT);
      __syncthreads();
    };
    int ia = 0;
    for (uint32_t c = cb; c < ce; c += 2) {
      body(c, ia, s1);
      ia = ia == 2 ? 0 : ia + 1;
      body(c + 1, ia, s0);
      ia = ia == 2 ? 0 : ia + 1;
    }
    // acc[mt][nt][e]: tile row 16 mt + 4 q + e, column 64 w + 16 nt + r
    uint16_t* out = (uint16_t*)gW;
#pragma unroll
    for (int mt_ = 0; mt_ < 4; ++mt_) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * mt_ + 4 * q + e;
        if (i0 + row < count) {
          if (NS > 1) {
            float* prow = part + ((int64_t)sp * mt * kHotM + i0 + row) * D + n0 + 64 * w + r;
#pragma unroll
            for (int nt_ = 0; nt_ < 4; ++nt_) prow[16 * nt_] = acc[mt_][nt_][e];
          } else {
            const int64_t base = (int64_t)rows[row] * D + n0 + 64 * w + r;
#pragma unroll
            for (int nt_ = 0; nt_ < 4; ++nt_) {
              float v = acc[mt_][nt_][e];
              if constexpr (ACC) v = bf16_to_f32(out[base + 16 * nt_]) + round_to<bf16_t>(v);
              out[base + 16 * nt_] = (uint16_t)f32_to_bf16_bits(v);
            }
          }
        }
      }
    }
    __syncthreads();  // rows and tags before the next tile
  }
}

// With S > 1 bag splits: gW[hot[i]] = bf16(sum over the splits, in split
// order, of the float32 partial rows) (ACC: added to the pending gradient as
// the product's own epilogue does); nothing with one split.
template <bool ACC>
__global__ __launch_bounds__(256) void hot_finish_kernel(const uint32_t* __restrict__ hot, int64_t hr_max,
                                                         uint32_t nc, int64_t D, const float* __restrict__ part,
                                                         int64_t part_rows, bf16_t* __restrict__ gW) {
  const uint32_t count = hot[hr_max];
  const uint32_t NS = hot_splits(count, D, nc, part_rows);
  if (NS == 1) return;
  const int64_t rows_per_split = (int64_t)((count + kHotM - 1) / kHotM) * kHotM;
  const int64_t per_row = D / 4;
  const int64_t n4 = (int64_t)count * per_row;
  uint16_t* out = (uint16_t*)gW;
  for (int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x; k < n4; k += (int64_t)gridDim.x * 256) {
    const int64_t i = k / per_row, c = 4 * (k % per_row);
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t sp = 0; sp < NS; ++sp) {
      const float4 v = *(const float4*)(part + (sp * rows_per_split + i) * D + c);
      a[0] += v.x;
      a[1] += v.y;
      a[2] += v.z;
      a[3] += v.w;
    }
    uint16_t* o = out + (int64_t)hot[i] * D + c;
    uint32_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = a[e];
      if constexpr (ACC) v = bf16_to_f32(o[e]) + round_to<bf16_t>(v);
      b[e] = f32_to_bf16_bits(v);
    }
    *(uint2*)o = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
  }
}

// dsorted[j] = <Wh[i], G[bag of j]> for the occurrences j of the hot rows:
// tiles of 128 hot rows x 128 bags, the dense product over D in chunks of 64
// dims (both operands row-major, copied straight into LDS, double-buffered,
// one barrier per chunk; loaded two chunks ahead into alternating register
// stages), then the tile through LDS to the tile's occurrences (po: the rows'
// occurrences by 32-bag chunk, chunk-major).
__global__ __launch_bounds__(kHotThreads) __attribute__((amdgpu_waves_per_eu(2))) void hot_dot_kernel(
    const uint32_t* __restrict__ hot, int64_t hr_max, const uint32_t* __restrict__ po, uint32_t nc,
    const uint2* __restrict__ meta, const uint16_t* __restrict__ Wh, const bf16_t* __restrict__ G, int64_t B,
    int64_t D, float* __restrict__ dsorted) {
  constexpr int T = kHotDM * kHotDK;  // bf16 per operand tile (16 KB)
  constexpr int EP = kHotDN + 4;      // E row pitch (floats)
  static_assert(4 * T * 2 <= kHotDM * EP * 4, "operand tiles fit the E buffer");
  __shared__ __align__(16) uint32_t smem[kHotDM * EP];  // 2 x (W tile, G tile), or E [row][bag]
  uint16_t* As = (uint16_t*)smem;
  uint16_t* Bs = As + 2 * T;
  float* E = (float*)smem;
  const uint32_t count = hot[hr_max];
  const uint32_t mt = (count + kHotDM - 1) / kHotDM, nt = (uint32_t)((B + kHotDN - 1) / kHotDN);
  const size_t H = (size_t)hr_max;
  const int nk = (int)(D / kHotDK);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w & 1, wn = w >> 1;
  const int r = lane & 15, q = lane >> 4;
  const int lrow = tid >> 3, lslot = tid & 7;  // operand loads: rows lrow + 32 u, 16-byte slot
  const uint32_t* meta32 = (const uint32_t*)meta;
  const uint16_t* g16 = (const uint16_t*)G;
  struct Stage {
    uint4 a[4], b[4];
  };
  for (uint32_t t = blockIdx.x; t < mt * nt; t += gridDim.x) {
    uint32_t m, n;
    hot_tile(t, mt, nt, m, n);
    const uint32_t i0 = m * kHotDM;
    const int64_t b0 = (int64_t)n * kHotDN;
    const uint16_t* wp[4];
    const uint16_t* gp[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t rr = i0 + lrow + 32 * u;
      wp[u] = Wh + (int64_t)(rr < count ? rr : count - 1) * D + 8 * lslot;
      const int64_t b = b0 + lrow + 32 * u < B ? b0 + lrow + 32 * u : B - 1;
      gp[u] = g16 + b * D + 8 * lslot;
    }
    auto load = [&](Stage& S, int k) {
      const int kc = (k < nk ? k : nk - 1) * kHotDK;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        S.a[u] = ld16(wp[u] + kc);
        S.b[u] = ld16(gp[u] + kc);
      }
    };
    auto put = [&](const Stage& S, int buf) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        *(uint4*)(As + buf * T + hot_swz64(lrow + 32 * u, 8 * lslot)) = S.a[u];
        *(uint4*)(Bs + buf * T + hot_swz64(lrow + 32 * u, 8 * lslot)) = S.b[u];
      }
    };
    hot_f32x4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = hot_f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](int buf) {
#pragma unroll
      for (int ks = 0; ks < kHotDK / 32; ++ks) {
        uint4 a[4], b[4];
#pragma unroll
        for (int mt_ = 0; mt_ < 4; ++mt_)
          a[mt_] = *(const uint4*)(As + buf * T + hot_swz64(64 * wm + 16 * mt_ + r, 32 * ks + 8 * q));
#pragma unroll
        for (int nt_ = 0; nt_ < 4; ++nt_)
          b[nt_] = *(const uint4*)(Bs + buf * T + hot_swz64(64 * wn + 16 * nt_ + r, 32 * ks + 8 * q));
#pragma unroll
        for (int nt_ = 0; nt_ < 4; ++nt_)
#pragma unroll
          for (int mt_ = 0; mt_ < 4; ++mt_) hot_mma(a[mt_], b[nt_], acc[mt_][nt_]);
      }
    };
    // stage k & 1 holds chunk k; iteration k: put chunk k + 1, reload its stage with chunk k + 3, multiply chunk k
    Stage s0, s1;
    load(s0, 0);
    load(s1, 1);
    put(s0, 0);
    load(s0, 2);
    __syncthreads();
    // both bodies of a trip run on every path (an odd count ends with an empty one): partial waits
    auto body = [&](int k, Stage& S) {
      if (k + 1 < nk) put(S, (k + 1) & 1);  // its buffer was last read by chunk k - 1, before the last barrier
      load(S, k + 3);
      if (k < nk) mma(k & 1);
      __syncthreads();
    };
    for (int k = 0; k < nk; k += 2) {
      body(k, s1);
      body(k + 1, s0);
    }
    // E tile through LDS: acc[mt][nt][e] is tile row 64 wm + 16 mt + 4 q + e, bag 64 wn + 16 nt + r
#pragma unroll
    for (int mt_ = 0; mt_ < 4; ++mt_)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int nt_ = 0; nt_ < 4; ++nt_) E[(64 * wm + 16 * mt_ + 4 * q + e) * EP + 64 * wn + 16 * nt_ + r] = acc[mt_][nt_][e];
    __syncthreads();
    // wave w: tile rows 32 w .. 32 w + 31; lanes < 32 hold a row's occurrence range in the tile's 4 chunks
    const uint32_t cb = (uint32_t)(b0 / kHotKC), ce = cb + kHotDN / kHotKC < nc ? cb + kHotDN / kHotKC : nc;
    uint32_t pA = 0, pB = 0;
    if (lane < 32 && i0 + 32 * w + lane < count) {
      pA = po[cb * H + i0 + 32 * w + lane];
      pB = po[ce * H + i0 + 32 * w + lane];
    }
    uint32_t len = pB - pA;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t x = (uint32_t)__shfl_xor((int)len, o);
      len = x > len ? x : len;
    }
    for (uint32_t p = 0; p < len; p += 64) {
      uint32_t bag[32];
#pragma unroll
      for (int qq = 0; qq < 32; ++qq) {
        const uint32_t j0 = (uint32_t)__builtin_amdgcn_readlane((int)pA, qq);
        const uint32_t j1 = (uint32_t)__builtin_amdgcn_readlane((int)pB, qq);
        const uint32_t j = j0 + p + (uint32_t)lane;
        bag[qq] = j < j1 ? meta32[2 * (size_t)j] : 0xFFFFFFFFu;
      }
#pragma unroll
      for (int qq = 0; qq < 32; ++qq) {
        if (bag[qq] != 0xFFFFFFFFu) {
          const uint32_t j = (uint32_t)__builtin_amdgcn_readlane((int)pA, qq) + p + (uint32_t)lane;
          const uint32_t col = bag[qq] - (uint32_t)b0;
          dsorted[j] = E[(32 * w + qq) * EP + (col < (uint32_t)kHotDN ? col : 0u)];
        }
      }
    }
    __syncthreads();  // E before the next tile
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct RadixPlan {
  int passes;
  int bits;
};

// Digit plan for keys in [0, K).
static RadixPlan radix_plan(int64_t K) {
  int tb = 0;
  if (K > 1)
    while (tb < 31 && ((uint64_t)(K - 1) >> tb) != 0) ++tb;
  if (tb <= 8) return {1, 8};
  if (tb <= 16) return {2, 8};
  if (tb <= 20) return {2, 10};
  if (tb <= 22) return {2, 11};
  if (tb <= 30) return {3, 10};
  return {3, 11};
}

struct BwdLayout {
  size_t offs, keys0, vals0, keys1, vals1, hist, parts, partials, meta, dsorted, zrow, dummy_row, long_rows, tickets,
      invalid, seg_tab, bseg, seg_hist, hot_rows, hot_pc, hot_po, hot_ent, hot_lo, total;
  int64_t ntiles, nbins, nchunks, nmeta, nbuckets, max_segs;
  // hot rows: at least hot_min lookups; at most hr_max of them; nc chunks of 32 bags
  int64_t hot_min, hr_max, hot_nc;
  size_t hot_gt, hot_wh, hot_bcnt, hot_part;
  int64_t hot_part_rows;  // float32 partial rows of the gradient product's bag splits  // the gradient transposed [D][32 nc] and the hot rows' table rows [hr_max][D] (bf16)
  RadixPlan plan;
};

static BwdLayout bwd_layout(int64_t K, int64_t D, int64_t bags, int64_t L) {
  const int64_t N = bags * L;
  BwdLayout l;
  l.plan = radix_plan(K);
  size_t off = 0;
  l.offs = off;
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
  l.nbins = ((int64_t)1 << l.plan.bits) * l.ntiles;
  l.hist = off;
  off += align256((size_t)(l.nbins + 1) * 4);
  const int64_t scan_n = (K + 1) > l.nbins ? (K + 1) : l.nbins;
  l.parts = off;
  off += align256((size_t)(cdiv(scan_n, kScanTile) + 1) * 4);
  l.nchunks = cdiv(N, kHeavyT);
  l.partials = off;
  off += align256((size_t)(2 * l.nchunks) * (size_t)D * 4);
  // row kernels: sorted occurrence metadata (padded so a row's U slots can be
  // read past any row start), dots in sorted order (+1 dummy slot), a zero row
  // read by unused prefetch slots and a dummy row written by tail rows
  l.nmeta = N + kMetaPad;
  l.meta = off;
  off += align256((size_t)l.nmeta * 8);
  l.dsorted = off;
  off += align256((size_t)(N + 1) * 4);
  l.zrow = off;
  off += align256((size_t)D * 4);
  l.dummy_row = off;
  off += align256((size_t)D * 4);
  // long light rows (at most one entry per row) and their count; the row kernel's ticket counters
  l.long_rows = off;
  off += align256((size_t)(K + 1) * 4);
  l.tickets = off;
  off += (size_t)kDynGroups * kDynSub * kCtrStride * 4;
  // out-of-range lookups: count, then positions
  l.invalid = off;
  off += align256((size_t)(N + 1) * 4);
  // two-digit plans: the local pass's segment table, per-bucket segment ranges and per-segment digit counts
  l.nbuckets = l.max_segs = 0;
  l.seg_tab = l.bseg = l.seg_hist = off;
  if (l.plan.passes == 2) {
    l.nbuckets = cdiv(K, (int64_t)1 << l.plan.bits);
    l.max_segs = cdiv(N, kSegItems) + l.nbuckets;
    l.seg_tab = off;
    off += align256((size_t)(2 * l.max_segs + 1) * 4);
    l.bseg = off;
    off += align256((size_t)(3 * l.nbuckets) * 4);
    l.seg_hist = off;
    off += align256((size_t)l.max_segs * ((size_t)1 << l.plan.bits) * 4);
  }
  // two-digit plans: the hot rows' list (count and lo flag after it), chunk pointers and merged entries
  l.hot_min = bags / 16 > (int64_t)kHeavyT ? bags / 16 : (int64_t)kHeavyT + 1;
  l.hr_max = (l.plan.passes == 2 && N > 0) ? (N / l.hot_min < K ? N / l.hot_min : K) : 0;
  l.hot_nc = cdiv(bags, kHotKC);
  l.hot_rows = l.hot_pc = l.hot_po = l.hot_ent = l.hot_lo = l.hot_gt = l.hot_wh = l.hot_bcnt = l.hot_part = off;
  l.hot_part_rows = 0;
  if (l.hr_max > 0) {
    l.hot_rows = off;
    off += align256((size_t)(l.hr_max + 2) * 4);
    l.hot_pc = off;
    off += align256((size_t)l.hr_max * (size_t)(l.hot_nc + 1) * 4);
    l.hot_po = off;
    off += align256((size_t)l.hr_max * (size_t)(l.hot_nc + 1) * 4);
    l.hot_ent = off;
    off += align256((size_t)N * 4);
    l.hot_lo = off;
    off += align256((size_t)N * 2);
    l.hot_gt = off;
    off += align256((size_t)D * (size_t)(l.hot_nc * kHotKC) * 2);
    l.hot_wh = off;
    off += align256((size_t)l.hr_max * (size_t)D * 2);
    l.hot_bcnt = off;
    off += align256((size_t)l.nbuckets * 4);
    // up to 4 splits of every hot row, at most 128 MiB
    const int64_t cap = ((int64_t)128 << 20) / (D * 4);
    l.hot_part_rows = 4 * cdiv(l.hr_max, kHotM) * kHotM < cap ? 4 * cdiv(l.hr_max, kHotM) * kHotM : cap;
    l.hot_part = off;
    off += align256((size_t)l.hot_part_rows * (size_t)D * 4);
  }
  l.total = off;
  return l;
}

// In-place exclusive prefix sum of data[0..n) with data[n] <- total.
static void device_exclusive_sum(uint32_t* data, int64_t n, uint32_t* parts, hipStream_t st) {
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

template <int BITS>
static void radix_pass(int pass, const int64_t* idx, uint32_t* const keys[2], uint32_t* const vals[2], int cur,
                       int nxt, int64_t N, int64_t K, const BwdLayout& l, uint32_t* hist, uint32_t* parts,
                       uint32_t* invalid, hipStream_t st) {
  const int shift = pass * BITS;
  const uint32_t* nvalid = hist + l.nbins;  // total of the previous pass's scan
  const dim3 grid((unsigned)l.ntiles), block(256);
  if (pass == 0) {
    hipLaunchKernelGGL((radix_hist_kernel<true, BITS>), grid, block, 0, st, idx, (const uint32_t*)nullptr, N,
                       (const uint32_t*)nullptr, K, shift, hist, l.ntiles, invalid);
    device_exclusive_sum(hist, l.nbins, parts, st);
    hipLaunchKernelGGL((radix_scatter_kernel<true, BITS>), grid, block, 0, st, idx, (const uint32_t*)nullptr,
                       (const uint32_t*)nullptr, N, (const uint32_t*)nullptr, K, shift, (const uint32_t*)hist,
                       l.ntiles, keys[nxt], vals[nxt]);
  } else {
    // the previous scan's total (nvalid) lives at hist[nbins]; this pass's hist
    // kernel reads it before the scan below rewrites it with the same value
    hipLaunchKernelGGL((radix_hist_kernel<false, BITS>), grid, block, 0, st, (const int64_t*)nullptr,
                       (const uint32_t*)keys[cur], N, nvalid, K, shift, hist, l.ntiles, (uint32_t*)nullptr);
    device_exclusive_sum(hist, l.nbins, parts, st);
    hipLaunchKernelGGL((radix_scatter_kernel<false, BITS>), grid, block, 0, st, (const int64_t*)nullptr,
                       (const uint32_t*)keys[cur], (const uint32_t*)vals[cur], N, nvalid, K, shift,
                       (const uint32_t*)hist, l.ntiles, keys[nxt], vals[nxt]);
  }
}

// Two-digit plans: a stable bucketing pass by the high digit (out-of-range
// lookups dropped and listed), then the local pass per bucket (row offsets
// and, with meta, the occurrence metadata included). Output in keys[1] /
// vals[1], as the two single-digit passes leave it.
template <int BITS>
static void two_level_sort(const int64_t* idx, uint32_t* const keys[2], uint32_t* const vals[2], int64_t N, int64_t K,
                           const BwdLayout& l, char* ws, uint32_t* hist, uint32_t* parts, uint32_t* invalid,
                           uint32_t* offs, uint2* meta, const void* psw, int pdt, int64_t L, uint32_t long_min,
                           uint32_t* long_rows, uint32_t* hot_rows, hipStream_t st) {
  const uint32_t* nvalid = hist + l.nbins;  // the first pass's scan total
  const dim3 grid((unsigned)l.ntiles), block(256);
  hipLaunchKernelGGL((radix_hist_kernel<true, BITS>), grid, block, 0, st, idx, (const uint32_t*)nullptr, N,
                     (const uint32_t*)nullptr, K, BITS, hist, l.ntiles, invalid);
  device_exclusive_sum(hist, l.nbins, parts, st);
  hipLaunchKernelGGL((radix_scatter_kernel<true, BITS>), grid, block, 0, st, idx, (const uint32_t*)nullptr,
                     (const uint32_t*)nullptr, N, (const uint32_t*)nullptr, K, BITS, (const uint32_t*)hist, l.ntiles,
                     keys[0], vals[0], SegTab{}, (uint2*)nullptr, (const void*)nullptr, 0, 1u);
  uint32_t* tab = (uint32_t*)(ws + l.seg_tab);
  uint32_t* bseg = (uint32_t*)(ws + l.bseg);
  uint32_t* shist = (uint32_t*)(ws + l.seg_hist);
  const SegTab seg{tab, l.max_segs};
  hipLaunchKernelGGL(seg_plan_kernel, dim3(1), dim3(256), 0, st, (const uint32_t*)hist, l.ntiles, (int)l.nbuckets,
                     1 << BITS, nvalid, tab, l.max_segs, bseg, K, offs, meta, l.nmeta);
  hipLaunchKernelGGL((seg_hist_kernel<BITS>), dim3((unsigned)l.max_segs), dim3(256), 0, st, (const uint32_t*)keys[0],
                     seg, shist);
  hipLaunchKernelGGL((seg_base_kernel<BITS>), dim3((unsigned)l.nbuckets), dim3(256), 0, st, (const uint32_t*)bseg, K,
                     shist, offs, long_min, long_rows, long_rows != nullptr ? long_rows + K : (uint32_t*)nullptr,
                     (uint32_t)l.hot_min, hot_rows != nullptr ? (uint32_t*)(ws + l.hot_bcnt) : (uint32_t*)nullptr);
  if (hot_rows != nullptr)
    hipLaunchKernelGGL((hot_order_kernel<BITS>), dim3((unsigned)l.nbuckets), dim3(256), 0, st,
                       (const uint32_t*)(ws + l.hot_bcnt), l.nbuckets, (const uint32_t*)offs, K, (uint32_t)l.hot_min,
                       hot_rows, l.hr_max);
  hipLaunchKernelGGL((radix_scatter_kernel<false, BITS, true>), dim3((unsigned)l.max_segs), block, 0, st,
                     (const int64_t*)nullptr, (const uint32_t*)keys[0], (const uint32_t*)vals[0], N, nvalid, K, 0,
                     (const uint32_t*)shist, (int64_t)0, keys[1], vals[1], seg, meta, psw, pdt, (uint32_t)L);
}

// Row-kernel prefetch depth (lookups per row reduced in the row kernel) for
// rows of 64 * VPL vectors: 8 when the lookups average more than ~3 per row.
static int rows_prefetch_of(int vpl, int64_t N, int64_t K) {
  if (vpl <= 2) return N > 3 * K ? 8 : 4;
  return vpl == 4 ? 2 : 1;
}
template <int VPL>
static int rows_prefetch(int64_t N, int64_t K) {
  return rows_prefetch_of(VPL, N, K);
}

// Whether the hot rows go to the matrix cores (for a bf16 table of 64-lane
// rows, the lookups sorted by the two-level sort): rows of whole 256-column
// tiles, and room for at least one hot row.
static bool hot_rows_enabled(const BwdLayout& l, int64_t D) { return l.hr_max > 0 && D % kHotN == 0; }

static unsigned hot_grid(int64_t tiles) {
  const int64_t g = tiles < 1024 ? tiles : 1024;
  return (unsigned)((g + 7) / 8 * 8);  // a multiple of 8: each workgroup stays on one XCD's tiles
}

// Prepare the row kernel's list: the light rows longer than 2 U (the row
// kernel reduces up to 2 U in place).
// (long_rows[K], the count, was zeroed by prep_fill_kernel.)
static void prepare_rows_dyn(int64_t K, int U, const uint32_t* offs, uint32_t* long_rows, hipStream_t st) {
  uint32_t* long_count = long_rows + K;
  const int64_t lwg = cdiv(K, 1024) < 256 ? cdiv(K, 1024) : 256;
  hipLaunchKernelGGL(list_long_rows_kernel, dim3((unsigned)lwg), dim3(256), 0, st, offs, K, (uint32_t)(2 * U),
                     cdiv(cdiv(K, lwg), 256) * 256, long_rows, long_count);
}

// The row reduction on the ticket schedule: the rows kernel, then the long
// rows listed by prepare_rows_dyn. Each reduction clears its own ticket
// counters first, so a prepared workspace can serve any number of reductions.
template <typename TW, typename TG, int VPL, int U, bool SGD, bool ACC>
static void launch_rows_dyn(const void* W, int64_t K, int64_t D, int want_dot, const void* g, const uint32_t* offs,
                            const uint2* meta, const float* partials, const void* zrow, void* dummy_row, void* gW,
                            float* dsorted, uint32_t dummy_slot, uint32_t* long_rows, uint32_t* tickets,
                            uint32_t long_min, uint32_t hot_min, const SgdArgs& S, hipStream_t st) {
  const uint32_t* long_count = long_rows + K;
  hipLaunchKernelGGL(fill_u32_kernel, dim3(4), dim3(256), 0, st, tickets, 0u,
                     (int64_t)kDynGroups * kDynSub * kCtrStride);
  // blocks of 1024 rows (the sub-key blocks of a 1024-key half) once every
  // group gets several; smaller tables use the smallest block
  const uint32_t blk = K >= (int64_t)kDynGroups * 8 * 1024 ? 1024u : (uint32_t)(kDynRC * kDynSub);
  int64_t wgs = cdiv(K, 64);
  wgs = wgs < 1280 ? wgs : 1280;
  wgs = cdiv(wgs, kDynGroups * kDynSub) * kDynGroups * kDynSub;  // every counter gets workgroups
  KernelSpan span("eb_bwd_rows", st);
  hipLaunchKernelGGL((eb_bwd_rows_dyn_kernel<TW, TG, VPL, U, SGD, ACC>), dim3((unsigned)wgs), dim3(256), 0, st, (const TW*)W,
                     K, D, want_dot, (const TG*)g, offs, meta, partials, (const TW*)zrow, (TW*)dummy_row, (TW*)gW,
                     dsorted, dummy_slot, tickets, blk, long_min, hot_min, S);
  const int64_t rb = cdiv(K, 4 * 64);
  const unsigned lb = (unsigned)(rb < 1024 ? rb : 1024);
  hipLaunchKernelGGL((eb_bwd_long_rows_kernel<TW, TG, VPL, U, SGD, ACC>), dim3(lb), dim3(256), 0, st, (const TW*)W, D,
                     want_dot, (const TG*)g, offs, meta, (const TW*)zrow, (TW*)gW, dsorted, dummy_slot,
                     (const uint32_t*)long_rows, long_count, S);
}

// Everything of the backward that depends only on the lookups (run by
// pkm_eb_bwd_prepare): for 64-lane rows, the occurrence metadata, the zero
// row and the row kernel's lists.
template <typename TW, int LPG, int VPL>
static void launch_prepare(int64_t K, int64_t D, const void* psw, int pdt, int64_t L, const uint32_t* offs,
                           const uint32_t* svals, const uint32_t* nvalid, int64_t N, const BwdLayout& l, char* ws,
                           bool hot, hipStream_t st) {
  if constexpr (LPG == 64) {
    uint2* meta = (uint2*)(ws + l.meta);
    // (the zero row was filled by prep_fill_kernel)
    if (N > 0 && l.plan.passes == 2) {
      // written by the sort's local pass
    } else if (N > 0)
      hipLaunchKernelGGL(occ_meta_kernel, dim3(grid_for(l.nmeta, 256, 16384)), dim3(256), 0, st, svals, nvalid,
                         l.nmeta, (uint32_t)L, psw, pdt, meta);
    else
      hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(2 * l.nmeta, 256, 4096)), dim3(256), 0, st,
                         (uint32_t*)meta, 0u, 2 * l.nmeta);
    if (K > 0 && !(N > 0 && l.plan.passes == 2))  // (the two-level sort lists the long rows itself)
      prepare_rows_dyn(K, rows_prefetch<VPL>(N, K), offs, (uint32_t*)(ws + l.long_rows), st);
    if constexpr (std::is_same<TW, bf16_t>::value) {
      if (hot && hot_rows_enabled(l, D)) {
        // the hot rows the sort listed: merged entries and chunk pointers
        const uint32_t* hot_list = (const uint32_t*)(ws + l.hot_rows);
        const unsigned gb = (unsigned)(l.hr_max < 8192 ? l.hr_max : 8192);  // a block per row, up to 8192
        hipLaunchKernelGGL(hot_list_kernel, dim3(gb), dim3(256), 0, st, hot_list, l.hr_max, offs,
                           (const uint2*)(ws + l.meta), (uint32_t)l.hot_nc, (uint32_t*)(ws + l.hot_pc),
                           (uint32_t*)(ws + l.hot_po), (uint32_t*)(ws + l.hot_ent), (uint16_t*)(ws + l.hot_lo),
                           (uint32_t*)(ws + l.hot_rows) + l.hr_max + 1);
      }
    }
  }
}

template <typename TW, typename TG, int LPG, int VPL, bool SGD, bool ACC = false>
static void launch_reduce(const void* W, int64_t K, int64_t D, const void* psw, int pdt, const void* g, int64_t L,
                          const uint32_t* offs, const uint32_t* skeys, const uint32_t* svals, const uint32_t* nvalid,
                          int64_t N, const BwdLayout& l, char* ws, void* gW, void* gpsw, const SgdArgs& S,
                          hipStream_t st) {
  constexpr int GPW = 64 / LPG;
  const int64_t groups_per_block = 4 * GPW;
  float* partials = (float*)(ws + l.partials);
  const unsigned hb = (unsigned)cdiv(l.nchunks, groups_per_block);
  if constexpr (LPG == 64) {
    const uint2* meta = (const uint2*)(ws + l.meta);
    float* dsorted = (float*)(ws + l.dsorted);
    void* zrow = ws + l.zrow;
    // hot rows on the matrix cores (bf16 table and gradient; not in the SGD epilogue)
    constexpr bool kHotTypes = std::is_same<TW, bf16_t>::value && std::is_same<TG, bf16_t>::value && !SGD;
    const bool hot = kHotTypes && N > 0 && hot_rows_enabled(l, D);
    const uint32_t hot_min = hot ? (uint32_t)l.hot_min : 0xFFFFFFFFu;
    if constexpr (kHotTypes) {
      if (hot) {
        KernelSpan span("eb_bwd_hot", st);
        const uint32_t* hot_list = (const uint32_t*)(ws + l.hot_rows);
        const int64_t bags = N / L;
        uint16_t* Gt = (uint16_t*)(ws + l.hot_gt);
        uint16_t* Wh = gpsw != nullptr ? (uint16_t*)(ws + l.hot_wh) : nullptr;
        hipLaunchKernelGGL(hot_operands_kernel, dim3(grid_for(l.hot_nc * (D / 64), 1, 2048)), dim3(256), 0, st,
                           hot_list, l.hr_max, (const bf16_t*)g, bags, (uint32_t)l.hot_nc, D, Gt, (const bf16_t*)W,
                           Wh);
        const int64_t tiles = cdiv(l.hr_max, kHotM) * (D / kHotN);
        float* part = (float*)(ws + l.hot_part);
        hipLaunchKernelGGL((hot_grad_kernel<ACC>), dim3(hot_grid(tiles > (int64_t)kHotTiles ? tiles : kHotTiles)),
                           dim3(kHotGradThreads), 0, st, hot_list, l.hr_max, (const uint32_t*)(ws + l.hot_pc),
                           (uint32_t)l.hot_nc, (const uint32_t*)(ws + l.hot_ent), (const uint16_t*)(ws + l.hot_lo),
                           (const uint16_t*)Gt, D, (bf16_t*)gW, part, l.hot_part_rows);
        hipLaunchKernelGGL((hot_finish_kernel<ACC>), dim3(grid_for(l.hr_max * (D / 4), 256, 4096)), dim3(256), 0, st,
                           hot_list, l.hr_max, (uint32_t)l.hot_nc, D, (const float*)part, l.hot_part_rows,
                           (bf16_t*)gW);
        if (gpsw != nullptr)
          hipLaunchKernelGGL(hot_dot_kernel, dim3(hot_grid(cdiv(l.hr_max, kHotDM) * cdiv(bags, kHotDN))),
                             dim3(kHotThreads), 0, st, hot_list, l.hr_max, (const uint32_t*)(ws + l.hot_po),
                             (uint32_t)l.hot_nc, meta, (const uint16_t*)Wh, (const bf16_t*)g, bags, D, dsorted);
      }
    }
    if (N > 0)
      hipLaunchKernelGGL((eb_bwd_heavy_kernel<TW, TG, LPG, VPL>), dim3(hb), dim3(256), 0, st, (const TW*)W, K, D,
                         psw, pdt, (const TG*)g, (uint32_t)L, offs, skeys, svals, nvalid, l.nchunks, partials, gpsw,
                         dsorted, hot_min);
    if (K > 0) {
      const int want_dot = gpsw != nullptr ? 1 : 0;
      // the prefetch depth the lists were prepared for (rows longer than twice it go to the
      // long-row kernel), halved when each gradient row is twice the table row's bytes
      const int u0 = rows_prefetch<VPL>(N, K);
      const uint32_t long_min = (uint32_t)(2 * u0);
      constexpr int NV = GradTraits<TW, TG>::NV;
      const uint32_t dslot = (uint32_t)N;
      void* dummy = ws + l.dummy_row;
      uint32_t* long_rows = (uint32_t*)(ws + l.long_rows);
      uint32_t* tickets = (uint32_t*)(ws + l.tickets);
#define PKM_ROWS(U_) \
  launch_rows_dyn<TW, TG, VPL, U_, SGD, ACC>(W, K, D, want_dot, g, offs, meta, partials, zrow, dummy, gW, dsorted, dslot, long_rows, tickets, long_min, hot_min, S, st)
      if constexpr (VPL <= 2 && NV == 1) {
        if (u0 == 8) PKM_ROWS(8); else PKM_ROWS(4);
      } else if constexpr (VPL <= 2) {
        if (u0 == 8) PKM_ROWS(4); else PKM_ROWS(2);
      } else if constexpr (VPL == 4 && NV == 1) {
        PKM_ROWS(2);
      } else {
        PKM_ROWS(1);
      }
#undef PKM_ROWS
    }
    if (N > 0 && gpsw != nullptr)
      hipLaunchKernelGGL(gpsw_scatter_kernel, dim3(grid_for(N, 256, 16384)), dim3(256), 0, st, svals,
                         (const float*)dsorted, nvalid, N, gpsw, pdt, (const uint32_t*)(ws + l.invalid));
  } else {
    static_assert(!ACC, "the accumulating reduction runs on 64-lane rows");
    if (N > 0)
      hipLaunchKernelGGL((eb_bwd_heavy_kernel<TW, TG, LPG, VPL>), dim3(hb), dim3(256), 0, st, (const TW*)W, K, D,
                         psw, pdt, (const TG*)g, (uint32_t)L, offs, skeys, svals, nvalid, l.nchunks, partials, gpsw,
                         (float*)nullptr, 0xFFFFFFFFu);
    if (K == 0) return;
    const int rows_per_group = 4;
    const int64_t groups = cdiv(K, rows_per_group);
    const unsigned rb = (unsigned)cdiv(groups, groups_per_block);
    KernelSpan span("eb_bwd_rows", st);
    hipLaunchKernelGGL((eb_bwd_rows_kernel<TW, TG, LPG, VPL, SGD>), dim3(rb), dim3(256), 0, st, (const TW*)W, K, D,
                       psw, pdt, (const TG*)g, (uint32_t)L, offs, svals, (const float*)partials, rows_per_group, (TW*)gW,
                       gpsw, S);
  }
}

// sgd != NULL: the reduction ends in the fast-weight SGD epilogue (SgdArgs)
// instead of writing the table gradient; instantiated where TG is TW.
template <typename TW, typename TG = TW>
static bool dispatch_reduce(bool prepare, const GroupCfg& c, const void* W, int64_t K, int64_t D, const void* psw, int pdt,
                            const void* g, int64_t L, const uint32_t* offs, const uint32_t* skeys,
                            const uint32_t* svals, const uint32_t* nvalid, int64_t N, const BwdLayout& l,
                            char* ws, void* gW, void* gpsw, hipStream_t st, const SgdArgs* sgd = nullptr,
                            bool acc = false, bool hot = true) {
  static const SgdArgs no_sgd = {};
#define PKM_RED_CASE(LPG_, VPL_)                                                                                  \
  if (c.lpg == LPG_ && c.vpl == VPL_) {                                                                           \
    if (prepare) {                                                                                                \
      launch_prepare<TW, LPG_, VPL_>(K, D, psw, pdt, L, offs, svals, nvalid, N, l, ws, hot, st);                  \
    } else if (sgd == nullptr && acc) {                                                                         \
      if constexpr (LPG_ == 64 && std::is_same<TW, TG>::value)                                                    \
        launch_reduce<TW, TG, LPG_, VPL_, false, true>(W, K, D, psw, pdt, g, L, offs, skeys, svals, nvalid, N, l, \
                                                       ws, gW, gpsw, no_sgd, st);                                 \
      else                                                                                                        \
        return false;                                                                                             \
    } else if (sgd == nullptr) {                                                                                  \
      launch_reduce<TW, TG, LPG_, VPL_, false>(W, K, D, psw, pdt, g, L, offs, skeys, svals, nvalid, N, l, ws, gW, \
                                               gpsw, no_sgd, st);                                                 \
    } else {                                                                                                      \
      if constexpr (std::is_same<TW, TG>::value && !std::is_same<TW, f16_t>::value)                               \
        launch_reduce<TW, TG, LPG_, VPL_, true>(W, K, D, psw, pdt, g, L, offs, skeys, svals, nvalid, N, l, ws,    \
                                                gW, gpsw, *sgd, st);                                              \
      else                                                                                                        \
        return false;                                                                                             \
    }                                                                                                             \
    return true;                                                                                                  \
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
  return bwd_layout(num_rows, dim, bags, bag_size).total;
}

namespace pkm {

// Checks shared by the backward's entry points; fills the kernel group
// configuration and the workspace layout.
static int eb_bwd_check(const char* fn, int64_t num_rows, int64_t dim, int weight_dtype, const int64_t* indices,
                        const void* psw, int psw_dtype, int64_t bags, int64_t bag_size, void* workspace,
                        size_t workspace_bytes, GroupCfg* c, BwdLayout* l) {
  PKM_REQUIRE(valid_dt(weight_dtype), PKM_ERR_INVALID_ARGUMENT, "%s: bad weight dtype %d", fn, weight_dtype);
  PKM_REQUIRE(psw_dtype == PKM_DTYPE_NONE ? psw == nullptr
                                          : (valid_dt(psw_dtype) && (psw != nullptr || bags * bag_size == 0)),
              PKM_ERR_INVALID_ARGUMENT, "%s: psw pointer / dtype %d mismatch", fn, psw_dtype);
  PKM_REQUIRE(num_rows >= 0 && dim > 0 && bags >= 0 && bag_size >= 0, PKM_ERR_INVALID_ARGUMENT,
              "%s: bad sizes num_rows=%lld dim=%lld bags=%lld bag_size=%lld", fn, (long long)num_rows,
              (long long)dim, (long long)bags, (long long)bag_size);
  const int64_t N = bags * bag_size;
  PKM_REQUIRE(N < ((int64_t)1 << 31) && num_rows < ((int64_t)1 << 31) - 1, PKM_ERR_INVALID_ARGUMENT,
              "%s: bags*bag_size=%lld must be < 2^31 and num_rows=%lld < 2^31-1", fn, (long long)N,
              (long long)num_rows);
  PKM_REQUIRE(N == 0 || indices != nullptr, PKM_ERR_INVALID_ARGUMENT, "%s: null indices", fn);
  const int epv = weight_dtype == PKM_DTYPE_F32 ? 4 : 8;
  PKM_REQUIRE(choose_group_cfg(dim, epv, true, c), PKM_ERR_UNSUPPORTED,
              "%s: dim %lld not supported (need dim/%d = LPG*VPL with LPG<=64, VPL<=8)", fn, (long long)dim, epv);
  *l = bwd_layout(num_rows, dim, bags, bag_size);
  PKM_REQUIRE(workspace != nullptr && workspace_bytes >= l->total, PKM_ERR_WORKSPACE,
              "%s: workspace of %zu bytes given, %zu needed", fn, workspace_bytes, l->total);
  PKM_REQUIRE((uintptr_t)workspace % 256 == 0, PKM_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned",
              fn);
  return PKM_OK;
}

// Buffers of the sorted lookups: the final ping-pong buffer of the sort
// (pass p writes buffer 0 for p = 0 and alternates after).
struct SortedView {
  uint32_t *offs, *keys, *vals, *hist, *parts, *invalid;
  const uint32_t* nvalid;
};
static SortedView sorted_view(const BwdLayout& l, char* ws) {
  SortedView v;
  v.offs = (uint32_t*)(ws + l.offs);
  const int cur = l.plan.passes % 2 == 1 ? 0 : 1;
  v.keys = (uint32_t*)(ws + (cur == 0 ? l.keys0 : l.keys1));
  v.vals = (uint32_t*)(ws + (cur == 0 ? l.vals0 : l.vals1));
  v.hist = (uint32_t*)(ws + l.hist);
  v.parts = (uint32_t*)(ws + l.parts);
  v.invalid = (uint32_t*)(ws + l.invalid);
  v.nvalid = v.hist + l.nbins;
  return v;
}

}  // namespace pkm

namespace pkm {
// pkm_eb_bwd_prepare; hot: also list the hot rows for the matrix-core
// products (the reductions other than the SGD epilogue use them).
static int eb_bwd_prepare(int64_t num_rows, int64_t dim, int weight_dtype, const int64_t* indices, const void* psw,
                          int psw_dtype, int64_t bags, int64_t bag_size, void* workspace, size_t workspace_bytes,
                          bool hot, void* stream) {
  GroupCfg c;
  BwdLayout l;
  const int rc = eb_bwd_check("pkm_eb_bwd_prepare", num_rows, dim, weight_dtype, indices, psw, psw_dtype, bags,
                              bag_size, workspace, workspace_bytes, &c, &l);
  if (rc != PKM_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int64_t K = num_rows, N = bags * bag_size;
  const SortedView v = sorted_view(l, ws);
  hot = hot && c.lpg == 64 && weight_dtype == PKM_DTYPE_BF16 && hot_rows_enabled(l, dim);
  // zeroed state: the out-of-range count, and for the 64-lane row kernels the long-row count, the hot-row
  // state and the zero row
  {
    const bool rows64 = c.lpg == 64;
    hipLaunchKernelGGL(prep_fill_kernel, dim3(rows64 ? grid_for(dim, 256, 64) : 1), dim3(256), 0, st, v.invalid,
                       rows64 && K > 0 ? (uint32_t*)(ws + l.long_rows) + K : (uint32_t*)nullptr,
                       hot ? (uint32_t*)(ws + l.hot_rows) + l.hr_max : (uint32_t*)nullptr,
                       rows64 ? (uint32_t*)(ws + l.zrow) : (uint32_t*)nullptr, rows64 ? dim : (int64_t)0);
  }
  uint2* meta = c.lpg == 64 ? (uint2*)(ws + l.meta) : nullptr;  // read by the 64-lane row kernels
  if (N > 0 && l.plan.passes == 2) {
    // 1-2. stable sort of (row, position) by bucketing and local passes, with the row offsets, the metadata and
    // the 64-lane row kernel's long-row list
    uint32_t* keys[2] = {(uint32_t*)(ws + l.keys0), (uint32_t*)(ws + l.keys1)};
    uint32_t* vals[2] = {(uint32_t*)(ws + l.vals0), (uint32_t*)(ws + l.vals1)};
    uint32_t* long_rows = c.lpg == 64 ? (uint32_t*)(ws + l.long_rows) : nullptr;
    uint32_t* hot_rows = hot ? (uint32_t*)(ws + l.hot_rows) : nullptr;
    const uint32_t long_min = (uint32_t)(2 * rows_prefetch_of(c.vpl, N, K));
#define PKM_TWO_LEVEL(B_)                                                                                      \
  two_level_sort<B_>(indices, keys, vals, N, K, l, ws, v.hist, v.parts, v.invalid, v.offs, meta, psw, psw_dtype, \
                     bag_size, long_min, long_rows, hot_rows, st)
    switch (l.plan.bits) {
      case 8:
        PKM_TWO_LEVEL(8);
        break;
      case 10:
        PKM_TWO_LEVEL(10);
        break;
      default:
        PKM_TWO_LEVEL(11);
        break;
    }
#undef PKM_TWO_LEVEL
  } else if (N > 0) {
    // 1. stable LSD radix sort of (row, position); out-of-range lookups dropped and listed
    uint32_t* keys[2] = {(uint32_t*)(ws + l.keys0), (uint32_t*)(ws + l.keys1)};
    uint32_t* vals[2] = {(uint32_t*)(ws + l.vals0), (uint32_t*)(ws + l.vals1)};
    int cur = 0;
    for (int pass = 0; pass < l.plan.passes; ++pass) {
      const int nxt = pass == 0 ? 0 : 1 - cur;
      switch (l.plan.bits) {
        case 8:
          radix_pass<8>(pass, indices, keys, vals, cur, nxt, N, K, l, v.hist, v.parts, v.invalid, st);
          break;
        case 10:
          radix_pass<10>(pass, indices, keys, vals, cur, nxt, N, K, l, v.hist, v.parts, v.invalid, st);
          break;
        default:
          radix_pass<11>(pass, indices, keys, vals, cur, nxt, N, K, l, v.hist, v.parts, v.invalid, st);
          break;
      }
      cur = nxt;
    }
    // 2. row offsets: a binary search of the sorted keys per row
    hipLaunchKernelGGL(row_offsets_kernel, dim3(grid_for(K + 1, 256, 65536)), dim3(256), 0, st,
                       (const uint32_t*)v.keys, v.nvalid, K, v.offs);
  } else {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(K + 1, 256, 4096)), dim3(256), 0, st, v.offs, 0u, K + 1);
  }
  // 3. metadata and the row kernel's lists
  bool ok;
  if (weight_dtype == PKM_DTYPE_F32)
    ok = dispatch_reduce<float>(true, c, nullptr, K, dim, psw, psw_dtype, nullptr, bag_size, v.offs, v.keys, v.vals,
                                v.nvalid, N, l, ws, nullptr, nullptr, st);
  else if (weight_dtype == PKM_DTYPE_BF16)
    ok = dispatch_reduce<bf16_t>(true, c, nullptr, K, dim, psw, psw_dtype, nullptr, bag_size, v.offs, v.keys, v.vals,
                                 v.nvalid, N, l, ws, nullptr, nullptr, st, nullptr, false, hot);
  else
    ok = dispatch_reduce<f16_t>(true, c, nullptr, K, dim, psw, psw_dtype, nullptr, bag_size, v.offs, v.keys, v.vals,
                                v.nvalid, N, l, ws, nullptr, nullptr, st);
  PKM_REQUIRE(ok, PKM_ERR_UNSUPPORTED, "pkm_eb_bwd_prepare: no kernel for lpg=%d vpl=%d", c.lpg, c.vpl);
  return pkm_check_launch("pkm_eb_bwd_prepare");
}
}  // namespace pkm

extern "C" int pkm_eb_bwd_prepare(int64_t num_rows, int64_t dim, int weight_dtype, const int64_t* indices,
                                  const void* psw, int psw_dtype, int64_t bags, int64_t bag_size, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return eb_bwd_prepare(num_rows, dim, weight_dtype, indices, psw, psw_dtype, bags, bag_size, workspace,
                        workspace_bytes, true, stream);
}

namespace pkm {
// The reduction on a prepared workspace; acc: grad_weight holds a gradient
// that the rows' sums are added to (rows without lookups keep it).
static int eb_bwd_reduce(const char* fn, bool acc, const void* weight, int64_t num_rows, int64_t dim,
                         int weight_dtype, const int64_t* indices, const void* psw, int psw_dtype,
                         const void* grad_out, int grad_dtype, int64_t bags, int64_t bag_size, void* grad_weight,
                         void* grad_psw, void* workspace, size_t workspace_bytes, void* stream) {
  GroupCfg c;
  BwdLayout l;
  const int rc = eb_bwd_check(fn, num_rows, dim, weight_dtype, indices, psw, psw_dtype, bags, bag_size, workspace,
                              workspace_bytes, &c, &l);
  if (rc != PKM_OK) return rc;
  const int64_t N = bags * bag_size;
  const bool wide_grad = grad_dtype == PKM_DTYPE_F32 && weight_dtype != PKM_DTYPE_F32;
  PKM_REQUIRE(grad_dtype == weight_dtype || wide_grad, PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd: grad_out dtype %d with weight dtype %d (supported: the same dtype, or a float32 "
              "grad_out for a 16-bit table)", grad_dtype, weight_dtype);
  PKM_REQUIRE(grad_weight != nullptr || num_rows == 0, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: null grad_weight");
  PKM_REQUIRE(N == 0 || grad_out != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: null grad_out");
  PKM_REQUIRE(psw == nullptr || N == 0 || (grad_psw != nullptr && (weight != nullptr || num_rows == 0)),
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: null weight / grad_psw");
  PKM_REQUIRE((uintptr_t)weight % 16 == 0 && (uintptr_t)grad_out % 16 == 0 && (uintptr_t)grad_weight % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd: weight, grad_out, grad_weight must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const SortedView v = sorted_view(l, ws);
  void* gpsw = psw != nullptr ? grad_psw : nullptr;
  const int64_t K = num_rows;
  // 4-5. heavy-row chunk partials, then every row once, then the psw-gradients to their positions
  bool ok;
#define PKM_REDUCE(TW_, TG_)                                                                                    \
  dispatch_reduce<TW_, TG_>(false, c, weight, K, dim, psw, psw_dtype, grad_out, bag_size, v.offs, v.keys, v.vals, \
                            v.nvalid, N, l, ws, grad_weight, gpsw, st, nullptr, acc)
  if (weight_dtype == PKM_DTYPE_F32)
    ok = PKM_REDUCE(float, float);
  else if (weight_dtype == PKM_DTYPE_BF16)
    ok = wide_grad ? PKM_REDUCE(bf16_t, float) : PKM_REDUCE(bf16_t, bf16_t);
  else
    ok = wide_grad ? PKM_REDUCE(f16_t, float) : PKM_REDUCE(f16_t, f16_t);
#undef PKM_REDUCE
  PKM_REQUIRE(ok, PKM_ERR_UNSUPPORTED, "%s: no kernel for lpg=%d vpl=%d%s", fn, c.lpg, c.vpl,
              acc ? " (accumulating: 64-lane rows, gradient in the table's dtype)" : "");
  if (N > 0 && gpsw != nullptr && c.lpg != 64)  // (64-lane rows: inside gpsw_scatter_kernel)
    hipLaunchKernelGGL(zero_invalid_gpsw_kernel, dim3(64), dim3(256), 0, st, (const uint32_t*)v.invalid, gpsw,
                       psw_dtype);
  return pkm_check_launch(fn);
}

// Whether the accumulating reduction has a kernel for these sizes and dtypes.
static bool eb_bwd_acc_supported(int64_t dim, int weight_dtype, int grad_dtype) {
  GroupCfg c;
  const int epv = weight_dtype == PKM_DTYPE_F32 ? 4 : 8;
  return grad_dtype == weight_dtype && valid_dt(weight_dtype) && choose_group_cfg(dim, epv, true, &c) && c.lpg == 64;
}
}  // namespace pkm

extern "C" int pkm_eb_bwd_prepared(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                                   const int64_t* indices, const void* psw, int psw_dtype, const void* grad_out,
                                   int grad_dtype, int64_t bags, int64_t bag_size, void* grad_weight, void* grad_psw,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  return eb_bwd_reduce("pkm_eb_bwd_prepared", false, weight, num_rows, dim, weight_dtype, indices, psw, psw_dtype,
                       grad_out, grad_dtype, bags, bag_size, grad_weight, grad_psw, workspace, workspace_bytes,
                       stream);
}

extern "C" int pkm_eb_bwd_accumulate(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                                     const int64_t* indices, const void* psw, int psw_dtype, const void* grad_out,
                                     int grad_dtype, int64_t bags, int64_t bag_size, void* grad_weight,
                                     void* grad_psw, void* workspace, size_t workspace_bytes, void* stream) {
  PKM_REQUIRE(eb_bwd_acc_supported(dim, weight_dtype, grad_dtype), PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd_accumulate: dim %lld, weight dtype %d, grad dtype %d not supported (grad_out in the "
              "table's dtype, rows of 64 16-byte vectors or more)",
              (long long)dim, weight_dtype, grad_dtype);
  const int rc = pkm_eb_bwd_prepare(num_rows, dim, weight_dtype, indices, psw, psw_dtype, bags, bag_size, workspace,
                                    workspace_bytes, stream);
  if (rc != PKM_OK) return rc;
  return eb_bwd_reduce("pkm_eb_bwd_accumulate", true, weight, num_rows, dim, weight_dtype, indices, psw, psw_dtype,
                       grad_out, grad_dtype, bags, bag_size, grad_weight, grad_psw, workspace, workspace_bytes,
                       stream);
}

extern "C" int pkm_eb_bwd(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype, const int64_t* indices,
                          const void* psw, int psw_dtype, const void* grad_out, int grad_dtype, int64_t bags,
                          int64_t bag_size, void* grad_weight, void* grad_psw, void* workspace,
                          size_t workspace_bytes, void* stream) {
  PKM_REQUIRE(grad_dtype == weight_dtype || (grad_dtype == PKM_DTYPE_F32 && valid_dt(weight_dtype)),
              PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd: grad_out dtype %d with weight dtype %d (supported: the same dtype, or a float32 "
              "grad_out for a 16-bit table)", grad_dtype, weight_dtype);
  const int rc = pkm_eb_bwd_prepare(num_rows, dim, weight_dtype, indices, psw, psw_dtype, bags, bag_size, workspace,
                                    workspace_bytes, stream);
  if (rc != PKM_OK) return rc;
  return pkm_eb_bwd_prepared(weight, num_rows, dim, weight_dtype, indices, psw, psw_dtype, grad_out, grad_dtype, bags,
                             bag_size, grad_weight, grad_psw, workspace, workspace_bytes, stream);
}

extern "C" int pkm_eb_bwd_sgd(const void* values, int64_t num_rows, int64_t dim, int dtype, const int64_t* indices,
                              const void* psw, int psw_dtype, const void* grad_out, int64_t bags, int64_t bag_size,
                              float scale, float lr, float weight_decay, int grad_clip, void* new_values,
                              void* scaled_grad, void* grad_psw, int32_t* counts, float* row_sumsq, void* workspace,
                              size_t workspace_bytes, void* stream) {
  PKM_REQUIRE(dtype == PKM_DTYPE_F32 || dtype == PKM_DTYPE_BF16, PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd_sgd: dtype %d not supported (float32, bfloat16 are)", dtype);
  GroupCfg c;
  BwdLayout l;
  int rc = eb_bwd_check("pkm_eb_bwd_sgd", num_rows, dim, dtype, indices, psw, psw_dtype, bags, bag_size, workspace,
                        workspace_bytes, &c, &l);
  if (rc != PKM_OK) return rc;
  const int64_t N = bags * bag_size;
  PKM_REQUIRE(num_rows == 0 || (values != nullptr && new_values != nullptr), PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd_sgd: null values / new_values");
  {
    const uintptr_t tb = (uintptr_t)num_rows * (uintptr_t)dim * (dtype == PKM_DTYPE_F32 ? 4u : 2u);
    const uintptr_t v0 = (uintptr_t)values, n0 = (uintptr_t)new_values;
    PKM_REQUIRE(num_rows == 0 || n0 + tb <= v0 || v0 + tb <= n0, PKM_ERR_INVALID_ARGUMENT,
                "pkm_eb_bwd_sgd: new_values overlaps values");
  }
  PKM_REQUIRE(N == 0 || grad_out != nullptr, PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd_sgd: null grad_out");
  PKM_REQUIRE(grad_psw == nullptr || psw != nullptr, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd_sgd: grad_psw given without psw");
  PKM_REQUIRE(((uintptr_t)values | (uintptr_t)grad_out | (uintptr_t)new_values | (uintptr_t)scaled_grad) % 16 == 0,
              PKM_ERR_INVALID_ARGUMENT, "pkm_eb_bwd_sgd: values, grad_out and outputs must be 16-byte aligned");
  rc = eb_bwd_prepare(num_rows, dim, dtype, indices, psw, psw_dtype, bags, bag_size, workspace, workspace_bytes,
                      false, stream);
  if (rc != PKM_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const SortedView v = sorted_view(l, ws);
  const SgdArgs S = {new_values, scaled_grad, counts, row_sumsq, scale, lr, weight_decay, grad_clip};
  bool ok;
  if (dtype == PKM_DTYPE_F32)
    ok = dispatch_reduce<float, float>(false, c, values, num_rows, dim, psw, psw_dtype, grad_out, bag_size, v.offs,
                                       v.keys, v.vals, v.nvalid, N, l, ws, nullptr, grad_psw, st, &S);
  else
    ok = dispatch_reduce<bf16_t, bf16_t>(false, c, values, num_rows, dim, psw, psw_dtype, grad_out, bag_size, v.offs,
                                         v.keys, v.vals, v.nvalid, N, l, ws, nullptr, grad_psw, st, &S);
  PKM_REQUIRE(ok, PKM_ERR_UNSUPPORTED, "pkm_eb_bwd_sgd: no kernel for lpg=%d vpl=%d", c.lpg, c.vpl);
  if (N > 0 && grad_psw != nullptr && c.lpg != 64)  // (64-lane rows: inside gpsw_scatter_kernel)
    hipLaunchKernelGGL(zero_invalid_gpsw_kernel, dim3(64), dim3(256), 0, st, (const uint32_t*)v.invalid, grad_psw,
                       psw_dtype);
  return pkm_check_launch("pkm_eb_bwd_sgd");
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

// ---------------------------------------------------------------------------
// pkm_eb_bwd_noalloc: pkm_eb_bwd on a fixed scratch array instead of a
// caller-provided workspace, for callers that cannot allocate.
// ---------------------------------------------------------------------------
namespace pkm {

constexpr size_t kNoallocScratchBytes = (size_t)64 << 20;
constexpr int kMaxScratchDevices = 64;

// One copy per GPU the library runs on, held until the process ends. Host
// code never passes `scratch` itself to a kernel (on the host the name is only
// a stand-in for the symbol): it uses the per-device address that
// hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the calling thread's current device, looked
// up once per device (with that device current) and kept.
static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  PKM_REQUIRE(e == hipSuccess, PKM_ERR_HIP, "pkm_eb_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  PKM_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, PKM_ERR_UNSUPPORTED,
              "pkm_eb_bwd_noalloc: device %d beyond the %d this library keeps scratch addresses for", dev,
              kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    PKM_REQUIRE(e == hipSuccess && p != nullptr, PKM_ERR_HIP,
                "pkm_eb_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PKM_OK;
}

}  // namespace pkm

extern "C" int pkm_eb_bwd_noalloc(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                                  const int64_t* indices, const void* psw, int psw_dtype, const void* grad_out,
                                  int grad_dtype, int64_t bags, int64_t bag_size, void* grad_weight, void* grad_psw,
                                  void* stream) {
  PKM_REQUIRE(num_rows >= 0 && dim > 0 && bags >= 0 && bag_size >= 0, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd_noalloc: bad sizes num_rows=%lld dim=%lld bags=%lld bag_size=%lld", (long long)num_rows,
              (long long)dim, (long long)bags, (long long)bag_size);
  PKM_REQUIRE(bags * bag_size < ((int64_t)1 << 31) && num_rows < ((int64_t)1 << 31) - 1, PKM_ERR_INVALID_ARGUMENT,
              "pkm_eb_bwd_noalloc: bags*bag_size=%lld must be < 2^31 and num_rows=%lld < 2^31-1",
              (long long)(bags * bag_size), (long long)num_rows);
  const size_t need = bwd_layout(num_rows, dim, bags, bag_size).total;
  PKM_REQUIRE(need <= kNoallocScratchBytes, PKM_ERR_WORKSPACE,
              "pkm_eb_bwd_noalloc: these sizes (num_rows=%lld dim=%lld bags=%lld bag_size=%lld) need %zu bytes of "
              "scratch, more than the fixed %zu bytes; use pkm_eb_bwd with a workspace",
              (long long)num_rows, (long long)dim, (long long)bags, (long long)bag_size, need,
              kNoallocScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != PKM_OK) return rc;
  return pkm_eb_bwd(weight, num_rows, dim, weight_dtype, indices, psw, psw_dtype, grad_out, grad_dtype, bags,
                    bag_size, grad_weight, grad_psw, ws, kNoallocScratchBytes, stream);
}

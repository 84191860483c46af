// fgs_binning.hip -- scans, tile duplication, stable LSD radix sort and tile
// ranges.
//
// The rasterize_gaussians path (reference binding.cpp:153-212) sorts K
// duplicates on the 64-bit key (tile << 32 | depth bits) with ties in input
// order.  The order that sort produces is (tile, depth bits, Gaussian index).
// It is produced here in two stable stages:
//   1. sort the P Gaussians by depth bits (32 bits, ties by index);
//   2. duplicate in that order and stable-sort the K duplicates by tile id
//      (ceil(log2 T) bits only, 13 bits at 1080p).
// That moves the 32 depth bits from a K-sized sort to a P-sized one.
//
// Radix sort: 8-bit digits, 4096-key chunks (256 threads x 16 keys),
// per-chunk digit histograms -> one exclusive scan over the digit-major
// histogram matrix -> a scatter pass.  The scatter ranks keys stably within
// a wavefront with ballots over the digit bits (wave64 match-any), combines
// the four wavefronts through LDS counters, permutes the chunk into digit
// order in LDS, and writes each digit run contiguously to HBM.
#include "fgs_common.hpp"

namespace fgs {

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kChunk = kThreads * kItems;  // 4096
constexpr int kWavesPerBlock = kThreads / kWave;

// ---------------------------------------------------------------------------
// Scan (u32, wrapping).  reduce -> scan partials -> final.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
scan_reduce_kernel(const uint32_t* __restrict__ in, int64_t n, uint32_t* __restrict__ partials) {
  __shared__ uint32_t s_tmp[kWavesPerBlock + 1];
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + i * kThreads + threadIdx.x;
    if (idx < n) sum += in[idx];
  }
  uint32_t total;
  block_excl_scan(sum, s_tmp, &total);
  if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Exclusive scan of partials[0..nb) in place by one 1024-thread block.
__global__ void __launch_bounds__(1024)
scan_partials_kernel(uint32_t* __restrict__ partials, int64_t nb) {
  __shared__ uint32_t s_tmp[1024 / kWave + 1];
  uint32_t carry = 0;
  for (int64_t base = 0; base < nb; base += 1024) {
    const int64_t idx = base + threadIdx.x;
    const uint32_t v = idx < nb ? partials[idx] : 0u;
    uint32_t total;
    const uint32_t ex = block_excl_scan(v, s_tmp, &total);
    if (idx < nb) partials[idx] = carry + ex;
    carry += total;
  }
}

// Padded LDS index so that thread t reading its 16 consecutive elements is
// free of bank conflicts.
__device__ __forceinline__ int pad_idx(int i) { return i + (i >> 4); }

__global__ void __launch_bounds__(kThreads)
scan_final_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, int64_t n,
                  const uint32_t* __restrict__ partials, int inclusive) {
  __shared__ uint32_t s_data[kChunk + kChunk / 16];
  __shared__ uint32_t s_tmp[kWavesPerBlock + 1];
  const int64_t base = (int64_t)blockIdx.x * kChunk;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int li = i * kThreads + threadIdx.x;
    const int64_t idx = base + li;
    s_data[pad_idx(li)] = idx < n ? in[idx] : 0u;
  }
  __syncthreads();
  uint32_t v[kItems];
  uint32_t tsum = 0;
#pragma unroll
  for (int k = 0; k < kItems; ++k) {
    v[k] = s_data[pad_idx(threadIdx.x * kItems + k)];
    tsum += v[k];
  }
  uint32_t total;
  uint32_t run = block_excl_scan(tsum, s_tmp, &total) + partials[blockIdx.x];
#pragma unroll
  for (int k = 0; k < kItems; ++k) {
    const uint32_t x = v[k];
    if (inclusive) {
      run += x;
      v[k] = run;
    } else {
      v[k] = run;
      run += x;
    }
  }
#pragma unroll
  for (int k = 0; k < kItems; ++k) s_data[pad_idx(threadIdx.x * kItems + k)] = v[k];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int li = i * kThreads + threadIdx.x;
    const int64_t idx = base + li;
    if (idx < n) out[idx] = s_data[pad_idx(li)];
  }
}

static size_t scan_ws_bytes(int64_t n) {
  const int64_t nb = (n + kChunk - 1) / kChunk;
  return (size_t)((nb + 1) * 4 + 255) & ~(size_t)255;
}

static int32_t launch_scan(const uint32_t* in, uint32_t* out, int64_t n, void* ws, bool inclusive,
                           hipStream_t st) {
  if (n <= 0) return FGS_OK;
  const int64_t nb = (n + kChunk - 1) / kChunk;
  uint32_t* partials = (uint32_t*)ws;
  hipLaunchKernelGGL(scan_reduce_kernel, dim3((unsigned)nb), dim3(kThreads), 0, st, in, n, partials);
  hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(1024), 0, st, partials, nb);
  hipLaunchKernelGGL(scan_final_kernel, dim3((unsigned)nb), dim3(kThreads), 0, st, in, out, n,
                     partials, inclusive ? 1 : 0);
  return check_launch("scan");
}

// ---------------------------------------------------------------------------
// Fill / copy helpers (kernels rather than hipMemsetAsync so that callers may
// capture these calls in HIP graphs).
// ---------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t value, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = value;
}

static void launch_fill(uint32_t* dst, uint32_t v, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, v, n);
}

template <typename K>
__global__ void copy_pairs_kernel(const K* __restrict__ ki, const uint32_t* __restrict__ vi,
                                  K* __restrict__ ko, uint32_t* __restrict__ vo, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    ko[i] = ki[i];
    vo[i] = vi ? vi[i] : (uint32_t)i;
  }
}

// ---------------------------------------------------------------------------
// Radix sort pass kernels.
// ---------------------------------------------------------------------------
template <typename K>
__global__ void __launch_bounds__(kThreads)
radix_hist_kernel(const K* __restrict__ keys, int64_t n, int shift, int nbits,
                  uint32_t* __restrict__ hist, int64_t nb) {
  __shared__ uint32_t s_h[256];
  s_h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  const uint32_t mask = (1u << nbits) - 1u;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + i * kThreads + threadIdx.x;
    if (idx < n) atomicAdd(&s_h[(uint32_t)(keys[idx] >> shift) & mask], 1u);
  }
  __syncthreads();
  if ((int)threadIdx.x <= (int)mask) hist[(int64_t)threadIdx.x * nb + blockIdx.x] = s_h[threadIdx.x];
}

template <typename K>
__global__ void __launch_bounds__(kThreads)
radix_scatter_kernel(const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                     K* __restrict__ keys_out, uint32_t* __restrict__ vals_out, int64_t n,
                     int shift, int nbits, const uint32_t* __restrict__ offsets, int64_t nb) {
  __shared__ uint32_t s_wh[kWavesPerBlock][256];
  __shared__ uint32_t s_dstart[256];
  __shared__ uint32_t s_goff[256];
  __shared__ uint32_t s_tmp[kWavesPerBlock + 1];
  __shared__ K s_keys[kChunk];
  __shared__ uint32_t s_vals[kChunk];
  const int t = (int)threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  const uint32_t mask = (1u << nbits) - 1u;
#pragma unroll
  for (int k = 0; k < kWavesPerBlock; ++k) s_wh[k][t] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kChunk + (int64_t)w * (kChunk / kWavesPerBlock);
  const uint64_t lt = lanemask_lt();
  K key[kItems];
  uint32_t val[kItems];
  uint32_t rank[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int64_t idx = base + it * kWave + lane;
    const bool valid = idx < n;
    key[it] = valid ? keys_in[idx] : (K)0;
    val[it] = valid ? (vals_in ? vals_in[idx] : (uint32_t)idx) : 0u;
    const uint32_t d = (uint32_t)(key[it] >> shift) & mask;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t r = (uint32_t)__popcll(peers & lt);
    uint32_t old = 0;
    if (valid) old = s_wh[w][d];
    if (valid && r == 0) s_wh[w][d] = old + (uint32_t)__popcll(peers);
    rank[it] = old + r;
  }
  __syncthreads();
  {
    uint32_t c[kWavesPerBlock];
    uint32_t tot = 0;
#pragma unroll
    for (int k = 0; k < kWavesPerBlock; ++k) {
      c[k] = ((uint32_t)t <= mask) ? s_wh[k][t] : 0u;
      tot += c[k];
    }
    uint32_t total;
    const uint32_t ds = block_excl_scan(tot, s_tmp, &total);
    uint32_t run = ds;
#pragma unroll
    for (int k = 0; k < kWavesPerBlock; ++k) {
      s_wh[k][t] = run;
      run += c[k];
    }
    s_dstart[t] = ds;
    s_goff[t] = ((uint32_t)t <= mask) ? offsets[(int64_t)t * nb + blockIdx.x] : 0u;
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int64_t idx = base + it * kWave + lane;
    if (idx < n) {
      const uint32_t d = (uint32_t)(key[it] >> shift) & mask;
      const uint32_t pos = s_wh[w][d] + rank[it];
      s_keys[pos] = key[it];
      s_vals[pos] = val[it];
    }
  }
  __syncthreads();
  const int64_t rem = n - (int64_t)blockIdx.x * kChunk;
  const int cnt = rem < kChunk ? (int)rem : kChunk;
  for (int j = t; j < cnt; j += kThreads) {
    const K k = s_keys[j];
    const uint32_t d = (uint32_t)(k >> shift) & mask;
    const uint32_t g = s_goff[d] + ((uint32_t)j - s_dstart[d]);
    keys_out[g] = k;
    vals_out[g] = s_vals[j];
  }
}

template <typename K>
static size_t sort_ws_bytes(int64_t n) {
  const int64_t nb = (n + kChunk - 1) / kChunk;
  size_t b = 0;
  b += ((size_t)n * sizeof(K) + 255) & ~(size_t)255;   // tmp keys
  b += ((size_t)n * 4 + 255) & ~(size_t)255;           // tmp vals
  b += ((size_t)nb * 256 * 4 + 255) & ~(size_t)255;    // histogram matrix
  b += scan_ws_bytes(nb * 256);
  return b;
}

// Stable sort on bits [begin, end).  vals_in may be NULL (values = index).
// keys_in/vals_in are not modified.
template <typename K>
static int32_t radix_sort_pairs(const K* keys_in, const uint32_t* vals_in, K* keys_out,
                                uint32_t* vals_out, int64_t n, int begin, int end, void* ws,
                                hipStream_t st) {
  if (n <= 0) return FGS_OK;
  const int nbits_total = end - begin;
  if (nbits_total <= 0) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(copy_pairs_kernel<K>, dim3((unsigned)blocks), dim3(256), 0, st, keys_in,
                       vals_in, keys_out, vals_out, n);
    return check_launch("copy_pairs");
  }
  const int passes = (nbits_total + 7) / 8;
  const int64_t nb = (n + kChunk - 1) / kChunk;
  char* p = (char*)ws;
  K* tk = (K*)p;
  p += ((size_t)n * sizeof(K) + 255) & ~(size_t)255;
  uint32_t* tv = (uint32_t*)p;
  p += ((size_t)n * 4 + 255) & ~(size_t)255;
  uint32_t* hist = (uint32_t*)p;
  p += ((size_t)nb * 256 * 4 + 255) & ~(size_t)255;
  void* scan_ws = p;
  const K* src_k = keys_in;
  const uint32_t* src_v = vals_in;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = begin + pass * 8;
    const int nbits = (end - shift) < 8 ? (end - shift) : 8;
    const bool to_out = ((passes - 1 - pass) % 2) == 0;
    K* dk = to_out ? keys_out : tk;
    uint32_t* dv = to_out ? vals_out : tv;
    hipLaunchKernelGGL(radix_hist_kernel<K>, dim3((unsigned)nb), dim3(kThreads), 0, st, src_k, n,
                       shift, nbits, hist, nb);
    const int32_t e = launch_scan(hist, hist, nb * (int64_t)(1 << nbits), scan_ws, false, st);
    if (e != FGS_OK) return e;
    hipLaunchKernelGGL(radix_scatter_kernel<K>, dim3((unsigned)nb), dim3(kThreads), 0, st, src_k,
                       src_v, dk, dv, n, shift, nbits, hist, nb);
    const int32_t e2 = check_launch("radix_scatter");
    if (e2 != FGS_OK) return e2;
    src_k = dk;
    src_v = dv;
  }
  return FGS_OK;
}

// ---------------------------------------------------------------------------
// Duplication.
// ---------------------------------------------------------------------------
struct EmitKeys64 {
  uint64_t* keys;
  uint32_t* vals;
  int64_t off;
  int64_t cap;
  uint32_t depth_bits;
  uint32_t idx;
  int gx;
  __device__ __forceinline__ void operator()(int u, int vmin, int vmax, bool is_y) {
    for (int v = vmin; v < vmax; ++v) {
      const int tile = is_y ? (u * gx + v) : (v * gx + u);
      if (off < cap) {
        keys[off] = ((uint64_t)(uint32_t)tile << 32) | (uint64_t)depth_bits;
        vals[off] = idx;
      }
      ++off;
    }
  }
};

// Gaussian-order duplication (fastgs_binning.metal:182-213).
__global__ void __launch_bounds__(256)
duplicate_keys_kernel(int32_t P, const float* __restrict__ xys, const float* __restrict__ depths,
                      const uint32_t* __restrict__ point_offsets,
                      const float* __restrict__ conic_opacity,
                      const uint32_t* __restrict__ tiles_touched, float mult, int gx, int gy,
                      int64_t K, uint64_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  if (tiles_touched[i] == 0u) return;
  EmitKeys64 e;
  e.keys = keys;
  e.vals = vals;
  e.off = (i == 0) ? 0 : (int64_t)point_offsets[i - 1];
  e.cap = K;
  e.depth_bits = __float_as_uint(depths[i]);
  e.idx = (uint32_t)i;
  e.gx = gx;
  const float2 xy = *reinterpret_cast<const float2*>(xys + 2 * (size_t)i);
  const float4 co = *reinterpret_cast<const float4*>(conic_opacity + 4 * (size_t)i);
  tiles_walk(xy.x, xy.y, co, gx, gy, mult, e);
}

// Depth keys of the stage-1 sort: visible Gaussians by depth bits, culled
// ones (tiles_touched == 0) last.
__global__ void depth_keys_kernel(int32_t P, const float* __restrict__ depths,
                                  const uint32_t* __restrict__ tiles_touched,
                                  uint32_t* __restrict__ dkeys) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  dkeys[i] = tiles_touched[i] ? __float_as_uint(depths[i]) : 0xFFFFFFFFu;
}

__global__ void gather_counts_kernel(int32_t P, const uint32_t* __restrict__ order,
                                     const uint32_t* __restrict__ tiles_touched,
                                     uint32_t* __restrict__ cnt) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  cnt[i] = tiles_touched[order[i]];
}

struct EmitTiles {
  uint32_t* tkeys;
  uint32_t* tvals;
  int64_t off;
  int64_t end;
  uint32_t idx;
  int gx;
  __device__ __forceinline__ void operator()(int u, int vmin, int vmax, bool is_y) {
    for (int v = vmin; v < vmax; ++v) {
      if (off < end) {
        tkeys[off] = (uint32_t)(is_y ? (u * gx + v) : (v * gx + u));
        tvals[off] = idx;
      }
      ++off;
    }
  }
};

// Depth-order duplication: thread i handles the i-th Gaussian by depth and
// writes (tile id, Gaussian index) at its depth-order offset.
__global__ void __launch_bounds__(256)
duplicate_sorted_kernel(int32_t P, const uint32_t* __restrict__ order,
                        const uint32_t* __restrict__ offs, const float* __restrict__ xys,
                        const float* __restrict__ conic_opacity,
                        const uint32_t* __restrict__ tiles_touched, float mult, int gx, int gy,
                        int64_t K, uint32_t* __restrict__ tkeys, uint32_t* __restrict__ tvals) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const uint32_t g = order[i];
  const uint32_t n = tiles_touched[g];
  if (n == 0u) return;
  EmitTiles e;
  e.tkeys = tkeys;
  e.tvals = tvals;
  e.off = (int64_t)offs[i];
  e.end = e.off + (int64_t)n;
  if (e.end > K) e.end = K;
  e.idx = g;
  e.gx = gx;
  const float2 xy = *reinterpret_cast<const float2*>(xys + 2 * (size_t)g);
  const float4 co = *reinterpret_cast<const float4*>(conic_opacity + 4 * (size_t)g);
  tiles_walk(xy.x, xy.y, co, gx, gy, mult, e);
}

// Sorted tile ids -> 64-bit keys and tile ranges (fastgs_tile_prep.metal:10-37).
__global__ void finalize_keys_ranges_kernel(int64_t K, const uint32_t* __restrict__ tiles,
                                            const uint32_t* __restrict__ point_list,
                                            const float* __restrict__ depths,
                                            uint64_t* __restrict__ keys64,
                                            uint32_t* __restrict__ ranges) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= K) return;
  const uint32_t cur = tiles[i];
  const uint32_t g = point_list[i];
  keys64[i] = ((uint64_t)cur << 32) | (uint64_t)__float_as_uint(depths[g]);
  if (i > 0) {
    const uint32_t prev = tiles[i - 1];
    if (cur != prev) {
      ranges[2 * (size_t)prev + 1] = (uint32_t)i;
      ranges[2 * (size_t)cur] = (uint32_t)i;
    }
  }
  if (i == K - 1) ranges[2 * (size_t)cur + 1] = (uint32_t)K;
}

// Reference tile_prep semantics on 64-bit keys (any order).
__global__ void tile_ranges64_kernel(int64_t K, const uint64_t* __restrict__ keys, int32_t T,
                                     uint32_t* __restrict__ ranges) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= K) return;
  const uint32_t cur = (uint32_t)(keys[i] >> 32);
  const bool valid = cur != 0xFFFFFFFFu;
  if (i == 0) {
    if (cur < (uint32_t)T) ranges[2 * (size_t)cur] = 0u;
  } else {
    const uint32_t prev = (uint32_t)(keys[i - 1] >> 32);
    if (cur != prev) {
      if (prev < (uint32_t)T) ranges[2 * (size_t)prev + 1] = (uint32_t)i;
      if (valid && cur < (uint32_t)T) ranges[2 * (size_t)cur] = (uint32_t)i;
    }
  }
  if (i == K - 1 && valid && cur < (uint32_t)T) ranges[2 * (size_t)cur + 1] = (uint32_t)K;
}

__global__ void bucket_count_kernel(int32_t T, const uint32_t* __restrict__ ranges,
                                    uint32_t* __restrict__ bucket_count) {
  const int t = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (t >= T) return;
  const int n = (int)(ranges[2 * t + 1] - ranges[2 * t]);
  bucket_count[t] = (uint32_t)((n + 31) / 32);
}

static int bits_for(int64_t count) {
  int b = 0;
  while (b < 32 && ((int64_t)1 << b) < count) ++b;
  return b;
}

struct BinningLayout {
  size_t dkeys, dkeys_s, order, cnt, scanP, sortP, tkeys, tvals, tkeys_s, sortK, scanT, total;
};

static size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

static BinningLayout binning_layout(int32_t P, int64_t K, int32_t T) {
  BinningLayout L;
  size_t o = 0;
  L.dkeys = o; o += al((size_t)P * 4);
  L.dkeys_s = o; o += al((size_t)P * 4);
  L.order = o; o += al((size_t)P * 4);
  L.cnt = o; o += al((size_t)P * 4);
  L.scanP = o; o += scan_ws_bytes(P);
  L.sortP = o; o += sort_ws_bytes<uint32_t>(P);
  L.tkeys = o; o += al((size_t)K * 4);
  L.tvals = o; o += al((size_t)K * 4);
  L.tkeys_s = o; o += al((size_t)K * 4);
  L.sortK = o; o += sort_ws_bytes<uint32_t>(K);
  L.scanT = o; o += scan_ws_bytes(T);
  L.total = o;
  return L;
}

}  // namespace fgs

using namespace fgs;

extern "C" size_t fgs_scan_workspace_bytes(int64_t n) { return scan_ws_bytes(n < 1 ? 1 : n); }

extern "C" int32_t fgs_inclusive_scan_u32(const uint32_t* in, uint32_t* out, int64_t n,
                                          void* workspace, void* stream) {
  if (n < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_inclusive_scan_u32: n < 0");
  if (n == 0) return FGS_OK;
  if (!in || !out || !workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_inclusive_scan_u32: null pointer");
  return launch_scan(in, out, n, workspace, true, (hipStream_t)stream);
}

extern "C" int32_t fgs_fill_u32(uint32_t* dst, uint32_t value, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && !dst)) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_fill_u32: bad argument");
  launch_fill(dst, value, n, (hipStream_t)stream);
  return check_launch("fill_u32");
}

extern "C" int32_t fgs_duplicate_with_keys(int32_t P, const float* xys, const float* depths,
                                           const uint32_t* point_offsets,
                                           const float* conic_opacity,
                                           const uint32_t* tiles_touched, float mult,
                                           int32_t grid_x, int32_t grid_y, int64_t num_rendered,
                                           uint64_t* keys_unsorted, uint32_t* values_unsorted,
                                           void* stream) {
  if (P < 0 || num_rendered < 0 || grid_x <= 0 || grid_y <= 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_duplicate_with_keys: bad sizes");
  if (num_rendered == 0) return FGS_OK;
  if (!keys_unsorted || !values_unsorted || (P > 0 && (!xys || !depths || !point_offsets ||
                                                       !conic_opacity || !tiles_touched)))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_duplicate_with_keys: null pointer");
  hipStream_t st = (hipStream_t)stream;
  launch_fill(reinterpret_cast<uint32_t*>(keys_unsorted), 0u, num_rendered * 2, st);
  launch_fill(values_unsorted, 0u, num_rendered, st);
  if (P > 0)
    hipLaunchKernelGGL(duplicate_keys_kernel, dim3(ceil_div_u(P, 256)), dim3(256), 0, st, P, xys,
                       depths, point_offsets, conic_opacity, tiles_touched, mult, grid_x, grid_y,
                       num_rendered, keys_unsorted, values_unsorted);
  return check_launch("duplicate_keys_kernel");
}

extern "C" size_t fgs_sort_workspace_bytes(int64_t n) { return sort_ws_bytes<uint64_t>(n < 1 ? 1 : n); }

extern "C" int32_t fgs_sort_pairs_u64(const uint64_t* keys_in, const uint32_t* values_in,
                                      uint64_t* keys_out, uint32_t* values_out, int64_t n,
                                      int32_t begin_bit, int32_t end_bit, void* workspace,
                                      void* stream) {
  if (n < 0 || begin_bit < 0 || end_bit > 64 || begin_bit > end_bit)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_sort_pairs_u64: bad arguments");
  if (n == 0) return FGS_OK;
  if (n > 0xFFFFFFFFll)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_sort_pairs_u64: n exceeds 2^32-1");
  if (!keys_in || !keys_out || !values_out || !workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_sort_pairs_u64: null pointer");
  return radix_sort_pairs<uint64_t>(keys_in, values_in, keys_out, values_out, n, begin_bit, end_bit,
                                    workspace, (hipStream_t)stream);
}

extern "C" int32_t fgs_tile_ranges(const uint64_t* keys, int64_t num_rendered, int32_t num_tiles,
                                   uint32_t* ranges, uint32_t* bucket_count, void* stream) {
  if (num_rendered < 0 || num_tiles < 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_tile_ranges: bad sizes");
  if (num_tiles == 0) return FGS_OK;
  if (!ranges || !bucket_count || (num_rendered > 0 && !keys))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_tile_ranges: null pointer");
  hipStream_t st = (hipStream_t)stream;
  launch_fill(ranges, 0u, 2 * (int64_t)num_tiles, st);
  if (num_rendered > 0)
    hipLaunchKernelGGL(tile_ranges64_kernel, dim3(ceil_div_u(num_rendered, 256)), dim3(256), 0, st,
                       num_rendered, keys, num_tiles, ranges);
  hipLaunchKernelGGL(bucket_count_kernel, dim3(ceil_div_u(num_tiles, 256)), dim3(256), 0, st,
                     num_tiles, ranges, bucket_count);
  return check_launch("tile_ranges");
}

extern "C" size_t fgs_binning_workspace_bytes(int32_t P, int64_t num_rendered, int32_t num_tiles) {
  return binning_layout(P < 1 ? 1 : P, num_rendered < 1 ? 1 : num_rendered,
                        num_tiles < 1 ? 1 : num_tiles).total;
}

extern "C" int32_t fgs_binning_sorted(const fgs_binning_io* io, void* stream) {
  if (!io) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: null io");
  const int32_t P = io->P;
  const int64_t K = io->num_rendered;
  if (P < 0 || K < 0 || io->grid_x <= 0 || io->grid_y <= 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: bad sizes");
  const int64_t T64 = (int64_t)io->grid_x * io->grid_y;
  if (T64 > 0x7FFFFFFFll) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: too many tiles");
  if (K > 0xFFFFFFFFll) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: K exceeds 2^32-1");
  const int32_t T = (int32_t)T64;
  if (!io->ranges || !io->bucket_count || !io->bucket_offsets || !io->workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const BinningLayout L = binning_layout(P < 1 ? 1 : P, K < 1 ? 1 : K, T);
  char* ws = (char*)io->workspace;
  uint32_t* dkeys = (uint32_t*)(ws + L.dkeys);
  uint32_t* dkeys_s = (uint32_t*)(ws + L.dkeys_s);
  uint32_t* order = (uint32_t*)(ws + L.order);
  uint32_t* cnt = (uint32_t*)(ws + L.cnt);
  uint32_t* tkeys = (uint32_t*)(ws + L.tkeys);
  uint32_t* tvals = (uint32_t*)(ws + L.tvals);
  uint32_t* tkeys_s = (uint32_t*)(ws + L.tkeys_s);
  launch_fill(io->ranges, 0u, 2 * (int64_t)T, st);
  if (K > 0 && P > 0) {
    if (!io->xys || !io->depths || !io->conic_opacity || !io->tiles_touched ||
        !io->point_list_keys || !io->point_list)
      return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: null pointer");
    const unsigned gP = ceil_div_u(P, 256);
    hipLaunchKernelGGL(depth_keys_kernel, dim3(gP), dim3(256), 0, st, P, io->depths,
                       io->tiles_touched, dkeys);
    int32_t e = radix_sort_pairs<uint32_t>(dkeys, nullptr, dkeys_s, order, P, 0, 32,
                                           ws + L.sortP, st);
    if (e != FGS_OK) return e;
    hipLaunchKernelGGL(gather_counts_kernel, dim3(gP), dim3(256), 0, st, P, order,
                       io->tiles_touched, cnt);
    e = launch_scan(cnt, cnt, P, ws + L.scanP, false, st);
    if (e != FGS_OK) return e;
    hipLaunchKernelGGL(duplicate_sorted_kernel, dim3(gP), dim3(256), 0, st, P, order, cnt, io->xys,
                       io->conic_opacity, io->tiles_touched, io->mult, io->grid_x, io->grid_y, K,
                       tkeys, tvals);
    e = radix_sort_pairs<uint32_t>(tkeys, tvals, tkeys_s, io->point_list, K, 0, bits_for(T),
                                   ws + L.sortK, st);
    if (e != FGS_OK) return e;
    hipLaunchKernelGGL(finalize_keys_ranges_kernel, dim3(ceil_div_u(K, 256)), dim3(256), 0, st, K,
                       tkeys_s, io->point_list, io->depths, io->point_list_keys, io->ranges);
  }
  hipLaunchKernelGGL(bucket_count_kernel, dim3(ceil_div_u(T, 256)), dim3(256), 0, st, T,
                     io->ranges, io->bucket_count);
  const int32_t e = launch_scan(io->bucket_count, io->bucket_offsets, T, ws + L.scanT, true, st);
  if (e != FGS_OK) return e;
  return check_launch("binning_sorted");
}

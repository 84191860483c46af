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
// Radix sort: digits of at most 8 bits (13 tile bits: 7 + 6), 4096-key
// chunks (256 threads x 16 keys).  One kernel counts the digits of every
// pass; each pass is then one kernel that ranks its chunk stably within each
// wavefront with ballots over the digit bits (wave64 match-any), combines the
// four wavefronts through LDS counters, gets each digit's global offset by
// decoupled look-back over the earlier chunks, permutes the chunk into digit
// order in LDS and writes each digit run contiguously to HBM.
#include "fgs_common.hpp"

#include <atomic>
#include <cstdio>
#include <mutex>

namespace fgs {

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kChunk = kThreads * kItems;  // 4096
constexpr int kWavesPerBlock = kThreads / kWave;

// ---------------------------------------------------------------------------
// Decoupled look-back.  A pass over n items runs one workgroup per chunk of
// kChunk items; a workgroup takes its chunk number from an atomic ticket, so
// chunk c is only ever waited on by chunks > c whose workgroups started
// later, and every wait ends.  Each chunk publishes, per counter, a 64-bit
// status word: (flag << 32) | value, flag 1 = the chunk's own aggregate,
// flag 2 = the inclusive prefix up to and including the chunk.  A chunk walks
// back over its predecessors adding aggregates until it meets an inclusive
// prefix.  Status words and tickets start at zero (one fill kernel per call).
// Radix passes keep their status words chunk-major ([chunk][digit]): a
// chunk's 256 counters are published and read as one contiguous block.  They
// look back in two levels: a chunk sums its predecessors inside its group of
// kLbGroup chunks directly, and every chunk also adds its counts into its
// group's running word ((arrivals << 32) + count, an atomic add), which is
// complete once all kLbGroup chunks have arrived.  The earlier groups are
// then walked from the nearest, adding complete group words, until one whose
// inclusive prefix the group's last chunk has published.  No chunk waits for
// another's look-back while the group words complete (a walk over every
// earlier chunk had made the last chunks of a 1M-key pass wait about 13 us
// longer than the first; group totals summed by each group's last chunk
// added about a microsecond per pass).
// Radix passes take their chunk number from the workgroup index: a chunk
// waits only on lower-numbered chunks, which each XCD dispatches before it.
// The spins are bounded as a backstop.
// ---------------------------------------------------------------------------
// Padded LDS index so that thread t reading its 16 consecutive elements is
// free of bank conflicts.
__device__ __forceinline__ int pad_idx(int i) { return i + (i >> 4); }

constexpr uint32_t kFlagAggregate = 1u;
constexpr uint32_t kFlagPrefix = 2u;
constexpr uint32_t kSpinLimit = 1u << 24;  // default polls of one bounded wait
// Bits of a wait-status word: which kind of bounded wait gave up.
constexpr uint32_t kWaitScan = 1u;      // a scan chunk summing its predecessors
constexpr uint32_t kWaitLookBack = 2u;  // a radix-pass chunk looking back

__device__ __forceinline__ void wait_gave_up(uint32_t* err, uint32_t bit) {
  __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void status_store(uint64_t* p, uint32_t flag, uint32_t value) {
  __hip_atomic_store(p, ((uint64_t)flag << 32) | (uint64_t)value, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// The two parts of the exclusive prefix of a chunk, chunk q of look-back
// group g, for one counter whose words are `stride` apart:
//  in_group: the counts of chunks first .. first + q - 1 (its predecessors
//    in the group), from their status words st[c] = (flag << 32) + count;
//    all are read at once (independent loads in flight), then the ones not
//    yet published are read again;
//  gexcl: the counts of groups 0 .. g - 1, from their words gsum[h] =
//    (arrivals << 32) + the arrived chunks' counts, complete at kLbGroup
//    arrivals, and gpre[h] = (kFlagPrefix << 32) + the inclusive prefix
//    through group h, once its last chunk has published it.  Windows of 16
//    groups are read at once and walked from the nearest: a published prefix
//    ends the walk, a complete group word is added, an incomplete one is read
//    again with its window.
// The group words are read after the predecessors: they complete about
// when those have published (one polling loop over both, whose batches need
// three times the registers, measured slower beside the preprocess's colour
// half, which then shared fewer CUs with the pass).  Rereads follow a short
// sleep.  After spin_limit rereads a wait gives up: kWaitLookBack is set in
// *err and the partial sums (never above the true ones, so every position
// stays in bounds) are used.  spin_limit == 0 gives up at once without
// polling.
constexpr int kLbGroup = 16;  // chunks per look-back group
__device__ __forceinline__ void chunk_offsets(const uint64_t* st, int64_t first, int q,
                                              const uint64_t* gsum, const uint64_t* gpre,
                                              int64_t g, int64_t stride, uint32_t* err,
                                              uint32_t spin_limit, uint32_t& in_group,
                                              uint32_t& gexcl) {
  constexpr int kWin = 16;
  in_group = 0u;
  gexcl = 0u;
  if (q == 0 && g == 0) return;
  if (spin_limit == 0u) {
    wait_gave_up(err, kWaitLookBack);
    return;
  }
  uint32_t spins = 0;
  uint32_t pending = (1u << q) - 1u;  // q < kLbGroup
  while (pending) {
    uint64_t w[kLbGroup];
#pragma unroll
    for (int i = 0; i < kLbGroup; ++i)
      w[i] = ((pending >> i) & 1u) ? __hip_atomic_load(st + (first + i) * stride,
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : 0ull;
#pragma unroll
    for (int i = 0; i < kLbGroup; ++i) {
      if (((pending >> i) & 1u) && (uint32_t)(w[i] >> 32) != 0u) {
        in_group += (uint32_t)w[i];
        pending &= ~(1u << i);
      }
    }
    if (pending) {
      if (++spins > spin_limit) {
        wait_gave_up(err, kWaitLookBack);
        return;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  int64_t c = g - 1;  // the nearest group not added yet
  while (c >= 0) {
    const int64_t lo = c >= kWin - 1 ? c - (kWin - 1) : 0;
    uint64_t wp[kWin], ws[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
      const bool in = lo + i <= c;
      wp[i] = in ? __hip_atomic_load(gpre + (lo + i) * stride, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT)
                 : 0ull;
      ws[i] = in ? __hip_atomic_load(gsum + (lo + i) * stride, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT)
                 : 0ull;
    }
    bool stalled = false;
#pragma unroll
    for (int i = kWin - 1; i >= 0; --i) {
      if (stalled || lo + i > c) continue;
      if ((uint32_t)(wp[i] >> 32) == kFlagPrefix) {
        gexcl += (uint32_t)wp[i];
        c = -1;
      } else if ((uint32_t)(ws[i] >> 32) == (uint32_t)kLbGroup) {
        gexcl += (uint32_t)ws[i];
        --c;
      } else {
        stalled = true;  // group c is still incomplete
      }
    }
    if (stalled) {
      if (++spins > spin_limit) {
        wait_gave_up(err, kWaitLookBack);
        return;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
}

// Exclusive prefix of chunk `chunk` of a single counter from the aggregates
// its predecessors publish (status[c], flag kFlagAggregate): the threads of
// the workgroup take predecessors t, t + blockDim, ... (polling each until
// published), then one block reduction.  All loads are in flight at once, so
// there is no chain of waits.  Called by every thread of the workgroup.  A
// predecessor still unpublished after spin_limit polls counts as 0 and sets
// kWaitScan in *err; spin_limit == 0 gives up at once without polling.
__device__ __forceinline__ uint32_t block_sum_predecessors(const uint64_t* status, int64_t chunk,
                                                           uint32_t* err, uint32_t* s_tmp,
                                                           uint32_t spin_limit) {
  if (spin_limit == 0u) {  // uniform
    if (chunk > 0 && threadIdx.x == 0) wait_gave_up(err, kWaitScan);
    return 0u;
  }
  uint32_t acc = 0;
  for (int64_t c = threadIdx.x; c < chunk; c += blockDim.x) {
    uint64_t w = __hip_atomic_load(status + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t spins = 0;
    while ((uint32_t)(w >> 32) == 0u) {
      if (++spins > spin_limit) {
        wait_gave_up(err, kWaitScan);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      w = __hip_atomic_load(status + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    acc += (uint32_t)w;
  }
  uint32_t total;
  block_excl_scan(acc, s_tmp, &total);
  return total;
}

// The workgroup's chunk number from an atomic ticket (the chained scans).
__device__ __forceinline__ int64_t take_ticket(uint32_t* ticket, uint32_t* s_slot) {
  if (threadIdx.x == 0) *s_slot = atomicAdd(ticket, 1u);
  __syncthreads();
  return (int64_t)*s_slot;
}

// ---------------------------------------------------------------------------
// Scan (u32, wrapping): one pass; each chunk publishes its sum and adds up
// its predecessors' sums (block_sum_predecessors).
// kGather: the input element i is tiles_touched[order[i]].
// ---------------------------------------------------------------------------
template <bool kGather>
__global__ void __launch_bounds__(kThreads)
chained_scan_kernel(const uint32_t* __restrict__ in, const uint32_t* __restrict__ order,
                    int64_t n_in, uint32_t* __restrict__ out, int64_t n, int inclusive,
                    uint64_t* status, uint32_t* ticket, uint32_t* err, uint32_t spin_limit) {
  __shared__ uint32_t s_data[kChunk + kChunk / 16];
  __shared__ uint32_t s_tmp[kWavesPerBlock + 1];
  __shared__ uint32_t s_slot;
  const int64_t chunk = take_ticket(ticket, &s_slot);
  const int64_t base = chunk * kChunk;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int li = i * kThreads + threadIdx.x;
    const int64_t idx = base + li;
    uint32_t v = 0u;
    if (idx < n) {
      if (kGather) {
        const uint32_t o = order[idx];  // indices outside [0, n_in) read as 0
        v = (int64_t)o < n_in ? in[o] : 0u;
      } else {
        v = in[idx];
      }
    }
    s_data[pad_idx(li)] = v;
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
  const uint32_t texcl = block_excl_scan(tsum, s_tmp, &total);
  if (threadIdx.x == 0) status_store(status + chunk, kFlagAggregate, total);
  const uint32_t excl = block_sum_predecessors(status, chunk, err, s_tmp, spin_limit);
  uint32_t run = texcl + excl;
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

// Zero-initialised state of one chained scan: status words, ticket, error.
static constexpr size_t scan_state_bytes(int64_t n) {
  return (size_t)(((((n + kChunk - 1) / kChunk) < 1 ? 1 : ((n + kChunk - 1) / kChunk)) * 8 + 16 +
                   255) &
                  ~(int64_t)255);
}
static size_t scan_ws_bytes(int64_t n) { return scan_state_bytes(n); }

// ---------------------------------------------------------------------------
// Fill / copy helpers (kernels rather than hipMemsetAsync so that callers may
// capture these calls in HIP graphs).
// ---------------------------------------------------------------------------
// Up to kFillSpans arrays filled with one value in one launch: 16-byte stores
// from each array's first 16-byte boundary, single words for the ends.
__global__ void __launch_bounds__(256) fill_spans_kernel(FillSpans f) {
  fill_spans_body(f, (int64_t)blockIdx.x * blockDim.x + threadIdx.x,
                  (int64_t)gridDim.x * blockDim.x);
}

void launch_fill_spans(const FillSpans& f, hipStream_t st) {
  int64_t words = 0;
  for (int s = 0; s < f.count; ++s) words += f.n[s] > 0 ? f.n[s] : 0;
  if (words <= 0) return;
  int64_t blocks = (words / 4 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(fill_spans_kernel, dim3((unsigned)blocks), dim3(256), 0, st, f);
}

static void launch_fill(uint32_t* dst, uint32_t v, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  FillSpans f{};
  f.p[0] = dst;
  f.n[0] = n;
  f.count = 1;
  f.value = v;
  launch_fill_spans(f, st);
}

// Polls of one bounded wait before it gives up (fgs_set_wait_spin_limit).
static std::atomic<uint32_t> g_spin_limit{kSpinLimit};

// Scan with its state at `state` (scan_state_bytes(n), zeroed here unless
// the caller has zeroed it already).  A wait that gives up sets kWaitScan in
// *werr when werr is given (cleared here first, by the same fill), else in the
// state's own error word.
template <bool kGather>
static int32_t launch_chained_scan(const uint32_t* in, const uint32_t* order, int64_t n_in,
                                   uint32_t* out, int64_t n, void* state, bool inclusive,
                                   bool zeroed, hipStream_t st, uint32_t* werr = nullptr) {
  if (n <= 0) {
    if (werr) launch_fill(werr, 0u, 1, st);
    return FGS_OK;
  }
  const int64_t nc = (n + kChunk - 1) / kChunk;
  uint64_t* status = (uint64_t*)state;
  uint32_t* ticket = (uint32_t*)(status + nc);
  uint32_t* err = werr ? werr : ticket + 1;
  if (!zeroed || werr) {
    FillSpans f{};
    f.value = 0u;
    if (!zeroed) {
      f.p[f.count] = (uint32_t*)state;
      f.n[f.count++] = (int64_t)(scan_state_bytes(n) / 4);
    }
    if (werr) {
      f.p[f.count] = werr;
      f.n[f.count++] = 1;
    }
    launch_fill_spans(f, st);
  }
  hipLaunchKernelGGL(chained_scan_kernel<kGather>, dim3((unsigned)nc), dim3(kThreads), 0, st, in,
                     order, n_in, out, n, inclusive ? 1 : 0, status, ticket, err,
                     g_spin_limit.load(std::memory_order_relaxed));
  return check_launch("chained_scan");
}

static int32_t launch_scan(const uint32_t* in, uint32_t* out, int64_t n, void* ws, bool inclusive,
                           hipStream_t st, uint32_t* werr = nullptr) {
  return launch_chained_scan<false>(in, nullptr, n, out, n, ws, inclusive, false, st, werr);
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

// Wave64 match-any over the low 8 bits of d: the lanes of `peers` whose d
// has the same 8 bits.  sel is all ones where bit b of d is 0, so (m ^ sel)
// is the ballot m or its complement; with the AND that is one three-input
// bit operation per 32-bit half on gfx950 (v_bitop3_b32), after one compare.
__device__ __forceinline__ uint64_t match_any_8(uint32_t d, uint64_t peers) {
  const uint32_t nd = ~d;
  uint32_t plo = (uint32_t)peers, phi = (uint32_t)(peers >> 32);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const uint32_t sel = (uint32_t)__builtin_amdgcn_sbfe((int32_t)nd, (uint32_t)b, 1u);
    const uint64_t m = __ballot(sel == 0u);
    plo &= (uint32_t)m ^ sel;
    phi &= (uint32_t)(m >> 32) ^ sel;
  }
  return ((uint64_t)phi << 32) | plo;
}

// ---------------------------------------------------------------------------
// One-sweep LSD radix sort: one histogram kernel for every digit pass, then
// one kernel per pass that ranks its chunk, gets each digit's offset by
// look-back and writes the chunk's digit runs.
// ---------------------------------------------------------------------------
struct SortPlan {
  int begin, passes, bits[8];
};

static SortPlan sort_plan(int begin, int end) {
  SortPlan pl{};
  pl.begin = begin;
  const int total = end - begin;
  pl.passes = total <= 0 ? 0 : (total + 7) / 8;
  for (int i = 0; i < pl.passes; ++i) {
    const int rem = total - (total / pl.passes) * pl.passes;  // first `rem` passes take one more
    pl.bits[i] = total / pl.passes + (i < rem ? 1 : 0);
  }
  return pl;
}

// Digit histograms of every pass: hist[pass * 256 + digit] (zeroed by the
// caller).  kDepthKeys: the keys are made here from depths and tiles_touched
// (visible Gaussians by depth bits, culled ones 0xFFFFFFFF) and written out.
template <typename K, bool kDepthKeys>
__global__ void __launch_bounds__(kThreads)
radix_hist_kernel(const K* __restrict__ keys, int64_t n, SortPlan pl, uint32_t* __restrict__ hist,
                  const float* __restrict__ depths, const uint32_t* __restrict__ tiles_touched,
                  uint32_t* __restrict__ dkeys_out, uint32_t* __restrict__ nvis) {
  __shared__ uint32_t s_h[8][256];
  __shared__ uint32_t s_vis;
  for (int p = 0; p < pl.passes; ++p) s_h[p][threadIdx.x] = 0;
  if (threadIdx.x == 0) s_vis = 0;
  uint32_t vis = 0;  // kDepthKeys: this thread's visible keys
  __syncthreads();
  // Grid-stride in batches of kHistBatch keys per thread, all loaded before
  // the first is counted (clamped indices, so the loads carry no branch).
  constexpr int kHistBatch = 16;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; i0 < n;
       i0 += stride * kHistBatch) {
    K kk[kHistBatch];
#pragma unroll
    for (int b = 0; b < kHistBatch; ++b) {
      const int64_t i = i0 + b * stride;
      const int64_t ci = i < n ? i : n - 1;
      if (kDepthKeys) {
        const uint32_t tt = tiles_touched[ci];
        const uint32_t db = __float_as_uint(depths[ci]);
        kk[b] = (K)(tt ? db : 0xFFFFFFFFu);
      } else {
        kk[b] = keys[ci];
      }
    }
#pragma unroll
    for (int b = 0; b < kHistBatch; ++b) {
      const int64_t i = i0 + b * stride;
      if (i < n) {
        const K k = kk[b];
        if (kDepthKeys) {
          dkeys_out[i] = (uint32_t)k;
          // culled keys (all ones) are dropped by the first pass: not counted
          if ((uint32_t)k == 0xFFFFFFFFu) continue;
          ++vis;
        }
        if (kDepthKeys) {  // the depth sort's plan: four 8-bit digits from bit 0
#pragma unroll
          for (int p = 0; p < 4; ++p) atomicAdd(&s_h[p][(uint32_t)(k >> (8 * p)) & 0xFFu], 1u);
        } else {
          int shift = pl.begin;
          for (int p = 0; p < pl.passes; ++p) {
            const uint32_t d = (uint32_t)(k >> shift) & ((1u << pl.bits[p]) - 1u);
            atomicAdd(&s_h[p][d], 1u);
            shift += pl.bits[p];
          }
        }
      }
    }
  }
  if (kDepthKeys) {
    vis = wave_sum_u32(vis);
    if (lane_id() == 0 && vis) atomicAdd(&s_vis, vis);
  }
  // orders LDS only: the key stores stay in flight
  lds_barrier();
  for (int p = 0; p < pl.passes; ++p) {
    const uint32_t c = s_h[p][threadIdx.x];
    if (c) atomicAdd(&hist[p * 256 + threadIdx.x], c);
  }
  if (kDepthKeys && threadIdx.x == 0 && s_vis) atomicAdd(nvis, s_vis);
}

// Per-pass options of radix_pass_kernel (all off for a plain sort).
//  drop_ones: keys equal to all ones are not sorted; the pass writes the
//    others densely (the depth sort's first pass drops the culled Gaussians,
//    whose keys are all ones and which its histograms do not count).
//  n_dev: the number of keys in play, read on the device (at most n_max):
//    the passes after a dropping one, which the host sizes for n_max.
//  fill_tail: the last pass writes the sentinel pair (all-ones key, value
//    0xFFFFFFFF) at positions [n, n_max), so the output keeps n_max entries.
struct SortPassOpts {
  const uint32_t* n_dev;
  bool drop_ones;
  bool fill_tail;
};

// kT threads per workgroup, kT * kIt keys per chunk.  Digit-wise steps
// (histograms, offsets, look-back) run on the first 256 threads.  kBits: the
// digit width when fixed at compile time (8), else 0 (nbits at run time).
// status: [chunk][digit] words; gsum, gpre: [group][digit] words.
template <typename K, int kT, int kIt, int kBits>
__global__ void __launch_bounds__(kT)
radix_pass_kernel(const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                  K* __restrict__ keys_out, uint32_t* __restrict__ vals_out, int64_t n_max,
                  int shift, int nbits_rt, const uint32_t* __restrict__ hist, uint64_t* status,
                  uint64_t* gsum, uint64_t* gpre, int64_t nchunks, uint32_t* err,
                  uint32_t spin_limit, SortPassOpts opt) {
  static_assert(kBits == 0 || kBits == 8, "fixed digits are 8 bits wide");
  const int nbits = kBits ? kBits : nbits_rt;
  constexpr int kW = kT / kWave;
  constexpr int kC = kT * kIt;
  __shared__ uint32_t s_wh[kW][256];
  __shared__ uint32_t s_dstart[256];
  __shared__ uint32_t s_goff[256];
  __shared__ uint32_t s_tmp[kW + 1];
  __shared__ uint32_t s_tmp2[kW + 1];
  __shared__ uint32_t s_total;
  __shared__ K s_keys[kC];
  __shared__ uint32_t s_vals[kC];
  const int t = (int)threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  const uint32_t mask = (1u << nbits) - 1u;
  for (int i = t; i < kW * 256; i += kT) (&s_wh[0][0])[i] = 0;
  // the pass's global digit count, loaded now: its latency overlaps the
  // ticket, the key loads and the ranking
  const uint32_t gcount = (uint32_t)t <= mask ? hist[t] : 0u;
  // the keys in play: n_max, or fewer when an earlier pass dropped some
  int64_t n = n_max;
  if (opt.n_dev) {
    const int64_t nd = (int64_t)*opt.n_dev;
    n = nd < n_max ? nd : n_max;
  }
  // chunks in workgroup order: a chunk waits only on lower-numbered chunks,
  // which each XCD dispatches before it (the bounded waits are the backstop)
  const int64_t chunk = (int64_t)blockIdx.x;
  lds_barrier();  // the digit counters' clear
  if (opt.fill_tail) {
    // positions [n, n_max) get the sentinel pair (all-ones key, value)
    for (int64_t j = n + chunk * kC + t; j < n + (chunk + 1) * kC && j < n_max; j += kT) {
      keys_out[j] = (K)~(K)0;
      vals_out[j] = 0xFFFFFFFFu;
    }
  }
  if (chunk * kC >= n) return;  // uniform: no key of this chunk is in play
  const int64_t base = chunk * kC + (int64_t)w * (kC / kW);
  const uint64_t lt = lanemask_lt();
  K key[kIt];
  uint32_t val[kIt];
  uint32_t rank[kIt];
  bool vld[kIt];  // the item is a key in play (in range, not dropped)
  // Every load is issued before the first ranking step (indices past the end
  // are clamped to the last element, so the loads carry no branch); ranking
  // item by item through LDS would otherwise wait out one memory latency per
  // item.
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int64_t idx = base + it * kWave + lane;
    key[it] = keys_in[idx < n ? idx : n - 1];
  }
  if (vals_in) {  // uniform
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int64_t idx = base + it * kWave + lane;
      val[it] = vals_in[idx < n ? idx : n - 1];
    }
  } else {
#pragma unroll
    for (int it = 0; it < kIt; ++it) val[it] = (uint32_t)(base + it * kWave + lane);
  }
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int64_t idx = base + it * kWave + lane;
    const bool valid = idx < n && !(opt.drop_ones && key[it] == (K)~(K)0);
    vld[it] = valid;
    if (!valid) key[it] = (K)0;
    const uint32_t d = (uint32_t)(key[it] >> shift) & mask;
    uint64_t peers = __ballot(valid);
    if constexpr (kBits > 0) {
      peers = match_any_8(d, peers);
    } else {
      for (int b = 0; b < nbits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
    }
    const uint32_t r = (uint32_t)__popcll(peers & lt);
    uint32_t old = 0;
    if (valid) old = s_wh[w][d];
    if (valid && r == 0) s_wh[w][d] = old + (uint32_t)__popcll(peers);
    rank[it] = old + r;
  }
  // The pass's barriers order LDS only: its global stores (the sentinel tail,
  // the status words) stay in flight instead of being waited out at each
  // barrier, which the full __syncthreads() would do.
  lds_barrier();
  {
    const bool dig = (uint32_t)t <= mask;  // t < 256 as nbits <= 8
    uint32_t c[kW];
    uint32_t tot = 0;
#pragma unroll
    for (int k = 0; k < kW; ++k) {
      c[k] = dig ? s_wh[k][t] : 0u;
      tot += c[k];
    }
    uint64_t* st = status + (size_t)t;  // chunk-major: [chunk][digit]
    // the chunk's digit counts are published before the scans, so that the
    // look-backs of later chunks can pass this one sooner
    const int64_t g = chunk / kLbGroup;
    const int q = (int)(chunk - g * kLbGroup);
    uint64_t* gs = gsum + (size_t)t;
    uint64_t* gp = gpre + (size_t)t;
    if (dig) {
      status_store(st + chunk * 256, kFlagAggregate, tot);
      // the chunk's counts join its group's running word
      __hip_atomic_fetch_add(gs + g * 256, (1ull << 32) | (uint64_t)tot, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
    // both exclusive scans (global digit bases, chunk digit starts) at once
    uint32_t gbase, ds, total;
    {
      const uint32_t ia = wave_incl_scan(gcount), ib = wave_incl_scan(tot);
      if (lane == kWave - 1) {
        s_tmp[w] = ia;
        s_tmp2[w] = ib;
      }
      lds_barrier();
      if (w == 0) {
        const uint32_t xa = lane < kW ? s_tmp[lane] : 0u, xb = lane < kW ? s_tmp2[lane] : 0u;
        const uint32_t ya = wave_incl_scan(xa), yb = wave_incl_scan(xb);
        if (lane < kW) {
          s_tmp[lane] = ya - xa;
          s_tmp2[lane] = yb - xb;
        }
        if (lane == kW - 1) s_tmp2[kW] = yb;
      }
      lds_barrier();
      gbase = s_tmp[w] + ia - gcount;
      ds = s_tmp2[w] + ib - tot;
      total = s_tmp2[kW];
    }
    if (t == 0) s_total = total;
    if (t < 256) {
      uint32_t run = ds;
#pragma unroll
      for (int k = 0; k < kW; ++k) {
        s_wh[k][t] = run;
        run += c[k];
      }
      s_dstart[t] = ds;
    }
    lds_barrier();
    // the chunk in digit order in LDS (chunk-local positions), before the
    // look-back: its time overlaps the predecessors' publishing, and the
    // keys' registers are free during the wait
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      if (vld[it]) {
        const uint32_t d = (uint32_t)(key[it] >> shift) & mask;
        const uint32_t pos = s_wh[w][d] + rank[it];
        s_keys[pos] = key[it];
        s_vals[pos] = val[it];
      }
    }
    if (dig) {
      // Two-level offsets: the chunk's predecessors in its group of
      // kLbGroup chunks are summed directly; the earlier groups come from
      // their running words and the prefixes the groups' last chunks publish.
      uint32_t in_group, gexcl;
      chunk_offsets(st, g * kLbGroup, q, gs, gp, g, 256, err, spin_limit, in_group, gexcl);
      if (q == kLbGroup - 1) status_store(gp + g * 256, kFlagPrefix, gexcl + in_group + tot);
      const uint32_t excl = gexcl + in_group;
      s_goff[t] = gbase + excl;
    }
  }
  lds_barrier();
  const int cnt = (int)s_total;  // the chunk's keys in play (all of them unless dropped)
  for (int j = t; j < cnt; j += kT) {
    const K k = s_keys[j];
    const uint32_t d = (uint32_t)(k >> shift) & mask;
    const uint32_t g = s_goff[d] + ((uint32_t)j - s_dstart[d]);
    // always below n unless an earlier wait gave up and left this pass keys
    // the digit histogram did not count
    if ((int64_t)g < n) {
      keys_out[g] = k;
      vals_out[g] = s_vals[j];
    }
  }
}

// Radix passes run kSortT threads per workgroup and sort_items(n) keys per
// thread: large sorts take big chunks (fewer chunks to look back over), small
// ones smaller chunks so that more workgroups share the ranking.
constexpr int kSortT = 512;
// At 1M keys 8 items per thread measured about 21 us per pass (binning
// 295-298 us against 299-301 with 16 items, 27.1 us per pass with 4); at 200k
// keys 4 items measured 13.4 us against 17.4 for 16.
constexpr int64_t kSortSmallN = 393216;
static int sort_items(int64_t n) { return n > kSortSmallN ? 8 : 4; }
static int64_t sort_chunks(int64_t n) {
  const int64_t c = (int64_t)kSortT * sort_items(n);
  return (n + c - 1) / c;
}

// Zero-initialised state of one sort: histograms (8 x 256), eight reserved
// words, the error word, the visible-key count of a depth sort, then the
// status words of every pass (per chunk), then the running words of the
// look-back groups of every pass, then their prefix words.
static size_t sort_state_bytes(int64_t n, int passes) {
  const int64_t nc = sort_chunks(n);
  const int64_t ng = (nc + kLbGroup - 1) / kLbGroup;
  return (size_t)((8 * 256 * 4 + 64 + (int64_t)passes * ((nc < 1 ? 1 : nc) + 2 * ng) * 256 * 8 +
                   255) &
                  ~(int64_t)255);
}

// The error word inside a sort workspace (tmp keys, tmp values, then the state:
// histograms, eight reserved words, error word).
template <typename K>
static uint32_t* sort_err_word(void* ws, int64_t n) {
  char* p = (char*)ws;
  p += ((size_t)n * sizeof(K) + 255) & ~(size_t)255;
  p += ((size_t)n * 4 + 255) & ~(size_t)255;
  return (uint32_t*)(p + 8 * 256 * 4) + 8;
}

template <typename K>
static size_t sort_ws_bytes(int64_t n, int passes = (int)sizeof(K)) {
  size_t b = 0;
  b += ((size_t)n * sizeof(K) + 255) & ~(size_t)255;  // tmp keys
  b += ((size_t)n * 4 + 255) & ~(size_t)255;          // tmp vals
  b += sort_state_bytes(n, passes);
  return b;
}

// Stable sort on bits [begin, end).  vals_in may be NULL (values = index).
// keys_in/vals_in are not modified.  kDepthKeys: keys_in is ignored and the
// keys are made from depths / tiles_touched (written to dkeys_out).
template <typename K, bool kDepthKeys = false>
static int32_t radix_sort_pairs(const K* keys_in, const uint32_t* vals_in, K* keys_out,
                                uint32_t* vals_out, int64_t n, int begin, int end, void* ws,
                                hipStream_t st, const float* depths = nullptr,
                                const uint32_t* tiles_touched = nullptr,
                                uint32_t* dkeys_out = nullptr, uint32_t* werr = nullptr) {
  if (n <= 0) {
    if (werr) launch_fill(werr, 0u, 1, st);
    return FGS_OK;
  }
  const SortPlan pl = sort_plan(begin, end);
  // depth keys drop the culled Gaussians in pass 0 (which runs on all n) and
  // fill the sentinel tail in the last pass over the visible count, so they
  // need two distinct passes; their histogram kernel counts the four 8-bit
  // digits of a 32-bit key
  if (kDepthKeys && (begin != 0 || end != 32 || pl.passes != 4))
    return set_error(FGS_ERR_UNSUPPORTED, "radix_sort_pairs: depth keys take 32 bits from bit 0");
  if (pl.passes == 0) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(copy_pairs_kernel<K>, dim3((unsigned)blocks), dim3(256), 0, st, keys_in,
                       vals_in, keys_out, vals_out, n);
    if (werr) launch_fill(werr, 0u, 1, st);
    return check_launch("copy_pairs");
  }
  const int64_t nc = sort_chunks(n);
  const int items = sort_items(n);
  char* p = (char*)ws;
  K* tk = (K*)p;
  p += ((size_t)n * sizeof(K) + 255) & ~(size_t)255;
  uint32_t* tv = (uint32_t*)p;
  p += ((size_t)n * 4 + 255) & ~(size_t)255;
  uint32_t* hist = (uint32_t*)p;
  uint32_t* words = hist + 8 * 256;  // eight reserved words, the error word, the count
  uint32_t* err = werr ? werr : words + 8;
  uint64_t* status = (uint64_t*)(p + 8 * 256 * 4 + 64);
  const int64_t ngr = (nc + kLbGroup - 1) / kLbGroup;
  uint64_t* gsum = status + (size_t)pl.passes * nc * 256;
  uint64_t* gpre = gsum + (size_t)pl.passes * ngr * 256;
  {
    FillSpans f{};
    f.value = 0u;
    f.p[0] = hist;
    f.n[0] = (int64_t)(sort_state_bytes(n, pl.passes) / 4);
    f.count = 1;
    if (werr) {
      f.p[1] = werr;
      f.n[1] = 1;
      f.count = 2;
    }
    launch_fill_spans(f, st);
  }
  const uint32_t spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  const int64_t hn = (n + kChunk - 1) / kChunk;  // histogram workgroups: 4096 keys each
  const int64_t hb = hn < 1024 ? hn : 1024;
  // the depth sort's visible-key count, in the zeroed state
  uint32_t* nvis = words + 10;
  hipLaunchKernelGGL((radix_hist_kernel<K, kDepthKeys>), dim3((unsigned)hb), dim3(kThreads), 0, st,
                     keys_in, n, pl, hist, depths, tiles_touched, dkeys_out, nvis);
  const K* src_k = kDepthKeys ? (const K*)dkeys_out : keys_in;
  const uint32_t* src_v = vals_in;
  int shift = begin;
  for (int pass = 0; pass < pl.passes; ++pass) {
    const bool to_out = ((pl.passes - 1 - pass) % 2) == 0;
    K* dk = to_out ? keys_out : tk;
    uint32_t* dv = to_out ? vals_out : tv;
    // depth keys: the culled Gaussians (all-ones keys) leave in the first
    // pass; the later passes sort the visible ones, and the last fills the
    // tail with sentinels
    SortPassOpts opt{};
    if (kDepthKeys) {
      opt.drop_ones = pass == 0;
      opt.n_dev = pass > 0 ? nvis : nullptr;
      opt.fill_tail = pass == pl.passes - 1;
    }
    uint64_t* const ps = status + (size_t)pass * nc * 256;
    uint64_t* const pgs = gsum + (size_t)pass * ngr * 256;
    uint64_t* const pgp = gpre + (size_t)pass * ngr * 256;
    const int nb = pl.bits[pass];
    if (items == 8 && nb == 8)
      hipLaunchKernelGGL((radix_pass_kernel<K, kSortT, 8, 8>), dim3((unsigned)nc), dim3(kSortT), 0,
                         st, src_k, src_v, dk, dv, n, shift, nb, hist + pass * 256, ps, pgs, pgp,
                         nc, err, spin_limit, opt);
    else if (items == 8)
      hipLaunchKernelGGL((radix_pass_kernel<K, kSortT, 8, 0>), dim3((unsigned)nc), dim3(kSortT), 0,
                         st, src_k, src_v, dk, dv, n, shift, nb, hist + pass * 256, ps, pgs, pgp,
                         nc, err, spin_limit, opt);
    else if (nb == 8)
      hipLaunchKernelGGL((radix_pass_kernel<K, kSortT, 4, 8>), dim3((unsigned)nc), dim3(kSortT), 0,
                         st, src_k, src_v, dk, dv, n, shift, nb, hist + pass * 256, ps, pgs, pgp,
                         nc, err, spin_limit, opt);
    else
      hipLaunchKernelGGL((radix_pass_kernel<K, kSortT, 4, 0>), dim3((unsigned)nc), dim3(kSortT), 0,
                         st, src_k, src_v, dk, dv, n, shift, nb, hist + pass * 256, ps, pgs, pgp,
                         nc, err, spin_limit, opt);
    const int32_t e2 = check_launch("radix_pass");
    if (e2 != FGS_OK) return e2;
    shift += pl.bits[pass];
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
  if (g >= (uint32_t)P) return;
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
// Tile ids >= T and Gaussian indices >= P are never used as addresses.
__global__ void finalize_keys_ranges_kernel(int64_t K, int32_t T, int32_t P,
                                            const uint32_t* __restrict__ tiles,
                                            const uint32_t* __restrict__ point_list,
                                            const float* __restrict__ depths,
                                            uint64_t* __restrict__ keys64,
                                            uint32_t* __restrict__ ranges) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= K) return;
  const uint32_t cur = tiles[i];
  const uint32_t g = point_list[i];
  const uint32_t db = g < (uint32_t)P ? __float_as_uint(depths[g]) : 0xFFFFFFFFu;
  keys64[i] = ((uint64_t)cur << 32) | (uint64_t)db;
  if (i > 0) {
    const uint32_t prev = tiles[i - 1];
    if (cur != prev) {
      if (prev < (uint32_t)T) ranges[2 * (size_t)prev + 1] = (uint32_t)i;
      if (cur < (uint32_t)T) ranges[2 * (size_t)cur] = (uint32_t)i;
    }
  }
  if (i == K - 1 && cur < (uint32_t)T) ranges[2 * (size_t)cur + 1] = (uint32_t)K;
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

// The wait status of a binning call: the OR of the error words of the waits it
// (and the depth order it consumes) ran, written by the call's last kernel
// (one workgroup, after every wait in stream order).  Unused words are NULL.
struct WaitWords {
  const uint32_t* w[3];
  uint32_t* out;
  uint64_t* host;  // NULL, or host memory for (status << 32) | B
};
// The OR of the waits' words (thread 0; 0 elsewhere), written to ww.out.
__device__ __forceinline__ uint32_t report_waits(const WaitWords& ww) {
  uint32_t v = 0u;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (ww.w[k]) v |= __hip_atomic_load(ww.w[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (ww.out) *ww.out = v;
  }
  return v;
}
// Thread 0: the wait status and B to the caller's host word, as one 64-bit
// store at system scope (it reaches host memory as one write, so the host,
// polling the word, sees both halves together).
__device__ __forceinline__ void report_host(const WaitWords& ww, uint32_t status, uint32_t B) {
  if (threadIdx.x == 0 && ww.host)
    __hip_atomic_store(ww.host, ((uint64_t)status << 32) | (uint64_t)B, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

// Bucket counts (ceil(n / 32) per tile) and their inclusive scan, by one
// 1024-thread workgroup walking the tiles in chunks of 1024.
__global__ void __launch_bounds__(1024)
bucket_scan_kernel(int32_t T, const uint32_t* __restrict__ ranges,
                   uint32_t* __restrict__ bucket_count, uint32_t* __restrict__ bucket_offsets,
                   WaitWords ww) {
  __shared__ uint32_t s_tmp[1024 / kWave + 1];
  const uint32_t status = report_waits(ww);
  uint32_t carry = 0;
  for (int base = 0; base < T; base += 1024) {
    const int t = base + (int)threadIdx.x;
    uint32_t c = 0;
    if (t < T) {
      const int n = (int)(ranges[2 * t + 1] - ranges[2 * t]);
      c = (uint32_t)((n + 31) / 32);
      bucket_count[t] = c;
    }
    uint32_t total;
    const uint32_t ex = block_excl_scan(c, s_tmp, &total);
    if (t < T) bucket_offsets[t] = carry + ex + c;
    carry += total;
  }
  report_host(ww, status, carry);
}

// ---------------------------------------------------------------------------
// Two-level tile binning (grids of at most 256 super-tiles).
//
// The tiles are grouped into super-tiles of 8x8.  Level 1 lists, for every
// super-tile, the Gaussians whose walk touches it, in depth order (a stable
// partition of the depth-sorted Gaussians: per-workgroup counts, a scan, then
// ranks by ballots).  Level 2 cuts each list into chunks of 512 and, per
// entry, walks the Gaussian inside the super-tile window to get its 64-bit
// tile mask; per-tile counts -> per-tile starts (ranges) -> every entry's
// position = tile start + entries of that tile in earlier chunks + rank in
// the chunk (ballots in list order).  A tile's entries therefore come out in
// (depth bits, index) order and are written straight to point_list and
// point_list_keys: no K-sized sort.
// ---------------------------------------------------------------------------
constexpr int kSt = 8;          // super-tile edge in tiles
constexpr int kMaxSt = 256;     // super-tiles of the two-level path
constexpr int kL1Group = 256;   // level-1 Gaussians per workgroup
constexpr int kL1Segs = 64;     // level-1 row segments of the count scan
constexpr int kL2Chunk = 512;   // level-2 entries per workgroup (4 wavefronts x 128)
constexpr int kL2EmitGrid = 4096;  // workgroups of l2_count and l2_emit at most (chunk loops)
constexpr int kScanBatch = 32;    // loads in flight per serial-scan batch

struct StGrid {
  int gx, gy, sgx, sgy, S;
};

// Level 1: the set of super-tiles a Gaussian's walk touches (256 bits).
struct EmitStSet {
  uint64_t m[4];
  int sgx;
  __device__ __forceinline__ void set_bit(int b) { m[b >> 6] |= 1ull << (b & 63); }
  __device__ __forceinline__ void set_range(int lo, int hi) {  // inclusive
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int a = imax(lo, 64 * w), z = imin(hi, 64 * w + 63);
      if (z < a) continue;
      const int n = z - a + 1;
      const uint64_t bits = (n >= 64) ? ~0ull : ((1ull << n) - 1ull);
      m[w] |= bits << (a - 64 * w);
    }
  }
  __device__ __forceinline__ void operator()(int u, int vmin, int vmax, bool is_y) {
    const int b = u / kSt;
    const int c0 = vmin / kSt, c1 = (vmax - 1) / kSt;
    if (is_y) {  // row u, columns [vmin, vmax): contiguous super-tile ids
      set_range(b * sgx + c0, b * sgx + c1);
    } else {  // column u, rows [vmin, vmax)
      for (int c = c0; c <= c1; ++c) set_bit(c * sgx + b);
    }
  }
};

// Level 2: 64-bit mask of the tiles of one super-tile window (bit
// (y - y0) * 8 + (x - x0)).  The walk is clipped to the window on its own
// axis; spans are clipped here on the other.
struct EmitTileMask {
  uint64_t m;
  int x0, y0;
  __device__ __forceinline__ void operator()(int u, int vmin, int vmax, bool is_y) {
    if (is_y) {
      const int xs = imax(vmin, x0), xe = imin(vmax, x0 + kSt);
      if (xe > xs) m |= ((1ull << (xe - xs)) - 1ull) << ((u - y0) * kSt + (xs - x0));
    } else {
      const int ys = imax(vmin, y0), ye = imin(vmax, y0 + kSt);
      if (ye > ys) {
        const uint64_t hi = (ye - y0 >= kSt) ? ~0ull : ((1ull << (kSt * (ye - y0))) - 1ull);
        const uint64_t lo = (1ull << (kSt * (ys - y0))) - 1ull;
        m |= (hi & ~lo) & (0x0101010101010101ull << (u - x0));
      }
    }
  }
};

__device__ __forceinline__ bool st_has(const uint64_t (&m)[4], int s) {
  return (m[s >> 6] >> (s & 63)) & 1ull;
}

// Super-tile of mask k of record word w; a record made for another grid can
// give ids >= S, which both level-1 kernels skip.
__device__ __forceinline__ int rec_st(uint32_t w, int k, const StGrid& sg) {
  const int bx = (int)(w & 0xFFFu) + (k & 1), by = (int)((w >> 12) & 0xFFFu) + (k >> 1);
  return (bx < sg.sgx && by < sg.sgy) ? by * sg.sgx + bx : kMaxSt;
}

// Level 1a: per depth-ordered Gaussian its super-tiles, and per workgroup
// the number of its Gaussians touching each super-tile.  The preprocess
// record (word != 0) gives either four super-tile masks (fits, or compact:
// one 8x8 board expanded here) or the 256-bit super-tile set (the masks and
// the set are gathered from st_masks; a compact record is its 16 bytes
// alone); a Gaussian without one walks its tiles into the
// set.  Stored in depth order for l1_place: recw[i] (the record word; 0 or
// kStRecSet mean a set) and sets[4i..4i+3] (the masks, or the set).
__global__ void __launch_bounds__(kL1Group)
l1_count_kernel(int32_t P, StGrid sg, float mult, const uint32_t* __restrict__ order,
                const uint32_t* __restrict__ nvis, const float* __restrict__ xys,
                const float* __restrict__ conic_opacity,
                const uint32_t* __restrict__ tiles_touched, const uint32_t* __restrict__ st_rec,
                const uint64_t* __restrict__ st_masks, uint32_t* __restrict__ recw,
                uint64_t* __restrict__ sets, uint32_t* __restrict__ cnt1) {
  __shared__ uint32_t s_cnt[kMaxSt];
  const int t = (int)threadIdx.x;
  const int i = (int)blockIdx.x * kL1Group + t;
  s_cnt[t] = 0;
  uint64_t m[4] = {0ull, 0ull, 0ull, 0ull};
  uint32_t w = 0u;
  // entries from the visible count on are the sort's sentinel tail (culled
  // Gaussians): nothing to read, and l1_place does not read them back
  const int nv = nvis ? (int)min((uint32_t)P, *nvis) : P;
  if (i < nv) {
    const uint32_t g = order[i];
    if (g < (uint32_t)P) {
      uint4 rec = make_uint4(0u, 0u, 0u, 0u);
      if (st_rec) rec = reinterpret_cast<const uint4*>(st_rec)[g];
      w = rec.x;
      if (w & kStRecCompact) {  // the board alone: back to the fits form
        const uint32_t x0 = w & 0xFFFu, y0 = (w >> 12) & 0xFFFu;
        st_expand_compact((uint64_t)rec.z | ((uint64_t)rec.w << 32), (int)(x0 & 7u),
                          (int)(y0 & 7u), m);
        w = (x0 >> 3) | ((y0 >> 3) << 12) | kStRecFits;
      } else if (w != 0u) {
        const uint4* src = reinterpret_cast<const uint4*>(st_masks + 4 * (size_t)g);
        const uint4 a = src[0], b = src[1];
        m[0] = (uint64_t)a.x | ((uint64_t)a.y << 32);
        m[1] = (uint64_t)a.z | ((uint64_t)a.w << 32);
        m[2] = (uint64_t)b.x | ((uint64_t)b.y << 32);
        m[3] = (uint64_t)b.z | ((uint64_t)b.w << 32);
      } else if (tiles_touched[g] != 0u) {
        EmitStSet e;
        e.m[0] = e.m[1] = e.m[2] = e.m[3] = 0ull;
        e.sgx = sg.sgx;
        const float2 xy = *reinterpret_cast<const float2*>(xys + 2 * (size_t)g);
        const float4 co = *reinterpret_cast<const float4*>(conic_opacity + 4 * (size_t)g);
        tiles_walk(xy.x, xy.y, co, sg.gx, sg.gy, mult, e);
#pragma unroll
        for (int k = 0; k < 4; ++k) m[k] = e.m[k];
      }
    }
    recw[i] = w;
    uint4* dst = reinterpret_cast<uint4*>(sets + 4 * (size_t)i);
    dst[0] = make_uint4((uint32_t)m[0], (uint32_t)(m[0] >> 32), (uint32_t)m[1],
                        (uint32_t)(m[1] >> 32));
    dst[1] = make_uint4((uint32_t)m[2], (uint32_t)(m[2] >> 32), (uint32_t)m[3],
                        (uint32_t)(m[3] >> 32));
  }
  __syncthreads();
  if (w & kStRecFits) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int sid = rec_st(w, k, sg);
      if (m[k] != 0ull && sid < sg.S) atomicAdd(&s_cnt[sid], 1u);
    }
  } else {
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      uint64_t b = m[wd];
      if (64 * (wd + 1) > sg.S) b &= (64 * wd >= sg.S) ? 0ull : ((1ull << (sg.S - 64 * wd)) - 1ull);
      while (b) {
        const int k = __builtin_ctzll(b);
        b &= b - 1ull;
        atomicAdd(&s_cnt[64 * wd + k], 1u);
      }
    }
  }
  __syncthreads();
  if (t < sg.S) cnt1[(size_t)blockIdx.x * sg.S + t] = s_cnt[t];
}

// Level 1b: exclusive prefix of cnt1 over the workgroups of each of kL1Segs
// row segments (in place), and each segment's totals.
__global__ void __launch_bounds__(kMaxSt)
l1_seg_scan_kernel(int nwg, int S, uint32_t* __restrict__ cnt1, uint32_t* __restrict__ segsum) {
  const int s = (int)threadIdx.x;
  if (s >= S) return;
  const int rows = (nwg + kL1Segs - 1) / kL1Segs;
  const int r0 = (int)blockIdx.x * rows, r1 = imin(nwg, r0 + rows);
  uint32_t run = 0;
  for (int r = r0; r < r1; r += kScanBatch) {
    // the batch's loads are all issued before its first store
    uint32_t v[kScanBatch];
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) v[i] = r + i < r1 ? cnt1[(size_t)(r + i) * S + s] : 0u;
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) {
      if (r + i < r1) cnt1[(size_t)(r + i) * S + s] = run;
      run += v[i];
    }
  }
  segsum[(size_t)blockIdx.x * S + s] = run;
}

// Level 1c (one workgroup): segment prefixes, list starts st_start[0..S], the
// level-2 chunk table (chunk_first[0..S], chunk_st[c]) and the chunk count.
__global__ void __launch_bounds__(kMaxSt)
l1_top_scan_kernel(int S, uint32_t* __restrict__ segsum, uint32_t* __restrict__ st_start,
                   uint32_t* __restrict__ chunk_first, uint32_t* __restrict__ chunk_st,
                   uint32_t* __restrict__ nchunks, int64_t max_chunks) {
  __shared__ uint32_t s_tmp[kMaxSt / kWave + 1];
  const int s = (int)threadIdx.x;
  uint32_t run = 0;
  if (s < S) {
    for (int g0 = 0; g0 < kL1Segs; g0 += kScanBatch) {
      uint32_t v[kScanBatch];
#pragma unroll
      for (int i = 0; i < kScanBatch; ++i) v[i] = segsum[(size_t)(g0 + i) * S + s];
#pragma unroll
      for (int i = 0; i < kScanBatch; ++i) {
        segsum[(size_t)(g0 + i) * S + s] = run;
        run += v[i];
      }
    }
  }
  uint32_t total;
  const uint32_t start = block_excl_scan(s < S ? run : 0u, s_tmp, &total);
  const uint32_t nch = s < S ? (run + kL2Chunk - 1) / kL2Chunk : 0u;
  uint32_t ctotal;
  const uint32_t cfirst = block_excl_scan(nch, s_tmp, &ctotal);
  if (s < S) {
    st_start[s] = start;
    chunk_first[s] = cfirst;
    for (uint32_t k = 0; k < nch; ++k)
      if ((int64_t)(cfirst + k) < max_chunks) chunk_st[cfirst + k] = (uint32_t)s;
  }
  if (s == 0) {
    st_start[S] = total;
    chunk_first[S] = ctotal;
    nchunks[0] = (int64_t)ctotal < max_chunks ? ctotal : (uint32_t)max_chunks;
  }
}

// Level 1d: each Gaussian written into the lists of its super-tiles, with
// its 64-bit tile mask there.  The workgroup's (Gaussian, super-tile, mask)
// triples are laid out in LDS in thread order (a thread's super-tiles are
// distinct, so their order among themselves is free) and ranked per
// super-tile in that order, 256 at a time: wave64 match-any over the 8
// super-tile bits, then the four waves through LDS counters, as in a radix
// pass.  A record's masks are written as they are.  The pairs of a Gaussian
// given by its super-tile set (a wide one) carry no mask: the workgroup
// collects them in LDS and, after its last round, walks each one clipped to
// its super-tile's window, one pair per thread, so the few walks run side by
// side (beyond kL1Wide pairs, the thread that places a pair walks it).
constexpr int kL1Pairs = 1024;  // LDS pair capacity per round
constexpr int kL1Wide = 256;    // wide pairs a workgroup collects before walking them

// The tile mask of Gaussian g in super-tile sid: its walk clipped to the
// super-tile's 8x8-tile window.
__device__ __forceinline__ uint64_t wide_pair_mask(const StGrid& sg, float mult,
                                                   const float* __restrict__ xys,
                                                   const float* __restrict__ conic_opacity,
                                                   uint32_t g, int sid) {
  EmitTileMask em;
  em.m = 0ull;
  em.x0 = (sid % sg.sgx) * kSt;
  em.y0 = (sid / sg.sgx) * kSt;
  const float2 xy = *reinterpret_cast<const float2*>(xys + 2 * (size_t)g);
  const float4 co = *reinterpret_cast<const float4*>(conic_opacity + 4 * (size_t)g);
  tiles_walk_window(xy.x, xy.y, co, sg.gx, sg.gy, mult, em.x0, em.x0 + kSt, em.y0, em.y0 + kSt,
                    em);
  return em.m;
}
template <bool kCarry>
__global__ void __launch_bounds__(kL1Group)
l1_place_kernel(int32_t P, StGrid sg, const uint32_t* __restrict__ order,
                const uint32_t* __restrict__ nvis,
                const uint32_t* __restrict__ skeys, const uint32_t* __restrict__ recw,
                const uint64_t* __restrict__ sets, const uint32_t* __restrict__ cnt1,
                const uint32_t* __restrict__ segsum, const uint32_t* __restrict__ st_start,
                int64_t cap, uint32_t* __restrict__ list, uint64_t* __restrict__ masks,
                uint32_t* __restrict__ ldb, float mult, const float* __restrict__ xys,
                const float* __restrict__ conic_opacity) {
  __shared__ uint64_t s_pm[kL1Pairs];  // mask of each pair (0: walk it)
  __shared__ uint32_t s_wpos[kL1Wide];  // wide pairs: list position
  __shared__ uint32_t s_wg[kL1Wide];    // its Gaussian
  __shared__ uint8_t s_wd[kL1Wide];     // and super-tile
  __shared__ uint32_t s_nw;
  __shared__ uint32_t s_pg[kL1Pairs];  // Gaussian of each pair
  __shared__ uint32_t s_pd[kCarry ? kL1Pairs : 1];  // kCarry: its depth bits (sorted key)
  __shared__ uint8_t s_ps[kL1Pairs];   // super-tile of each pair
  __shared__ uint32_t s_wh[kWavesPerBlock][kMaxSt];
  __shared__ uint32_t s_base[kMaxSt];
  __shared__ uint32_t s_tmp[kWavesPerBlock + 1];
  const int S = sg.S;
  const int t = (int)threadIdx.x;
  const int w = t / kWave;
  const int i = (int)blockIdx.x * kL1Group + t;
  if (t == 0) s_nw = 0u;  // ordered before its use by the barriers of the scan below
  uint64_t m[4] = {0ull, 0ull, 0ull, 0ull};
  uint32_t g = 0, rw = 0, db = 0;
  // the sentinel tail from the visible count on was not written by l1_count
  const int nv = nvis ? (int)min((uint32_t)P, *nvis) : P;
  if (i < nv) {
    const uint4* src = reinterpret_cast<const uint4*>(sets + 4 * (size_t)i);
    const uint4 a = src[0], b = src[1];
    m[0] = (uint64_t)a.x | ((uint64_t)a.y << 32);
    m[1] = (uint64_t)a.z | ((uint64_t)a.w << 32);
    m[2] = (uint64_t)b.x | ((uint64_t)b.y << 32);
    m[3] = (uint64_t)b.z | ((uint64_t)b.w << 32);
    g = order[i];
    rw = recw[i];
    if (kCarry) db = skeys[i];
  }
  const int rows = (int)((gridDim.x + kL1Segs - 1) / kL1Segs);
  const int seg = (int)blockIdx.x / rows;
  if (t < S)
    s_base[t] = st_start[t] + segsum[(size_t)seg * S + t] + cnt1[(size_t)blockIdx.x * S + t];
  const bool fits = (rw & kStRecFits) != 0u;
  uint32_t np = 0;
  if (fits) {
#pragma unroll
    for (int k = 0; k < 4; ++k) np += (m[k] != 0ull && rec_st(rw, k, sg) < S) ? 1u : 0u;
  } else {
#pragma unroll
    for (int wd = 0; wd < 4; ++wd)  // super-tile ids >= S are never set; clear them anyway
      if (64 * (wd + 1) > S) m[wd] &= (64 * wd >= S) ? 0ull : ((1ull << (S - 64 * wd)) - 1ull);
    np = (uint32_t)(__popcll(m[0]) + __popcll(m[1]) + __popcll(m[2]) + __popcll(m[3]));
  }
  uint32_t total;
  const uint32_t off = block_excl_scan(np, s_tmp, &total);  // has barriers
  const uint64_t lt = lanemask_lt();
  for (uint32_t r0 = 0; r0 < total; r0 += kL1Pairs) {
    // this round's pairs into LDS
    uint32_t p = off;
    if (fits) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int sid = rec_st(rw, k, sg);
        if (m[k] == 0ull || sid >= S) continue;
        if (p >= r0 && p < r0 + kL1Pairs) {
          s_ps[p - r0] = (uint8_t)sid;
          s_pg[p - r0] = g;
          if (kCarry) s_pd[p - r0] = db;
          s_pm[p - r0] = m[k];
        }
        ++p;
      }
    } else {
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        uint64_t b = m[wd];
        while (b) {
          const int k = __builtin_ctzll(b);
          b &= b - 1ull;
          if (p >= r0 && p < r0 + kL1Pairs) {
            s_ps[p - r0] = (uint8_t)(64 * wd + k);
            s_pg[p - r0] = g;
            if (kCarry) s_pd[p - r0] = db;
            s_pm[p - r0] = 0ull;
          }
          ++p;
        }
      }
    }
    __syncthreads();
    const uint32_t rn = (total - r0) < (uint32_t)kL1Pairs ? (total - r0) : (uint32_t)kL1Pairs;
    for (uint32_t q0 = 0; q0 < rn; q0 += kL1Group) {
#pragma unroll
      for (int k = 0; k < kWavesPerBlock; ++k) s_wh[k][t] = 0u;
      __syncthreads();
      const uint32_t q = q0 + (uint32_t)t;
      const bool valid = q < rn;
      const uint32_t d = valid ? s_ps[q] : 0u;
      const uint64_t peers = match_any_8(d, __ballot(valid));
      const uint32_t rk = (uint32_t)__popcll(peers & lt);
      if (valid && rk == 0) s_wh[w][d] = (uint32_t)__popcll(peers);
      __syncthreads();
      if (valid) {
        uint32_t pos = s_base[d] + rk;
        for (int k = 0; k < w; ++k) pos += s_wh[k][d];
        if ((int64_t)pos < cap) {
          const uint32_t g = s_pg[q];
          const uint64_t pm = s_pm[q];
          list[pos] = g;
          if (kCarry) ldb[pos] = s_pd[q];
          if (pm != 0ull || g >= (uint32_t)P) {
            masks[pos] = pm;
          } else {  // a wide pair: its mask is walked below (here, if the list is full)
            const uint32_t k = atomicAdd(&s_nw, 1u);
            if (k < (uint32_t)kL1Wide) {
              s_wpos[k] = pos;
              s_wg[k] = g;
              s_wd[k] = (uint8_t)d;
            } else {
              masks[pos] = wide_pair_mask(sg, mult, xys, conic_opacity, g, (int)d);
            }
          }
        }
      }
      __syncthreads();
      if (t < S) s_base[t] += s_wh[0][t] + s_wh[1][t] + s_wh[2][t] + s_wh[3][t];
      __syncthreads();
    }
  }
  // the workgroup's wide pairs, one walk per thread, side by side
  const uint32_t nw = s_nw < (uint32_t)kL1Wide ? s_nw : (uint32_t)kL1Wide;
  for (uint32_t k = (uint32_t)t; k < nw; k += kL1Group) {
    masks[s_wpos[k]] = wide_pair_mask(sg, mult, xys, conic_opacity, s_wg[k], (int)s_wd[k]);
  }
}

// Transpose of the 64x64 bit matrix whose row l is lane l's value: lane j
// returns column j (bit i = bit j of lane i's value).  Blocks of 32, 16, ...,
// 1 bits are exchanged with lane ^ d; each lane sends only the half of a
// block that moves.
__device__ __forceinline__ uint64_t transpose64(uint64_t row) {
  const int l = lane_id();
  uint32_t lo = (uint32_t)row, hi = (uint32_t)(row >> 32);
  {
    const bool up = (l & 32) != 0;
    const uint32_t recv = (uint32_t)__shfl_xor((int)(up ? lo : hi), 32);
    if (up) lo = recv;
    else hi = recv;
  }
  // the five steps written out (inside a loop over chunks the unroll pragma
  // was not applied)
  auto step = [&](const int d, const uint32_t m) {
    const bool up = (l & d) != 0;
    const uint32_t rl = (uint32_t)__shfl_xor((int)(up ? (lo & m) : (lo & ~m)), d);
    const uint32_t rh = (uint32_t)__shfl_xor((int)(up ? (hi & m) : (hi & ~m)), d);
    lo = up ? ((lo & ~m) | (rl >> d)) : ((lo & m) | (rl << d));
    hi = up ? ((hi & ~m) | (rh >> d)) : ((hi & m) | (rh << d));
  };
  step(16, 0x0000FFFFu);
  step(8, 0x00FF00FFu);
  step(4, 0x0F0F0F0Fu);
  step(2, 0x33333333u);
  step(1, 0x55555555u);
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

// Level 2b: per chunk of 512 entries of one super-tile list (four
// wavefronts, 128 entries each), the number of entries per tile.  Workgroups
// take chunks c = blockIdx.x, blockIdx.x + gridDim.x, ... up to the chunk
// count on the device.
__global__ void __launch_bounds__(kL1Group)
l2_count_kernel(const uint32_t* __restrict__ st_start, const uint32_t* __restrict__ chunk_first,
                const uint32_t* __restrict__ chunk_st, const uint32_t* __restrict__ nchunks,
                int64_t cap, const uint64_t* __restrict__ masks, uint32_t* __restrict__ cnt2) {
  __shared__ uint32_t s_wc[kWavesPerBlock][kWave];
  const uint32_t nch = nchunks[0];
  const int t = (int)threadIdx.x, w = t / kWave, l = lane_id();
  for (uint32_t c = blockIdx.x; c < nch; c += gridDim.x) {
    const uint32_t s = chunk_st[c];
    const uint32_t e0 = st_start[s] + (c - chunk_first[s]) * kL2Chunk;
    const uint32_t e1 = (uint32_t)imin(imin((int)st_start[s + 1], (int)(e0 + kL2Chunk)), (int)cap);
    uint32_t cnt = 0;
    const uint32_t q0 = e0 + (uint32_t)w * (kL2Chunk / kWavesPerBlock);
    const uint32_t q1 = (uint32_t)imin((int)e1, (int)(q0 + kL2Chunk / kWavesPerBlock));
    for (uint32_t base = q0; base < q1; base += kWave) {
      const uint32_t e = base + (uint32_t)l;
      const uint64_t m = e < q1 ? masks[e] : 0ull;
      cnt += (uint32_t)__popcll(transpose64(m));  // lane j: entries with tile j
    }
    s_wc[w][l] = cnt;
    __syncthreads();
    if (t < kWave) cnt2[(size_t)c * kWave + t] = s_wc[0][t] + s_wc[1][t] + s_wc[2][t] + s_wc[3][t];
    __syncthreads();  // before the next chunk's counts
  }
}

// Level 2c: per super-tile, each chunk's exclusive prefix per tile (base2)
// and the tile totals.
__global__ void __launch_bounds__(kWave)
l2_st_scan_kernel(StGrid sg, const uint32_t* __restrict__ chunk_first,
                  const uint32_t* __restrict__ cnt2, uint32_t* __restrict__ base2,
                  uint32_t* __restrict__ tile_total, int64_t max_chunks) {
  const int s = (int)blockIdx.x;
  const int l = (int)threadIdx.x;
  uint32_t run = 0;
  const uint32_t c1 = (int64_t)chunk_first[s + 1] < max_chunks ? chunk_first[s + 1]
                                                                 : (uint32_t)max_chunks;
  for (uint32_t c = chunk_first[s]; c < c1; c += kScanBatch) {
    uint32_t v[kScanBatch];
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) v[i] = c + i < c1 ? cnt2[(size_t)(c + i) * kWave + l] : 0u;
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) {
      if (c + i < c1) base2[(size_t)(c + i) * kWave + l] = run;
      run += v[i];
    }
  }
  const int x = (s % sg.sgx) * kSt + (l % kSt), y = (s / sg.sgx) * kSt + (l / kSt);
  if (x < sg.gx && y < sg.gy) tile_total[y * sg.gx + x] = run;
}

// Level 2d (one workgroup): tile starts, ranges (empty tiles [0,0], as the
// reference's zero-filled ranges), bucket counts and their inclusive scan.
// Thread t owns tiles [t*kTilesPer, (t+1)*kTilesPer) (the two-level path has
// at most kMaxSt * 64 = 16384 tiles, 16 per thread); global loads and stores
// go through LDS so they stay coalesced.
constexpr int kTilesPer = kMaxSt * kWave / 1024;
constexpr int kTileLds = 1024 * kTilesPer + 1024 * kTilesPer / 32;
__device__ __forceinline__ int tpad(int i) { return i + (i >> 5); }
__global__ void __launch_bounds__(1024)
l2_tile_scan_kernel(int32_t T, const uint32_t* __restrict__ tile_total,
                    uint32_t* __restrict__ tile_start, uint32_t* __restrict__ ranges,
                    uint32_t* __restrict__ bucket_count, uint32_t* __restrict__ bucket_offsets,
                    WaitWords ww) {
  __shared__ uint32_t s_tmp[1024 / kWave + 1];
  const uint32_t status = report_waits(ww);
  __shared__ uint32_t s_v[kTileLds];
  const int t = (int)threadIdx.x;
  const int t0 = t * kTilesPer;
#pragma unroll
  for (int i = 0; i < kTilesPer; ++i) {
    const int idx = i * 1024 + t;
    s_v[tpad(idx)] = idx < T ? tile_total[idx] : 0u;
  }
  __syncthreads();
  uint32_t n[kTilesPer];
  uint32_t sum = 0, bsum = 0;
#pragma unroll
  for (int i = 0; i < kTilesPer; ++i) {
    n[i] = s_v[tpad(t0 + i)];
    sum += n[i];
    bsum += (n[i] + 31u) / 32u;
  }
  uint32_t st = block_excl_scan(sum, s_tmp, nullptr);  // has barriers
  uint32_t bo = block_excl_scan(bsum, s_tmp, nullptr);
  // tile starts into LDS, then tile_start and ranges
#pragma unroll
  for (int i = 0; i < kTilesPer; ++i) {
    s_v[tpad(t0 + i)] = st;
    st += n[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTilesPer; ++i) {
    const int idx = i * 1024 + t;
    if (idx < T) {
      const uint32_t a = s_v[tpad(idx)];
      const uint32_t m = tile_total[idx];
      tile_start[idx] = a;
      *reinterpret_cast<uint2*>(ranges + 2 * (size_t)idx) = m ? make_uint2(a, a + m)
                                                               : make_uint2(0u, 0u);
      bucket_count[idx] = (m + 31u) / 32u;
    }
  }
  __syncthreads();
  // inclusive bucket offsets
#pragma unroll
  for (int i = 0; i < kTilesPer; ++i) {
    bo += (n[i] + 31u) / 32u;
    s_v[tpad(t0 + i)] = bo;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTilesPer; ++i) {
    const int idx = i * 1024 + t;
    if (idx < T) bucket_offsets[idx] = s_v[tpad(idx)];
  }
  if (T > 0) report_host(ww, status, s_v[tpad(T - 1)]);
}

// Level 2e: every entry's tiles written at tile start + entries of the tile
// in earlier chunks + rank in this chunk (list order).
//
// The chunk's 512 entries (index, depth bits) are kept in LDS.  A chunk whose
// output fits the stage (at most kL2Stage outputs): four wavefronts take 128
// entries each.  Per round of 64 entries, a 64x64 bit transpose gives lane j
// the ballot of the entries having tile j; each lane then walks the set bits
// of its own mask and stages the entries' chunk positions (16 bits each)
// grouped by tile.  The output is then written run by run (consecutive lanes,
// consecutive positions; wavefront w writes tiles j = w mod 4), each slot's
// index and depth bits read from the chunk's entries.  The stage holds 9216
// outputs in 18 KB and the entries take 4 KB, so LDS admits six workgroups
// per CU (with 4608 outputs, eight: fewer chunks fit the stage, and at 1M
// Gaussians / 1080p the binning took 5 us longer).
//
// A larger chunk (wide Gaussians, whose masks are dense) is written tile by
// tile: every wavefront holds the chunk's 512 masks in registers (eight per
// lane) and takes tiles j = w mod 4; per tile and round of 64 entries, the
// ballot of "has tile j" and the lane's rank below it place the entries at
// consecutive positions, so each store is one contiguous run.
//
// Workgroups take chunks c = blockIdx.x, blockIdx.x + gridDim.x, ... up to the
// chunk count on the device, so the grid need not cover the host's bound.
constexpr int kL2Stage = 9216;
constexpr int kL2PerLane = kL2Chunk / kWave;  // 8 entries per lane on the tile-by-tile path
static_assert(kL2Stage * 2 >= kL2Chunk * 8, "the tile-by-tile path keeps a chunk's masks in the stage");
template <bool kCarry>
__global__ void __launch_bounds__(kL1Group, 8)
l2_emit_kernel(StGrid sg, const uint32_t* __restrict__ list,
               const uint32_t* __restrict__ st_start, const uint32_t* __restrict__ chunk_first,
               const uint32_t* __restrict__ chunk_st, const uint32_t* __restrict__ nchunks,
               const uint64_t* __restrict__ masks, const uint32_t* __restrict__ cnt2,
               const uint32_t* __restrict__ base2, const uint32_t* __restrict__ tile_start,
               int32_t P, const float* __restrict__ depths, const uint32_t* __restrict__ ldb,
               int64_t K, uint64_t* __restrict__ keys, uint32_t* __restrict__ point_list) {
  __shared__ __align__(16) uint16_t s_idx[kL2Stage];   // staged outputs: chunk positions
  __shared__ __align__(16) uint32_t s_eg[kL2Chunk];    // the chunk's entries: Gaussian index
  __shared__ __align__(16) uint32_t s_edb[kL2Chunk];   // and depth bits
  __shared__ uint32_t s_wc[kWavesPerBlock][kWave];
  const uint32_t nch = nchunks[0];
  const int t = (int)threadIdx.x, w = t / kWave, l = lane_id();
  for (uint32_t c = blockIdx.x; c < nch; c += gridDim.x) {
    const uint32_t s = chunk_st[c];
    const uint32_t e0 = st_start[s] + (c - chunk_first[s]) * kL2Chunk;
    const uint32_t e1 = (uint32_t)imin(imin((int)st_start[s + 1], (int)(e0 + kL2Chunk)), (int)K);
    const int x0 = (int)(s % (uint32_t)sg.sgx) * kSt, y0 = (int)(s / (uint32_t)sg.sgx) * kSt;
    // lane j: tile j's chunk count, staging offset and global base
    const uint32_t cj = cnt2[(size_t)c * kWave + l];
    const uint32_t ci = wave_incl_scan(cj);
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)ci, kWave - 1);
    uint32_t gbase = 0;
    {
      const int x = x0 + (l % kSt), y = y0 + (l / kSt);
      if (x < sg.gx && y < sg.gy) gbase = tile_start[y * sg.gx + x] + base2[(size_t)c * kWave + l];
    }
    if (total > (uint32_t)kL2Stage) {  // uniform: the tile-by-tile path
      // the chunk's entries are loaded once per workgroup: masks in the
      // (here unused) stage, indices and depth bits in the entry arrays
      uint64_t* s_m = reinterpret_cast<uint64_t*>(s_idx);
      for (int q = t; q < kL2Chunk; q += kL1Group) {
        const uint32_t e = e0 + (uint32_t)q;
        const bool valid = e < e1;
        const uint64_t m = valid ? masks[e] : 0ull;
        const uint32_t g = valid ? list[e] : 0u;
        s_m[q] = m;
        s_eg[q] = g;
        s_edb[q] = kCarry ? (valid ? ldb[e] : 0xFFFFFFFFu)
                          : ((m != 0ull && g < (uint32_t)P) ? __float_as_uint(depths[g]) : 0xFFFFFFFFu);
      }
      __syncthreads();
      uint64_t em[kL2PerLane];  // the masks in registers; index and depth bits read when taken
#pragma unroll
      for (int r = 0; r < kL2PerLane; ++r) em[r] = s_m[r * kWave + l];
      for (int j = w; j < kWave; j += kWavesPerBlock) {
        const uint32_t nj = (uint32_t)__builtin_amdgcn_readlane((int)cj, j);
        if (nj == 0u) continue;
        uint32_t pos = (uint32_t)__builtin_amdgcn_readlane((int)gbase, j);
        const uint32_t end = pos + nj;
        const uint64_t tile = (uint64_t)((y0 + j / kSt) * sg.gx + x0 + (j % kSt)) << 32;
#pragma unroll
        for (int r = 0; r < kL2PerLane; ++r) {
          const bool has = ((em[r] >> j) & 1ull) != 0ull;
          const uint64_t bal = __ballot(has);
          const uint32_t at = pos + (uint32_t)__popcll(bal & lanemask_lt());
          // positions stay inside tile j's range of this chunk
          if (has && at < end && (int64_t)at < K) {
            keys[at] = tile | (uint64_t)s_edb[r * kWave + l];
            point_list[at] = s_eg[r * kWave + l];
          }
          pos += (uint32_t)__popcll(bal);
        }
      }
      __syncthreads();  // before the next chunk restages the arrays
      continue;
    }
    const int qw = w * (kL2Chunk / kWavesPerBlock);  // the wavefront's first chunk position
    const uint32_t q0 = e0 + (uint32_t)qw;
    const uint32_t q1 = (uint32_t)imin((int)e1, (int)(q0 + kL2Chunk / kWavesPerBlock));
    // the wavefront's entries, two rounds of 64, all loaded at once (the depth
    // gathers follow the indices and stay in flight across the barrier)
    constexpr int kRounds = kL2Chunk / kWavesPerBlock / kWave;
    static_assert(kRounds == 2, "two rounds of 64 entries per wavefront");
    uint64_t m[kRounds], bt[kRounds];
    uint32_t g[kRounds], db[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const uint32_t e = q0 + (uint32_t)(r * kWave + l);
      const bool in = e < q1;
      m[r] = in ? masks[e] : 0ull;
      g[r] = in ? list[e] : 0u;
      if (kCarry) db[r] = in ? ldb[e] : 0u;
    }
    if (!kCarry) {
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const uint32_t e = q0 + (uint32_t)(r * kWave + l);
        db[r] = (e < q1 && g[r] < (uint32_t)P) ? __float_as_uint(depths[g[r]]) : 0xFFFFFFFFu;
      }
    }
    // this wavefront's entries per tile (lane j)
    {
      uint32_t cnt = 0;
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        bt[r] = transpose64(m[r]);
        cnt += (uint32_t)__popcll(bt[r]);
      }
      s_wc[w][l] = cnt;
    }
    const uint32_t soff = ci - cj;
    lds_barrier();
    uint32_t cur = soff;
    for (int k = 0; k < w; ++k) cur += s_wc[k][l];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      // lane j: the round's entries having tile j (bit i = entry i).  Lane j
      // walks them in entry (depth) order and stages each one's chunk
      // position; the loop runs as often as the busiest tile of the round
      // has entries.
      const uint32_t qr = (uint32_t)(qw + r * kWave);
      uint64_t b = bt[r];
      uint32_t at = cur;
      while (__ballot(b != 0ull) != 0ull) {
        const bool act = b != 0ull;
        const uint32_t src = act ? (uint32_t)__builtin_ctzll(b) : 0u;
        b &= b - 1ull;
        if (act && at < (uint32_t)kL2Stage) s_idx[at] = (uint16_t)(qr + src);
        if (act) ++at;
      }
      cur += (uint32_t)__popcll(bt[r]);  // lane j: tile j's entries in this round
    }
    // the entries themselves, after the loads have landed (the walk above
    // needs only the masks)
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      s_eg[qw + r * kWave + l] = g[r];
      s_edb[qw + r * kWave + l] = db[r];
    }
    lds_barrier();
    for (int j = w; j < kWave; j += kWavesPerBlock) {
      const uint32_t nj = (uint32_t)__builtin_amdgcn_readlane((int)cj, j);
      if (nj == 0u) continue;
      const uint32_t oj = (uint32_t)__builtin_amdgcn_readlane((int)soff, j);
      const uint32_t gj = (uint32_t)__builtin_amdgcn_readlane((int)gbase, j);
      const uint64_t tile = (uint64_t)((y0 + j / kSt) * sg.gx + x0 + (j % kSt)) << 32;
      for (uint32_t k = (uint32_t)l; k < nj; k += kWave) {
        const uint32_t pos = gj + k;
        if ((int64_t)pos < K && oj + k < (uint32_t)kL2Stage) {
          const uint32_t q = s_idx[oj + k] & (uint32_t)(kL2Chunk - 1);
          keys[pos] = tile | (uint64_t)s_edb[q];
          point_list[pos] = s_eg[q];
        }
      }
    }
    lds_barrier();  // before the next chunk restages the arrays
  }
}

static StGrid st_grid(int gx, int gy) {
  StGrid g;
  g.gx = gx;
  g.gy = gy;
  g.sgx = (gx + kSt - 1) / kSt;
  g.sgy = (gy + kSt - 1) / kSt;
  g.S = g.sgx * g.sgy;
  return g;
}

static int bits_for(int64_t count) {
  int b = 0;
  while (b < 32 && ((int64_t)1 << b) < count) ++b;
  return b;
}

static size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

// Depth-order state (depth keys, sorted keys, the order and the sort's own
// state): a depth workspace, and the first part of every binning workspace.
struct DepthLayout {
  size_t dkeys, dkeys_s, order, sort, total;
};

static DepthLayout depth_layout(int32_t P) {
  DepthLayout D;
  size_t o = 0;
  D.dkeys = o; o += al((size_t)P * 4);
  D.dkeys_s = o; o += al((size_t)P * 4);
  D.order = o; o += al((size_t)P * 4);
  D.sort = o; o += sort_ws_bytes<uint32_t>(P, 4);
  D.total = o;
  return D;
}

// The error word of the depth sort in a depth workspace.
static const uint32_t* depth_err_word(const char* dws, int32_t P) {
  return sort_err_word<uint32_t>((void*)(dws + depth_layout(P).sort), P);
}
// Its count of visible Gaussians (the entries of the order before the
// sentinel tail), two words after the error word in the sort's state.
static const uint32_t* depth_nvis_word(const char* dws, int32_t P) {
  return depth_err_word(dws, P) + 2;
}

// The P Gaussians by depth bits, culled ones last (keys made inside the
// histogram kernel); the order lands at D.order of dws.
static int32_t run_depth_order(int32_t P, const float* depths, const uint32_t* tiles_touched,
                               char* dws, hipStream_t st) {
  const DepthLayout D = depth_layout(P);
  return radix_sort_pairs<uint32_t, true>(nullptr, nullptr, (uint32_t*)(dws + D.dkeys_s),
                                          (uint32_t*)(dws + D.order), P, 0, 32, dws + D.sort, st,
                                          depths, tiles_touched, (uint32_t*)(dws + D.dkeys));
}

struct BinningLayout {
  size_t cnt, scanP, tkeys, tvals, tkeys_s, sortK, total;
};

static BinningLayout binning_layout(int32_t P, int64_t K, int32_t T) {
  BinningLayout L;
  size_t o = depth_layout(P).total;
  L.cnt = o; o += al((size_t)P * 4);
  L.scanP = o; o += scan_ws_bytes(P);
  L.tkeys = o; o += al((size_t)K * 4);
  L.tvals = o; o += al((size_t)K * 4);
  L.tkeys_s = o; o += al((size_t)K * 4);
  L.sortK = o; o += sort_ws_bytes<uint32_t>(K, (bits_for(T) + 7) / 8);
  L.total = o;
  return L;
}

// Workspace of the two-level path (sized for kMaxSt super-tiles).
// The list entries' depth bits: above this many Gaussians, l1_place writes
// each entry's depth bits (its sorted key) beside it and l2_emit reads them
// in list order; below, l2_emit gathers depths[g], whose array then stays in
// the L2 cache (at 1M Gaussians carrying them measured slower, at 3M the
// gather fetched about 1.1 GB per frame).
constexpr int32_t kCarryDepthMinP = 1 << 21;
static inline bool carry_depth_bits(int32_t P) { return P > kCarryDepthMinP; }

struct TwoLevelLayout {
  size_t recw, sets, cnt1, segsum, st_start, chunk_first, nchunks, chunk_st, list, masks, ldb,
      cnt2, base2, tile_total, tile_start, total;
  int64_t max_chunks;
};

static TwoLevelLayout two_level_layout(int32_t P, int64_t K, int32_t T) {
  TwoLevelLayout L;
  const int64_t nwg1 = (P + kL1Group - 1) / kL1Group;
  L.max_chunks = K / kL2Chunk + kMaxSt + 1;
  size_t o = depth_layout(P).total;
  L.recw = o; o += al((size_t)P * 4);
  L.sets = o; o += al((size_t)P * 32);
  L.cnt1 = o; o += al((size_t)nwg1 * kMaxSt * 4);
  L.segsum = o; o += al((size_t)kL1Segs * kMaxSt * 4);
  L.st_start = o; o += al((kMaxSt + 1) * 4);
  L.chunk_first = o; o += al((kMaxSt + 1) * 4);
  L.nchunks = o; o += al(4);
  L.chunk_st = o; o += al((size_t)L.max_chunks * 4);
  L.list = o; o += al((size_t)K * 4);
  L.masks = o; o += al((size_t)K * 8);
  L.ldb = o; o += carry_depth_bits(P) ? al((size_t)K * 4) : 0;
  L.cnt2 = o; o += al((size_t)L.max_chunks * kWave * 4);
  L.base2 = o; o += al((size_t)L.max_chunks * kWave * 4);
  L.tile_total = o; o += al((size_t)T * 4);
  L.tile_start = o; o += al((size_t)T * 4);
  L.total = o;
  return L;
}

static bool use_two_level(const StGrid& sg, int64_t K) {
  return sg.S <= kMaxSt && K < (int64_t)0x7FFFFFFF;
}

}  // namespace fgs

using namespace fgs;

extern "C" size_t fgs_scan_workspace_bytes(int64_t n) { return scan_ws_bytes(n < 1 ? 1 : n); }

extern "C" uint32_t fgs_set_wait_spin_limit(uint32_t limit) { return g_spin_limit.exchange(limit); }

extern "C" int32_t fgs_inclusive_scan_u32(const uint32_t* in, uint32_t* out, int64_t n,
                                          void* workspace, uint32_t* wait_status, void* stream) {
  if (n < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_inclusive_scan_u32: n < 0");
  if (n > 0 && (!in || !out || !workspace))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_inclusive_scan_u32: null pointer");
  return launch_scan(in, out, n, workspace, true, (hipStream_t)stream, wait_status);
}

// ---------------------------------------------------------------------------
// Allocation-free inclusive scan: the scan's state (one status word per
// 4096-element chunk, the chunk ticket, the wait-error word) lives in a
// file-scope device array instead of a caller workspace.  Each device holds its
// own copy; its address is looked up once per device with that device current
// and cached.  The state is cleared by the scan's fill kernel on every call
// (graph-safe), so a call needs no initial contents; calls that overlap on one
// device share the array and race.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocMaxN = (int64_t)1 << 28;
constexpr int64_t kNoAllocChunks = kNoAllocMaxN / kChunk;  // 65536
constexpr size_t kNoAllocScratchBytes = scan_state_bytes(kNoAllocMaxN);  // 512.25 KiB
static_assert(kNoAllocScratchBytes == (size_t)kNoAllocChunks * 8 + 256, "scan state size");
static __device__ __align__(256) uint64_t scratch[kNoAllocScratchBytes / 8];

constexpr int kNoAllocMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kNoAllocMaxDevices];
static std::mutex g_scratch_mu;

// The current device's copy of `scratch` (host code never uses the array's
// name as an address: it is a host-side stand-in).
static int32_t noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(FGS_ERR_LAUNCH, "fgs_inclusive_scan_u32_noalloc: no current HIP device");
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        char msg[256];
        std::snprintf(msg, sizeof(msg),
                      "fgs_inclusive_scan_u32_noalloc: hipGetSymbolAddress failed on device %d: %s",
                      dev, hipGetErrorString(e));
        return set_error(FGS_ERR_LAUNCH, msg);
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FGS_OK;
}

extern "C" int32_t fgs_inclusive_scan_u32_noalloc(const uint32_t* in, uint32_t* out, int64_t n,
                                                  uint32_t* wait_status, void* stream) {
  if (n < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_inclusive_scan_u32_noalloc: n < 0");
  if (n > kNoAllocMaxN) {
    char msg[160];
    std::snprintf(msg, sizeof(msg),
                  "fgs_inclusive_scan_u32_noalloc: n = %lld exceeds the maximum of %lld elements",
                  (long long)n, (long long)kNoAllocMaxN);
    return set_error(FGS_ERR_INVALID_ARGUMENT, msg);
  }
  if (n == 0) {
    if (wait_status) launch_fill(wait_status, 0u, 1, (hipStream_t)stream);
    return wait_status ? check_launch("fgs_inclusive_scan_u32_noalloc") : FGS_OK;
  }
  if (!in || !out)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_inclusive_scan_u32_noalloc: null pointer");
  void* state = nullptr;
  const int32_t e = noalloc_scratch(&state);
  if (e != FGS_OK) return e;
  return launch_scan(in, out, n, state, true, (hipStream_t)stream, wait_status);
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

extern "C" size_t fgs_sort_workspace_bytes(int64_t n) { return sort_ws_bytes<uint64_t>(n < 1 ? 1 : n, 8); }

extern "C" int32_t fgs_sort_pairs_u64(const uint64_t* keys_in, const uint32_t* values_in,
                                      uint64_t* keys_out, uint32_t* values_out, int64_t n,
                                      int32_t begin_bit, int32_t end_bit, void* workspace,
                                      uint32_t* wait_status, void* stream) {
  if (n < 0 || begin_bit < 0 || end_bit > 64 || begin_bit > end_bit)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_sort_pairs_u64: bad arguments");
  if (n == 0) {
    if (wait_status) launch_fill(wait_status, 0u, 1, (hipStream_t)stream);
    return wait_status ? check_launch("fgs_sort_pairs_u64") : FGS_OK;
  }
  if (n > 0xFFFFFFFFll)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_sort_pairs_u64: n exceeds 2^32-1");
  if (!keys_in || !keys_out || !values_out || !workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_sort_pairs_u64: null pointer");
  return radix_sort_pairs<uint64_t>(keys_in, values_in, keys_out, values_out, n, begin_bit, end_bit,
                                    workspace, (hipStream_t)stream, nullptr, nullptr, nullptr,
                                    wait_status);
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
  const int32_t p = P < 1 ? 1 : P, t = num_tiles < 1 ? 1 : num_tiles;
  const int64_t k = num_rendered < 1 ? 1 : num_rendered;
  const size_t a = binning_layout(p, k, t).total, b = two_level_layout(p, k, t).total;
  return a > b ? a : b;
}

extern "C" size_t fgs_depth_order_workspace_bytes(int32_t P) {
  return depth_layout(P < 1 ? 1 : P).total;
}

extern "C" int32_t fgs_depth_order(int32_t P, const float* depths, const uint32_t* tiles_touched,
                                   void* depth_workspace, void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_depth_order: P < 0");
  if (P == 0) return FGS_OK;
  if (!depths || !tiles_touched || !depth_workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_depth_order: null pointer");
  const int32_t e = run_depth_order(P, depths, tiles_touched, (char*)depth_workspace,
                                    (hipStream_t)stream);
  if (e != FGS_OK) return e;
  return check_launch("depth_order");
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
  if (!io->st_rec != !io->st_masks || (reinterpret_cast<uintptr_t>(io->st_masks) & 15u) ||
      (reinterpret_cast<uintptr_t>(io->st_rec) & 15u))
    return set_error(FGS_ERR_INVALID_ARGUMENT,
                     "fgs_binning_sorted: st_rec and st_masks must both be set (16-byte aligned) "
                     "or both NULL");
  hipStream_t st = (hipStream_t)stream;
  const StGrid sg = st_grid(io->grid_x, io->grid_y);
  char* ws = (char*)io->workspace;
  WaitWords ww{};
  ww.out = io->wait_status;
  ww.host = io->host_result;
  if (io->depth_order) ww.w[0] = depth_err_word((const char*)io->depth_order, P);
  else if (K > 0 && P > 0) ww.w[0] = depth_err_word(ws, P);
  // Gaussians by depth bits: from the caller's depth workspace, or sorted here
  // into the front of the binning workspace
  const char* dws = io->depth_order ? (const char*)io->depth_order : ws;
  const uint32_t* order = (const uint32_t*)(dws + depth_layout(P).order);
  if (K > 0 && P > 0) {
    if (!io->xys || !io->depths || !io->conic_opacity || !io->tiles_touched ||
        !io->point_list_keys || !io->point_list)
      return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_binning_sorted: null pointer");
    if (!io->depth_order) {
      const int32_t e = run_depth_order(P, io->depths, io->tiles_touched, ws, st);
      if (e != FGS_OK) return e;
    }
  }
  if (K > 0 && P > 0 && use_two_level(sg, K)) {
    const TwoLevelLayout L = two_level_layout(P, K, T);
    uint64_t* sets = (uint64_t*)(ws + L.sets);
    uint32_t* cnt1 = (uint32_t*)(ws + L.cnt1);
    uint32_t* segsum = (uint32_t*)(ws + L.segsum);
    uint32_t* st_start = (uint32_t*)(ws + L.st_start);
    uint32_t* chunk_first = (uint32_t*)(ws + L.chunk_first);
    uint32_t* nchunks = (uint32_t*)(ws + L.nchunks);
    uint32_t* chunk_st = (uint32_t*)(ws + L.chunk_st);
    uint32_t* list = (uint32_t*)(ws + L.list);
    uint64_t* masks = (uint64_t*)(ws + L.masks);
    uint32_t* cnt2 = (uint32_t*)(ws + L.cnt2);
    uint32_t* base2 = (uint32_t*)(ws + L.base2);
    uint32_t* tile_total = (uint32_t*)(ws + L.tile_total);
    uint32_t* tile_start = (uint32_t*)(ws + L.tile_start);
    const unsigned nwg1 = ceil_div_u(P, kL1Group);
    uint32_t* recw = (uint32_t*)(ws + L.recw);
    const uint32_t* nvis = depth_nvis_word(dws, P);
    hipLaunchKernelGGL(l1_count_kernel, dim3(nwg1), dim3(kL1Group), 0, st, P, sg, io->mult, order,
                       nvis, io->xys, io->conic_opacity, io->tiles_touched, io->st_rec,
                       io->st_masks, recw, sets, cnt1);
    hipLaunchKernelGGL(l1_seg_scan_kernel, dim3(kL1Segs), dim3(kMaxSt), 0, st, (int)nwg1, sg.S,
                       cnt1, segsum);
    hipLaunchKernelGGL(l1_top_scan_kernel, dim3(1), dim3(kMaxSt), 0, st, sg.S, segsum, st_start,
                       chunk_first, chunk_st, nchunks, L.max_chunks);
    const bool carry = carry_depth_bits(P);
    const uint32_t* skeys = (const uint32_t*)(dws + depth_layout(P).dkeys_s);
    uint32_t* ldb = carry ? (uint32_t*)(ws + L.ldb) : nullptr;
    if (carry)
      hipLaunchKernelGGL(l1_place_kernel<true>, dim3(nwg1), dim3(kL1Group), 0, st, P, sg, order,
                         nvis, skeys, recw, sets, cnt1, segsum, st_start, K, list, masks, ldb,
                         io->mult, io->xys, io->conic_opacity);
    else
      hipLaunchKernelGGL(l1_place_kernel<false>, dim3(nwg1), dim3(kL1Group), 0, st, P, sg, order,
                         nvis, skeys, recw, sets, cnt1, segsum, st_start, K, list, masks, ldb,
                         io->mult, io->xys, io->conic_opacity);
    const unsigned nch = (unsigned)L.max_chunks;
    const unsigned egrid = nch < (unsigned)kL2EmitGrid ? nch : (unsigned)kL2EmitGrid;
    hipLaunchKernelGGL(l2_count_kernel, dim3(egrid), dim3(kL1Group), 0, st, st_start, chunk_first,
                       chunk_st, nchunks, K, masks, cnt2);
    hipLaunchKernelGGL(l2_st_scan_kernel, dim3(sg.S), dim3(kWave), 0, st, sg, chunk_first, cnt2,
                       base2, tile_total, L.max_chunks);
    hipLaunchKernelGGL(l2_tile_scan_kernel, dim3(1), dim3(1024), 0, st, T, tile_total, tile_start,
                       io->ranges, io->bucket_count, io->bucket_offsets, ww);
    if (carry)
      hipLaunchKernelGGL(l2_emit_kernel<true>, dim3(egrid), dim3(kL1Group), 0, st, sg, list,
                         st_start, chunk_first, chunk_st, nchunks, masks, cnt2, base2, tile_start,
                         P, io->depths, ldb, K, io->point_list_keys, io->point_list);
    else
      hipLaunchKernelGGL(l2_emit_kernel<false>, dim3(egrid), dim3(kL1Group), 0, st, sg, list,
                         st_start, chunk_first, chunk_st, nchunks, masks, cnt2, base2, tile_start,
                         P, io->depths, ldb, K, io->point_list_keys, io->point_list);
    return check_launch("binning_sorted (two-level)");
  }
  const BinningLayout L = binning_layout(P < 1 ? 1 : P, K < 1 ? 1 : K, T);
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
    // duplicate offsets in depth order: exclusive scan of tiles_touched[order[i]]
    int32_t e = launch_chained_scan<true>(io->tiles_touched, order, P, cnt, P, ws + L.scanP, false, false,
                                  st);
    if (e != FGS_OK) return e;
    ww.w[1] = (const uint32_t*)((const uint64_t*)(ws + L.scanP) + (P + kChunk - 1) / kChunk) + 1;
    hipLaunchKernelGGL(duplicate_sorted_kernel, dim3(gP), dim3(256), 0, st, P, order, cnt, io->xys,
                       io->conic_opacity, io->tiles_touched, io->mult, io->grid_x, io->grid_y, K,
                       tkeys, tvals);
    // stage 2: duplicates by tile id, stable
    e = radix_sort_pairs<uint32_t>(tkeys, tvals, tkeys_s, io->point_list, K, 0, bits_for(T),
                                   ws + L.sortK, st);
    if (e != FGS_OK) return e;
    if (bits_for(T) > 0) ww.w[2] = sort_err_word<uint32_t>(ws + L.sortK, K);
    hipLaunchKernelGGL(finalize_keys_ranges_kernel, dim3(ceil_div_u(K, 256)), dim3(256), 0, st, K,
                       T, P, tkeys_s, io->point_list, io->depths, io->point_list_keys,
                       io->ranges);
  }
  if (T > 0)
    hipLaunchKernelGGL(bucket_scan_kernel, dim3(1), dim3(1024), 0, st, T, io->ranges,
                       io->bucket_count, io->bucket_offsets, ww);
  else if (io->wait_status)
    launch_fill(io->wait_status, 0u, 1, st);
  return check_launch("binning_sorted");
}

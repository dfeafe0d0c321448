// CSR construction on the device: offsets, stable grouping order and the GIE
// grouping step.
//
// Restates python/kernels/segment.py:46-71 of the reference
// (segment_offsets = [0] ++ cumsum(bincount(keys)), group_by_source = stable
// argsort + offsets) as a bounded-key counting sort, written for wave64:
//
//   count     one pass over the int64 keys in tiles of 8192: the range and
//             sortedness checks (the reference's dst.min()/dst.max() test),
//             and each tile's histogram of the coarse digit (the key's high
//             bits, at most 1024 buckets) with LDS atomics;
//   scan      one wave per bucket scans the bucket's counts over the tiles:
//             every tile learns where its run of each bucket starts;
//   scatter   each tile ranks its elements stably within their bucket (a
//             wave matches equal digits with one ballot per digit bit and
//             counts the lower lanes with mbcnt, so equal keys keep their
//             order: wave by wave, round by round, lane by lane), sorts them
//             in LDS and writes each bucket's run contiguously, packed as
//             (index << fine_bits | fine digit) in 32 bits when it fits;
//   finish    one workgroup per bucket: LDS histogram of the fine digit (the
//             key's low bits) -> the offsets of the bucket's keys, then the
//             same stable ranking, chunk by chunk -> `order`.  When the keys
//             were already sorted (DeepMD's layout) the same launch instead
//             takes the offsets from the boundaries of the sorted list and
//             writes the identity order, and the count is the only pass.
//
// Keys of more than 21 bits take least-significant-digit passes of the same
// count / scan / scatter kernels instead ((key, index) pairs), then offsets
// from the sorted keys.  The count pass records in the status word whether
// the keys were sorted, and every later kernel reads it on the device, so the
// whole build is enqueued without a host round trip; the synchronous entry
// points read the word once at the end.  Loads go through buffer views with
// 32-bit offsets (past the end they return zeros), so no load waits in a
// branch and no lane does 64-bit address arithmetic.  Integer results are
// bit-exact and independent of scheduling (a stable order of a key list is
// unique).
#include <algorithm>

#include "common.h"

namespace dpa4k {
namespace {

constexpr int kThreads = 256;
constexpr int kGroupWaves = kThreads / 64;
constexpr int kItems = 32;                             // elements per thread in a tile
constexpr int kTile = kThreads * kItems;               // 8192 elements per count/scatter tile
constexpr int kDigitBits = 10;                         // at most 1024 buckets per scatter pass
constexpr int kMaxBuckets = 1 << kDigitBits;
constexpr int kFineBitsMax = 10;                       // the two-level path: keys of up to 20 bits
constexpr int kMaxFine = 1 << kFineBitsMax;
constexpr int kLocalItems = 16;
constexpr int kLocalChunk = kThreads * kLocalItems;    // 4096 elements per bucket-local round
constexpr int64_t kShortGap = 64;                      // offsets a thread fills alone

enum : int32_t { kFlagOutOfRange = 1, kFlagUnsorted = 2, kFlagSlotRange = 4, kFlagSlotShared = 8 };
constexpr int kSlotRowsShift = 16;  // bits 16..23: most rows reading one radial slot (GIE grouping)
enum Gate : int { kAlways = 0, kIfSorted = 1, kIfUnsorted = 2 };

static_assert(DPA4K_CSR_OUT_OF_RANGE == kFlagOutOfRange && DPA4K_CSR_UNSORTED == kFlagUnsorted,
              "status bits of the header");

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The status word as written by earlier launches on the stream (a new launch
// sees their writes; nothing writes it during a gated launch): one plain load
// per wave, at a uniform address.
__device__ __forceinline__ int32_t status_of(const int32_t* status) {
  return __builtin_amdgcn_readfirstlane(status[0]);
}

__device__ __forceinline__ bool gate_closed(const int32_t* status, int gate) {
  if (gate == kAlways) return false;
  const bool unsorted = (status_of(status) & kFlagUnsorted) != 0;
  return gate == kIfSorted ? unsorted : !unsorted;
}

__device__ __forceinline__ int64_t load_i64(BufferView view, uint32_t offset) {
  const u32x2 raw = __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(offset), 0, 0);
  return __builtin_bit_cast(int64_t, raw);
}

__device__ __forceinline__ uint32_t load_u32(BufferView view, uint32_t offset) {
  return __builtin_amdgcn_raw_buffer_load_b32(view, static_cast<int>(offset), 0, 0);
}

// Exclusive scan of one value per thread over the workgroup; `total` gets
// the sum.  Every thread must call it.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t value, uint32_t* wave_totals, uint32_t& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t inclusive = value;
#pragma unroll
  for (int offset = 1; offset < 64; offset <<= 1) {
    const uint32_t other = __shfl_up(inclusive, offset, 64);
    if (lane >= offset) inclusive += other;
  }
  if (lane == 63) wave_totals[wave] = inclusive;
  __syncthreads();
  uint32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kGroupWaves; ++w) {
    const uint32_t part = wave_totals[w];
    before += w < wave ? part : 0u;
    sum += part;
  }
  __syncthreads();
  total = sum;
  return before + inclusive - value;
}

// In-place exclusive scan of values[0, n) in LDS (plus `base`); returns the
// total.  Every thread must call it.
__device__ __forceinline__ uint32_t lds_exclusive_scan(uint32_t* values, int n, uint32_t base,
                                                       uint32_t* wave_totals) {
  const int per = (n + kThreads - 1) / kThreads;
  const int first = threadIdx.x * per;
  uint32_t sum = 0;
  for (int i = 0; i < per; ++i)
    if (first + i < n) sum += values[first + i];
  uint32_t total = 0;
  uint32_t running = base + block_exclusive_scan(sum, wave_totals, total);
  for (int i = 0; i < per; ++i)
    if (first + i < n) {
      const uint32_t value = values[first + i];
      values[first + i] = running;
      running += value;
    }
  __syncthreads();
  return total;
}

__device__ __forceinline__ int64_t element_limit(int64_t n, const uint32_t* count_limit) {
  if (count_limit == nullptr) return n;
  const int64_t limit = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(count_limit[0]));
  return limit < n ? limit : n;
}

// ---------------------------------------------------------------------------
// block-local stable counting sort in LDS
// ---------------------------------------------------------------------------
//
// Elements live in LDS at padded positions (one spare word per 32, so that a
// thread reading its 32 consecutive elements, or its 32 consecutive counters,
// touches 32 different banks).  Each pass sorts them stably by kSubBits of the
// digit: thread t owns the consecutive positions [t K, t K + K), counts them
// in its own column of a [digit][thread] counter array (no other thread
// touches the column), the array is scanned in digit-major order, and every
// element moves to (its digit's count before this thread) + (its rank among
// this thread's equal digits).  Least-significant sub-digit first, so after
// the last pass the elements are ordered by the whole digit and, within a
// digit, by their position before the sort.
constexpr int kSubBits = 5;
constexpr int kSubDigits = 1 << kSubBits;
constexpr int kCounterWords = kSubDigits * kThreads + kSubDigits * kThreads / 32;

__device__ __forceinline__ int padded(int position) { return position + (position >> 5); }

template <typename E>
__device__ __forceinline__ uint32_t digit_of(E element, int shift, uint32_t mask) {
  return static_cast<uint32_t>(element >> shift) & mask;
}

template <typename E, int K>
__device__ void block_stable_sort(E* buffer, int n, int shift, int bits, uint32_t* counters, uint32_t* wave_totals) {
  const int t = threadIdx.x;
  for (int done = 0; done < bits; done += kSubBits) {
    const int pass_bits = bits - done < kSubBits ? bits - done : kSubBits;
    const int pass_shift = shift + done;
    const int digits = 1 << pass_bits;
    const uint32_t mask = static_cast<uint32_t>(digits - 1);
    E element[K];
    uint32_t rank[K / 4];  // ranks below K <= 32: four per word
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int position = t * K + i;
      element[i] = position < n ? buffer[padded(position)] : E(0);
    }
    for (int d = 0; d < digits; ++d) counters[padded(d * kThreads + t)] = 0u;
#pragma unroll
    for (int i = 0; i < K / 4; ++i) rank[i] = 0u;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (t * K + i < n) {
        const int slot = padded(static_cast<int>(digit_of(element[i], pass_shift, mask)) * kThreads + t);
        const uint32_t count = counters[slot];
        rank[i / 4] |= count << (8 * (i % 4));
        counters[slot] = count + 1u;
      }
    }
    __syncthreads();
    // exclusive scan of counters[digit][thread] in flat order; thread t scans
    // the flat range [t * digits, (t + 1) * digits)
    const int first = t * digits;
    uint32_t sum = 0;
    for (int j = 0; j < digits; ++j) sum += counters[padded(first + j)];
    uint32_t total;
    uint32_t running = block_exclusive_scan(sum, wave_totals, total);
    for (int j = 0; j < digits; ++j) {
      const int slot = padded(first + j);
      const uint32_t value = counters[slot];
      counters[slot] = running;
      running += value;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (t * K + i < n) {
        const uint32_t digit = digit_of(element[i], pass_shift, mask);
        const uint32_t own = (rank[i / 4] >> (8 * (i % 4))) & 0xffu;
        buffer[padded(static_cast<int>(counters[padded(static_cast<int>(digit) * kThreads + t)] + own))] = element[i];
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(64) void clear_word_kernel(int32_t* __restrict__ word) {
  if (threadIdx.x == 0) *word = 0;
}

// Tile `blockIdx.x` of the keys (the caller's int64 keys, or the uint32 keys
// of an earlier pass): element q of the tile is q = 256 r + thread for
// r < kItems, so each wave's loads cover 64 consecutive elements.
struct TileKeys {
  uint32_t key[kItems];
  uint32_t ok = 0;        // bit r: element r exists and its key lies in [0, N)
  int n = 0;              // elements of the tile
};

__device__ __forceinline__ int tile_elements(int64_t tile_base, int64_t limit) {
  const int64_t rest = limit - tile_base;
  return static_cast<int>(rest < 0 ? 0 : (rest > kTile ? kTile : rest));
}

// The caller's int64 keys.  With kCheck, `flags` gets kFlagOutOfRange and
// kFlagUnsorted (some in-range key followed by a smaller one, the element
// after the tile included); `first_of_wave` is LDS scratch of
// (kItems + 1) * kGroupWaves words.
template <bool kCheck>
__device__ __forceinline__ void load_keys64(const int64_t* keys, int64_t tile_base, int64_t limit, uint64_t n_nodes,
                                            TileKeys& tile, int32_t& flags, uint32_t* first_of_wave,
                                            uint32_t* first_ok) {
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int64_t rest = limit - tile_base;
  tile.n = tile_elements(tile_base, limit);
  // one element past the tile, for the sortedness check at its end
  const int extent = static_cast<int>(rest < 0 ? 0 : (rest > kTile + 1 ? kTile + 1 : rest));
  const BufferView view = buffer_view(keys + (tile.n > 0 ? tile_base : 0), static_cast<int64_t>(extent) * 8);
  int64_t raw[kItems];
#pragma unroll
  for (int r = 0; r < kItems; ++r) raw[r] = load_i64(view, static_cast<uint32_t>(r * kThreads + t) * 8u);
  const int64_t after = kCheck ? load_i64(view, static_cast<uint32_t>(kTile) * 8u) : 0;
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const int q = r * kThreads + t;
    const bool valid = q < tile.n;
    const bool in = valid && static_cast<uint64_t>(raw[r]) < n_nodes;
    tile.key[r] = static_cast<uint32_t>(raw[r]);
    tile.ok |= in ? (1u << r) : 0u;
    if (kCheck && valid && !in) flags |= kFlagOutOfRange;
  }
  if constexpr (kCheck) {
    // element q against q + 1: the next lane's element of the round, or through LDS the first
    // element of the next wave (or of the next round, or the element after the tile)
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kItems; ++r) {
        first_of_wave[r * kGroupWaves + wave] = tile.key[r];
        first_ok[r * kGroupWaves + wave] = (tile.ok >> r) & 1u;
      }
    }
    if (t == 0) {
      first_of_wave[kItems * kGroupWaves] = static_cast<uint32_t>(after);
      first_ok[kItems * kGroupWaves] = extent > kTile && static_cast<uint64_t>(after) < n_nodes ? 1u : 0u;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
      uint32_t next = static_cast<uint32_t>(__shfl_down(static_cast<int>(tile.key[r]), 1, 64));
      uint32_t next_ok = static_cast<uint32_t>(__shfl_down(static_cast<int>((tile.ok >> r) & 1u), 1, 64));
      if (lane == 63) {
        const int slot = wave + 1 < kGroupWaves ? r * kGroupWaves + wave + 1 : (r + 1) * kGroupWaves;
        next = first_of_wave[slot];
        next_ok = first_ok[slot];
      }
      if (((tile.ok >> r) & 1u) && next_ok && next < tile.key[r]) flags |= kFlagUnsorted;
    }
  }
}

// uint32 keys of an earlier pass (in range by construction).
__device__ __forceinline__ void load_keys32(const uint32_t* keys, int64_t tile_base, int64_t limit, TileKeys& tile) {
  const int t = threadIdx.x;
  tile.n = tile_elements(tile_base, limit);
  const BufferView view = buffer_view(keys + (tile.n > 0 ? tile_base : 0), static_cast<int64_t>(tile.n) * 4);
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const int q = r * kThreads + t;
    tile.key[r] = load_u32(view, static_cast<uint32_t>(q) * 4u);
    tile.ok |= q < tile.n ? (1u << r) : 0u;
  }
}

// Per-tile histogram of the digit (key >> shift) & (2^bits - 1) over in-range
// keys, into column `tile` of counts[buckets][tiles].  kCheck (the first pass,
// on the caller's keys) also ORs the range and sortedness flags into the
// status word, once per workgroup and only when they add a bit.
template <bool kPairs, bool kCheck>
__global__ __launch_bounds__(kThreads) void tile_count_kernel(const int64_t* __restrict__ keys64,
                                                              const uint32_t* __restrict__ keys32, int64_t n,
                                                              const uint32_t* count_limit, uint64_t n_nodes,
                                                              int shift, int bits, int buckets, int64_t tiles,
                                                              uint32_t* __restrict__ counts,
                                                              int32_t* __restrict__ status, int gate) {
  __shared__ uint32_t histogram[kMaxBuckets];
  __shared__ uint32_t first_of_wave[(kItems + 1) * kGroupWaves];
  __shared__ uint32_t first_ok[(kItems + 1) * kGroupWaves];
  if (gate_closed(status, gate)) return;
  const int64_t limit = element_limit(n, count_limit);
  for (int b = threadIdx.x; b < buckets; b += kThreads) histogram[b] = 0u;
  const int64_t tile_base = static_cast<int64_t>(blockIdx.x) * kTile;
  const uint32_t digit_mask = (1u << bits) - 1u;
  TileKeys tile;
  int32_t local = 0;
  if constexpr (kPairs)
    load_keys32(keys32, tile_base, limit, tile);
  else
    load_keys64<kCheck>(keys64, tile_base, limit, n_nodes, tile, local, first_of_wave, first_ok);
  __syncthreads();
  // plain LDS atomics: a histogram needs no ranks
#pragma unroll
  for (int r = 0; r < kItems; ++r)
    if ((tile.ok >> r) & 1u) atomicAdd(&histogram[(tile.key[r] >> shift) & digit_mask], 1u);
  if constexpr (kCheck) {
    const int32_t found = (__syncthreads_or(local & kFlagOutOfRange) ? kFlagOutOfRange : 0) |
                          (__syncthreads_or(local & kFlagUnsorted) ? kFlagUnsorted : 0);
    if (threadIdx.x == 0 && found != 0 &&
        (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & found) != found)
      atomicOr(status, found);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < buckets; b += kThreads)
    counts[static_cast<int64_t>(b) * tiles + blockIdx.x] = histogram[b];
}

// counts[b][t] -> the number of bucket-b elements in tiles before t, and
// bucket_total[b] (one workgroup per bucket, reading its row in order).
__global__ __launch_bounds__(kThreads) void row_scan_kernel(uint32_t* __restrict__ counts, int64_t tiles,
                                                            uint32_t* __restrict__ bucket_total,
                                                            const int32_t* __restrict__ status, int gate) {
  __shared__ uint32_t wave_totals[kGroupWaves];
  if (gate_closed(status, gate)) return;
  uint32_t* row = counts + static_cast<int64_t>(blockIdx.x) * tiles;
  uint32_t running = 0;
  for (int64_t first = 0; first < tiles; first += kThreads) {
    const int64_t t = first + threadIdx.x;
    const uint32_t value = t < tiles ? row[t] : 0u;
    uint32_t total = 0;
    const uint32_t before = block_exclusive_scan(value, wave_totals, total);
    if (t < tiles) row[t] = running + before;
    running += total;
  }
  if (threadIdx.x == 0) bucket_total[blockIdx.x] = running;
}

// Elements of the scatter's LDS sort.  32-bit: key in bits [0, 19), position
// in the tile in [19, 32) (keys of at most 19 bits); 64-bit: key in the high
// word, the position (or, for pairs, the edge index) in the low word.
// Elements that are out of range take the largest key, which sorts them
// after every in-range element of the tile's last bucket.
template <typename E>
struct ElementCodec;

template <>
struct ElementCodec<uint32_t> {
  static constexpr int kKeyShift = 0;
  static constexpr uint32_t kBadKey = (1u << 19) - 1u;
  __device__ static uint32_t make(uint32_t key, uint32_t low) { return key | (low << 19); }
  __device__ static uint32_t key(uint32_t e) { return e & ((1u << 19) - 1u); }
  __device__ static uint32_t low(uint32_t e) { return e >> 19; }
};

template <>
struct ElementCodec<uint64_t> {
  static constexpr int kKeyShift = 32;
  static constexpr uint32_t kBadKey = 0xffffffffu;
  __device__ static uint64_t make(uint32_t key, uint32_t low) { return (static_cast<uint64_t>(key) << 32) | low; }
  __device__ static uint32_t key(uint64_t e) { return static_cast<uint32_t>(e >> 32); }
  __device__ static uint32_t low(uint64_t e) { return static_cast<uint32_t>(e); }
};

// (index << fine_bits) | fine digit, for the bucket-local pass.
template <typename P>
struct PackedOut {
  P* out;
  int fine_bits;
  __device__ __forceinline__ void store(uint32_t position, uint32_t key, uint32_t index) const {
    out[position] = (static_cast<P>(index) << fine_bits) | static_cast<P>(key & ((1u << fine_bits) - 1u));
  }
};

// (key, index) pairs, for the next least-significant-digit pass.
struct PairsOut {
  uint32_t* keys;
  uint32_t* index;
  __device__ __forceinline__ void store(uint32_t position, uint32_t key, uint32_t idx) const {
    keys[position] = key;
    index[position] = idx;
  }
};

// Stable scatter of one tile by digit: each element goes to
//   bucket_start[b] + (elements of b in earlier tiles) + (its rank within b in this tile).
// The tile is loaded (coalesced) into LDS, sorted there stably by the digit
// (block_stable_sort), and each bucket's run leaves as one contiguous write.
// Every block scans the bucket totals for itself; block 0 also publishes the
// bucket starts (and the count of in-range elements) for the next launch.
template <typename E, bool kPairs, typename Out>
__global__ __launch_bounds__(kThreads) void tile_scatter_kernel(
    const int64_t* __restrict__ keys64, const uint32_t* __restrict__ keys32, const uint32_t* __restrict__ index32,
    int64_t n, const uint32_t* count_limit, uint64_t n_nodes, int shift, int bits, int buckets, int64_t tiles,
    const uint32_t* __restrict__ counts, const uint32_t* __restrict__ bucket_total,
    uint32_t* __restrict__ bucket_start, uint32_t* __restrict__ valid_count, int64_t* __restrict__ offsets_last,
    Out out, const int32_t* __restrict__ status, int gate) {
  using Codec = ElementCodec<E>;
  __shared__ E elements[kTile + kTile / 32];
  __shared__ uint32_t counters[kCounterWords];
  __shared__ uint32_t tile_start[kMaxBuckets];
  __shared__ uint32_t shift_to_target[kMaxBuckets];
  __shared__ uint32_t wave_totals[kGroupWaves];
  if (gate_closed(status, gate)) return;
  const int64_t limit = element_limit(n, count_limit);
  const int t = threadIdx.x;
  const uint32_t digit_mask = (1u << bits) - 1u;
  const int64_t tile_base = static_cast<int64_t>(blockIdx.x) * kTile;
  const int n_tile = tile_elements(tile_base, limit);
  for (int b = t; b < buckets; b += kThreads) tile_start[b] = 0u;

  // the tile into LDS, in order; out-of-range keys become the largest key
  if constexpr (kPairs) {
    const BufferView key_view = buffer_view(keys32 + (n_tile > 0 ? tile_base : 0), static_cast<int64_t>(n_tile) * 4);
    const BufferView index_view = buffer_view(index32 + (n_tile > 0 ? tile_base : 0), static_cast<int64_t>(n_tile) * 4);
    __syncthreads();  // tile_start is zero
    for (int half = 0; half < 2; ++half) {
      constexpr int kHalf = kItems / 2;
      uint32_t key[kHalf], index[kHalf];
#pragma unroll
      for (int r = 0; r < kHalf; ++r) {
        const uint32_t q = static_cast<uint32_t>((half * kHalf + r) * kThreads + t);
        key[r] = load_u32(key_view, q * 4u);
        index[r] = load_u32(index_view, q * 4u);
      }
#pragma unroll
      for (int r = 0; r < kHalf; ++r) {
        const int q = (half * kHalf + r) * kThreads + t;
        if (q < n_tile) {
          elements[padded(q)] = Codec::make(key[r], index[r]);
          atomicAdd(&tile_start[(key[r] >> shift) & digit_mask], 1u);
        }
      }
    }
  } else {
    const BufferView view = buffer_view(keys64 + (n_tile > 0 ? tile_base : 0), static_cast<int64_t>(n_tile) * 8);
    __syncthreads();  // tile_start is zero
    for (int half = 0; half < 2; ++half) {
      constexpr int kHalf = kItems / 2;
      int64_t raw[kHalf];
#pragma unroll
      for (int r = 0; r < kHalf; ++r)
        raw[r] = load_i64(view, static_cast<uint32_t>((half * kHalf + r) * kThreads + t) * 8u);
#pragma unroll
      for (int r = 0; r < kHalf; ++r) {
        const int q = (half * kHalf + r) * kThreads + t;
        if (q < n_tile) {
          const bool in = static_cast<uint64_t>(raw[r]) < n_nodes;
          const uint32_t key = in ? static_cast<uint32_t>(raw[r]) : Codec::kBadKey;
          elements[padded(q)] = Codec::make(key, static_cast<uint32_t>(q));
          if (in) atomicAdd(&tile_start[(key >> shift) & digit_mask], 1u);
        }
      }
    }
  }
  __syncthreads();
  block_stable_sort<E, kItems>(elements, n_tile, Codec::kKeyShift + shift, bits, counters, wave_totals);

  // bucket starts: every block scans the bucket totals (block 0 publishes them)
  for (int b = t; b < buckets; b += kThreads) shift_to_target[b] = bucket_total[b];
  __syncthreads();
  const uint32_t in_range_total = lds_exclusive_scan(shift_to_target, buckets, 0u, wave_totals);
  if (blockIdx.x == 0) {
    for (int b = t; b < buckets; b += kThreads) bucket_start[b] = shift_to_target[b];
    if (t == 0) {
      bucket_start[buckets] = in_range_total;
      if (valid_count != nullptr) *valid_count = in_range_total;
      if (offsets_last != nullptr) *offsets_last = in_range_total;
    }
  }
  const uint32_t in_tile = lds_exclusive_scan(tile_start, buckets, 0u, wave_totals);
  for (int b = t; b < buckets; b += kThreads)
    shift_to_target[b] += counts[static_cast<int64_t>(b) * tiles + blockIdx.x] - tile_start[b];
  __syncthreads();
  // each bucket's run: sorted position p goes to shift_to_target[b] + p
  for (int p = t; p < static_cast<int>(in_tile); p += kThreads) {
    const E e = elements[padded(p)];
    const uint32_t key = Codec::key(e);
    const uint32_t target = shift_to_target[(key >> shift) & digit_mask] + static_cast<uint32_t>(p);
    const uint32_t index = kPairs ? Codec::low(e) : static_cast<uint32_t>(tile_base) + Codec::low(e);
    // unreachable past the element count: the count pass saw the same elements
    if (static_cast<int64_t>(target) < limit) out.store(target, key, index);
  }
}

// offsets[k] = first position e with key[e] >= k, for k in [0, N], of the
// non-decreasing keys[0, limit): position e writes offsets[k] = e for every k
// in (key[e-1], key[e]] (key[-1] = -1, key[limit] = N), so each entry is
// written once.  Gaps of up to kShortGap entries are filled by their thread;
// longer ones (sparse keys) are listed in LDS and filled by the whole
// workgroup.  With `identity`, also identity[e] = e.  Workgroups `block` of
// `blocks` stride over the list.
struct GapList {
  int64_t low[kThreads];
  int64_t high[kThreads];
  int64_t edge[kThreads];
  int count;
};

template <typename K>
__device__ __forceinline__ void boundary_offsets(const K* __restrict__ keys, int64_t limit, int64_t n_nodes,
                                                 int64_t* __restrict__ offsets, int64_t* __restrict__ identity,
                                                 int64_t block, int64_t blocks, GapList& gaps) {
  const int64_t stride = blocks * kThreads;
  for (int64_t first = block * kThreads; first <= limit; first += stride) {
    if (threadIdx.x == 0) gaps.count = 0;
    __syncthreads();
    const int64_t e = first + threadIdx.x;
    if (identity != nullptr && e < limit) identity[e] = e;
    if (e <= limit) {
      int64_t previous = e > 0 ? static_cast<int64_t>(keys[e - 1]) : -1;
      int64_t current = e < limit ? static_cast<int64_t>(keys[e]) : n_nodes;
      previous = previous < -1 ? -1 : (previous > n_nodes ? n_nodes : previous);
      current = current < -1 ? -1 : (current > n_nodes ? n_nodes : current);
      if (current - previous <= kShortGap) {
        for (int64_t k = previous + 1; k <= current; ++k) offsets[k] = e;
      } else {
        const int slot = atomicAdd(&gaps.count, 1);
        gaps.low[slot] = previous + 1;
        gaps.high[slot] = current;
        gaps.edge[slot] = e;
      }
    }
    __syncthreads();
    const int listed = gaps.count;
    for (int g = 0; g < listed; ++g)
      for (int64_t k = gaps.low[g] + threadIdx.x; k <= gaps.high[g]; k += kThreads) offsets[k] = gaps.edge[g];
    __syncthreads();
  }
}

template <typename K>
__global__ __launch_bounds__(kThreads) void offsets_from_sorted_kernel(const K* __restrict__ keys, int64_t n,
                                                                       const uint32_t* count_limit,
                                                                       int64_t n_nodes,
                                                                       int64_t* __restrict__ offsets,
                                                                       int64_t* __restrict__ identity,
                                                                       const int32_t* __restrict__ status,
                                                                       int gate) {
  __shared__ GapList gaps;
  if (gate_closed(status, gate)) return;
  boundary_offsets(keys, element_limit(n, count_limit), n_nodes, offsets, identity, blockIdx.x, gridDim.x, gaps);
}

// Last launch of the two-level path.  Unsorted keys: one workgroup per bucket
// of 2^fine_bits keys; the fine-digit histogram gives the offsets of the
// bucket's keys, and each chunk of the bucket, sorted stably by the fine
// digit in LDS, places its edge indices in `order`.  Sorted keys: every
// workgroup strides over the keys themselves for the offsets and the identity
// order.
template <typename P>
__global__ __launch_bounds__(kThreads) void finish_kernel(const P* __restrict__ packed,
                                                          const uint32_t* __restrict__ bucket_start, int buckets,
                                                          int fine_bits, const int64_t* __restrict__ keys,
                                                          int64_t n_edges, int64_t n_nodes,
                                                          int64_t* __restrict__ order,
                                                          int64_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ status) {
  __shared__ P elements[kLocalChunk + kLocalChunk / 32];
  __shared__ uint32_t counters[kCounterWords];
  __shared__ uint32_t fine_base[kMaxFine];
  __shared__ uint32_t chunk_start[kMaxFine];
  __shared__ uint32_t wave_totals[kGroupWaves];
  __shared__ GapList gaps;
  if (!(status_of(status) & kFlagUnsorted)) {
    boundary_offsets(keys, n_edges, n_nodes, offsets, order, blockIdx.x, gridDim.x, gaps);
    return;
  }
  const int b = blockIdx.x;
  if (b >= buckets) return;
  const int t = threadIdx.x;
  const int64_t start = bucket_start[b];
  const int64_t end = bucket_start[b + 1];
  const int64_t count = end - start;
  const int fines = 1 << fine_bits;
  const P fine_mask = static_cast<P>(fines - 1);

  // the bucket's fine-digit histogram -> offsets of its keys
  for (int f = t; f < fines; f += kThreads) fine_base[f] = 0u;
  __syncthreads();
  for (int64_t first = 0; first < count; first += kLocalChunk) {
    // a view per chunk keeps every offset small, however long the bucket
    const int in_chunk = static_cast<int>(count - first < kLocalChunk ? count - first : kLocalChunk);
    const BufferView view = buffer_view(packed + start + first, static_cast<int64_t>(in_chunk) * sizeof(P));
    P values[kLocalItems];
#pragma unroll
    for (int r = 0; r < kLocalItems; ++r) {
      const uint32_t offset = static_cast<uint32_t>(r * kThreads + t) * sizeof(P);
      if constexpr (sizeof(P) == 8)
        values[r] = static_cast<P>(load_i64(view, offset));
      else
        values[r] = load_u32(view, offset);
    }
#pragma unroll
    for (int r = 0; r < kLocalItems; ++r)
      if (r * kThreads + t < in_chunk) atomicAdd(&fine_base[static_cast<uint32_t>(values[r] & fine_mask)], 1u);
  }
  __syncthreads();
  lds_exclusive_scan(fine_base, fines, static_cast<uint32_t>(start), wave_totals);
  for (int f = t; f < fines; f += kThreads) {
    const int64_t key = (static_cast<int64_t>(b) << fine_bits) + f;
    if (key < n_nodes) offsets[key] = fine_base[f];
  }
  if (order == nullptr) return;

  for (int64_t first = 0; first < count; first += kLocalChunk) {
    const int in_chunk = static_cast<int>(count - first < kLocalChunk ? count - first : kLocalChunk);
    const BufferView view = buffer_view(packed + start + first, static_cast<int64_t>(in_chunk) * sizeof(P));
    for (int f = t; f < fines; f += kThreads) chunk_start[f] = 0u;
    P values[kLocalItems];
#pragma unroll
    for (int r = 0; r < kLocalItems; ++r) {
      const uint32_t offset = static_cast<uint32_t>(r * kThreads + t) * sizeof(P);
      if constexpr (sizeof(P) == 8)
        values[r] = static_cast<P>(load_i64(view, offset));
      else
        values[r] = load_u32(view, offset);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kLocalItems; ++r) {
      const int q = r * kThreads + t;
      if (q < in_chunk) {
        elements[padded(q)] = values[r];
        atomicAdd(&chunk_start[static_cast<uint32_t>(values[r] & fine_mask)], 1u);
      }
    }
    __syncthreads();
    block_stable_sort<P, kLocalItems>(elements, in_chunk, 0, fine_bits, counters, wave_totals);
    lds_exclusive_scan(chunk_start, fines, 0u, wave_totals);
    for (int p = t; p < in_chunk; p += kThreads) {
      const P e = elements[padded(p)];
      const uint32_t f = static_cast<uint32_t>(e & fine_mask);
      const int64_t target = static_cast<int64_t>(fine_base[f]) + (p - static_cast<int64_t>(chunk_start[f]));
      // unreachable outside the bucket: its fine digits were counted from the same elements
      if (target >= start && target < end) order[target] = static_cast<int64_t>(e >> fine_bits);
    }
    __syncthreads();
    // the next chunk's elements of digit f follow this chunk's
    for (int f = t; f < fines; f += kThreads) {
      const uint32_t next = f + 1 < fines ? chunk_start[f + 1] : static_cast<uint32_t>(in_chunk);
      fine_base[f] += next - chunk_start[f];
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kThreads) void widen_kernel(const uint32_t* __restrict__ index, int64_t n,
                                                         const uint32_t* count_limit, int64_t* __restrict__ order,
                                                         const int32_t* __restrict__ status, int gate) {
  if (gate_closed(status, gate)) return;
  const int64_t limit = element_limit(n, count_limit);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < limit; i += stride)
    order[i] = static_cast<int64_t>(index[i]);
}

// Range and sharing checks of the GIE radial slots (one block of 64).  Also
// ORs the largest number of rows that read one slot, capped at 255, into
// bits 16..23 of the status word (kSlotRowsShift).
__global__ __launch_bounds__(64) void slot_check_kernel(const int64_t* __restrict__ radial_slot, int64_t n_rows,
                                                        int64_t n_radial, int32_t* __restrict__ status) {
  __shared__ int most;
  if (threadIdx.x == 0) most = 0;
  __syncthreads();
  int32_t local = 0;
  int rows_of_slot = 0;
  for (int64_t r = threadIdx.x; r < n_rows; r += blockDim.x) {
    const int64_t slot = radial_slot[r];
    if (static_cast<uint64_t>(slot) >= static_cast<uint64_t>(n_radial)) local |= kFlagSlotRange;
    int64_t readers = 0;
    for (int64_t other = 0; other < n_rows; ++other) readers += radial_slot[other] == slot ? 1 : 0;
    if (readers > 1) local |= kFlagSlotShared;
    const int capped = readers > 255 ? 255 : static_cast<int>(readers);
    rows_of_slot = capped > rows_of_slot ? capped : rows_of_slot;
  }
  atomicMax(&most, rows_of_slot);
  __syncthreads();
  if (threadIdx.x == 0) local |= most << kSlotRowsShift;
  if (local != 0) atomicOr(status, local);
}

// ---------------------------------------------------------------------------
// host: the plan of one build and its workspace
// ---------------------------------------------------------------------------

unsigned int grid_stride_blocks(int64_t items, int64_t cap = 8192) {
  const int64_t wanted = (items + 255) / 256;
  return static_cast<unsigned int>(wanted < 1 ? 1 : (wanted > cap ? cap : wanted));
}

struct Plan {
  int64_t n_edges = 0;
  int64_t n_nodes = 0;
  int bits = 0;           // bits of the largest key, N - 1
  int64_t tiles = 0;
  bool two_level = true;  // coarse scatter + bucket-local pass; otherwise LSD passes
  // two-level path
  int bucket_bits = 0;
  int fine_bits = 0;
  int buckets = 1;
  bool wide = false;      // packed as uint64 (index << fine_bits does not fit 32 bits)
  bool narrow_elements = false;  // the scatter's LDS elements fit 32 bits (keys of at most 19 bits)
  // LSD path
  int passes = 0;
  int digit_bits = 0;

  Plan(int64_t edges, int64_t nodes) : n_edges(edges), n_nodes(nodes) {
    while (bits < 32 && (int64_t(1) << bits) < nodes) ++bits;
    tiles = (edges + kTile - 1) / kTile;
    bucket_bits = bits < kDigitBits ? bits : kDigitBits;
    fine_bits = bits - bucket_bits;
    two_level = fine_bits <= kFineBitsMax;
    if (two_level) {
      buckets = static_cast<int>((nodes + (int64_t(1) << fine_bits) - 1) >> fine_bits);
      wide = edges > 0 && ((static_cast<uint64_t>(edges) - 1) << fine_bits) > 0xffffffffull;
      narrow_elements = bits <= 19;
    } else {
      passes = (bits + kDigitBits - 1) / kDigitBits;
      digit_bits = (bits + passes - 1) / passes;
    }
  }
  int pass_shift(int p) const { return p * digit_bits; }
  int pass_bits(int p) const { return bits - p * digit_bits < digit_bits ? bits - p * digit_bits : digit_bits; }
  int pass_buckets(int p) const {
    const int64_t top = ((n_nodes - 1) >> pass_shift(p)) + 1;
    const int64_t all = int64_t(1) << pass_bits(p);
    return static_cast<int>(top < all ? top : all);
  }
};

struct Scratch {
  int32_t* flags = nullptr;       // the status word when the caller passes none
  uint32_t* valid_count = nullptr;
  uint32_t* counts = nullptr;     // [buckets of the pass][tiles]
  uint32_t* bucket_total = nullptr;
  uint32_t* bucket_start = nullptr;
  void* packed = nullptr;         // two-level path
  uint32_t* keys[2] = {nullptr, nullptr};   // LSD ping-pong
  uint32_t* index[2] = {nullptr, nullptr};
};

size_t scratch_bytes(const Plan& plan) {
  const size_t edges = static_cast<size_t>(plan.n_edges > 0 ? plan.n_edges : 1);
  const size_t tiles = static_cast<size_t>(plan.tiles > 0 ? plan.tiles : 1);
  size_t bytes = 256 + 256 + round_up_256(tiles * kMaxBuckets * 4) + round_up_256(kMaxBuckets * 4) +
                 round_up_256((kMaxBuckets + 1) * 4);
  if (plan.two_level)
    bytes += round_up_256(edges * (plan.wide ? 8 : 4));
  else
    bytes += 4 * round_up_256(edges * 4);
  return bytes;
}

bool carve(void* workspace, size_t bytes, const Plan& plan, Scratch& out) {
  if (workspace == nullptr || bytes < scratch_bytes(plan)) return false;
  const size_t edges = static_cast<size_t>(plan.n_edges > 0 ? plan.n_edges : 1);
  const size_t tiles = static_cast<size_t>(plan.tiles > 0 ? plan.tiles : 1);
  Carver carver{static_cast<char*>(workspace), bytes};
  out.flags = carver.take<int32_t>(1);
  out.valid_count = carver.take<uint32_t>(1);
  out.counts = carver.take<uint32_t>(tiles * kMaxBuckets);
  out.bucket_total = carver.take<uint32_t>(kMaxBuckets);
  out.bucket_start = carver.take<uint32_t>(kMaxBuckets + 1);
  if (plan.two_level) {
    out.packed = carver.take<char>(edges * (plan.wide ? 8 : 4));
    return out.flags && out.valid_count && out.counts && out.bucket_total && out.bucket_start && out.packed;
  }
  for (int k = 0; k < 2; ++k) {
    out.keys[k] = carver.take<uint32_t>(edges);
    out.index[k] = carver.take<uint32_t>(edges);
  }
  return out.flags && out.valid_count && out.counts && out.bucket_total && out.bucket_start && out.keys[0] &&
         out.keys[1] && out.index[0] && out.index[1];
}

int check_sizes(int64_t n_edges, int64_t n_nodes, const char* what) {
  if (n_edges < 0) return fail(DPA4K_EINVAL, "%s: negative edge count", what);
  if (n_nodes <= 0) return fail(DPA4K_EINVAL, "%s require a positive node count", what);
  if (n_nodes > (int64_t(1) << 32)) return fail(DPA4K_EINVAL, "%s supports at most 2^32 nodes", what);
  if (n_edges > 0xffffffffLL) return fail(DPA4K_EINVAL, "%s supports fewer than 2^32 edges", what);
  return DPA4K_OK;
}

// Enqueues the whole build: the status word cleared, then set by the count
// pass; offsets always; the order when `order` is given.  No host
// synchronisation.  Radial-slot checks of the GIE grouping when n_rows > 0.
int enqueue_build(const int64_t* keys, const Plan& plan, int64_t* offsets, int64_t* order, int32_t* status,
                  const int64_t* radial_slot, int64_t n_rows, int64_t n_radial, const Scratch& s,
                  hipStream_t stream) {
  clear_word_kernel<<<1, 64, 0, stream>>>(status);
  if (int code = launched("clear_word_kernel")) return code;
  if (n_rows > 0) {
    slot_check_kernel<<<1, 64, 0, stream>>>(radial_slot, n_rows, n_radial, status);
    if (int code = launched("slot_check_kernel")) return code;
  }
  if (plan.n_edges == 0) return zero_fill(offsets, static_cast<size_t>(plan.n_nodes + 1) * sizeof(int64_t), stream);

  const uint64_t nodes = static_cast<uint64_t>(plan.n_nodes);
  const unsigned int tiles = static_cast<unsigned int>(plan.tiles);
  const auto scan = [&](int buckets) {
    row_scan_kernel<<<buckets, kThreads, 0, stream>>>(s.counts, plan.tiles, s.bucket_total, status, kIfUnsorted);
    return launched("row_scan_kernel");
  };
  // sorted keys: the finish launch's boundary path (its grid also strides over the keys)
  const int64_t boundary_blocks = std::min<int64_t>((plan.n_edges + kThreads) / kThreads, 2048);
  if (plan.two_level) {
    const int shift = plan.fine_bits, bits = plan.bucket_bits, buckets = plan.buckets;
    tile_count_kernel<false, true><<<tiles, kThreads, 0, stream>>>(keys, nullptr, plan.n_edges, nullptr, nodes, shift,
                                                                   bits, buckets, plan.tiles, s.counts, status,
                                                                   kAlways);
    if (int code = launched("tile_count_kernel")) return code;
    if (int code = scan(buckets)) return code;
    const unsigned int finish_blocks = static_cast<unsigned int>(std::max<int64_t>(buckets, boundary_blocks));
    const auto scatter = [&](auto out, auto element) {
      using E = decltype(element);
      tile_scatter_kernel<E, false, decltype(out)><<<tiles, kThreads, 0, stream>>>(
          keys, nullptr, nullptr, plan.n_edges, nullptr, nodes, shift, bits, buckets, plan.tiles, s.counts,
          s.bucket_total, s.bucket_start, nullptr, offsets + plan.n_nodes, out, status, kIfUnsorted);
      return launched("tile_scatter_kernel");
    };
    if (plan.wide) {
      const PackedOut<uint64_t> packed{static_cast<uint64_t*>(s.packed), plan.fine_bits};
      if (int code = plan.narrow_elements ? scatter(packed, uint32_t(0)) : scatter(packed, uint64_t(0))) return code;
      finish_kernel<uint64_t><<<finish_blocks, kThreads, 0, stream>>>(
          static_cast<const uint64_t*>(s.packed), s.bucket_start, buckets, plan.fine_bits, keys, plan.n_edges,
          plan.n_nodes, order, offsets, status);
    } else {
      const PackedOut<uint32_t> packed{static_cast<uint32_t*>(s.packed), plan.fine_bits};
      if (int code = plan.narrow_elements ? scatter(packed, uint32_t(0)) : scatter(packed, uint64_t(0))) return code;
      finish_kernel<uint32_t><<<finish_blocks, kThreads, 0, stream>>>(
          static_cast<const uint32_t*>(s.packed), s.bucket_start, buckets, plan.fine_bits, keys, plan.n_edges,
          plan.n_nodes, order, offsets, status);
    }
    return launched("finish_kernel");
  }

  // least significant digit first; pass 0 reads the caller's keys and checks them
  int current = 0;
  for (int p = 0; p < plan.passes; ++p) {
    const int shift = plan.pass_shift(p), bits = plan.pass_bits(p), buckets = plan.pass_buckets(p);
    const PairsOut target{s.keys[current], s.index[current]};
    if (p == 0) {
      tile_count_kernel<false, true><<<tiles, kThreads, 0, stream>>>(keys, nullptr, plan.n_edges, nullptr, nodes,
                                                                     shift, bits, buckets, plan.tiles, s.counts,
                                                                     status, kAlways);
      if (int code = launched("tile_count_kernel")) return code;
      if (int code = scan(buckets)) return code;
      tile_scatter_kernel<uint64_t, false, PairsOut><<<tiles, kThreads, 0, stream>>>(
          keys, nullptr, nullptr, plan.n_edges, nullptr, nodes, shift, bits, buckets, plan.tiles, s.counts,
          s.bucket_total, s.bucket_start, s.valid_count, nullptr, target, status, kIfUnsorted);
    } else {
      const uint32_t* source_keys = s.keys[1 - current];
      const uint32_t* source_index = s.index[1 - current];
      tile_count_kernel<true, false><<<tiles, kThreads, 0, stream>>>(nullptr, source_keys, plan.n_edges,
                                                                     s.valid_count, nodes, shift, bits, buckets,
                                                                     plan.tiles, s.counts, status, kIfUnsorted);
      if (int code = launched("tile_count_kernel")) return code;
      if (int code = scan(buckets)) return code;
      tile_scatter_kernel<uint64_t, true, PairsOut><<<tiles, kThreads, 0, stream>>>(
          nullptr, source_keys, source_index, plan.n_edges, s.valid_count, nodes, shift, bits, buckets, plan.tiles,
          s.counts, s.bucket_total, s.bucket_start, nullptr, nullptr, target, status, kIfUnsorted);
    }
    if (int code = launched("tile_scatter_kernel")) return code;
    current = 1 - current;
  }
  const int last = 1 - current;
  offsets_from_sorted_kernel<uint32_t><<<grid_stride_blocks(plan.n_edges + 1), kThreads, 0, stream>>>(
      s.keys[last], plan.n_edges, s.valid_count, plan.n_nodes, offsets, nullptr, status, kIfUnsorted);
  if (int code = launched("offsets_from_sorted_kernel")) return code;
  if (order != nullptr) {
    widen_kernel<<<grid_stride_blocks(plan.n_edges), kThreads, 0, stream>>>(s.index[last], plan.n_edges,
                                                                            s.valid_count, order, status,
                                                                            kIfUnsorted);
    if (int code = launched("widen_kernel")) return code;
  }
  offsets_from_sorted_kernel<int64_t><<<static_cast<unsigned int>(boundary_blocks), kThreads, 0, stream>>>(
      keys, plan.n_edges, nullptr, plan.n_nodes, offsets, order, status, kIfSorted);
  return launched("offsets_from_sorted_kernel");
}

// Copies the flags word to the host once the stream has drained.
int read_flags(const int32_t* flags, int32_t& host, hipStream_t stream) {
  if (int s = hip_status(hipMemcpyAsync(&host, flags, sizeof(int32_t), hipMemcpyDeviceToHost, stream),
                         "hipMemcpyAsync(flags)"))
    return s;
  return hip_status(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

int prepare(int64_t n_edges, int64_t n_nodes, void* workspace, size_t workspace_bytes, const char* what,
            Scratch& scratch) {
  const Plan plan(n_edges, n_nodes);
  if (!carve(workspace, workspace_bytes, plan, scratch))
    return fail(DPA4K_EWORKSPACE, "%s: workspace of %zu bytes is smaller than %zu", what, workspace_bytes,
                scratch_bytes(plan));
  return DPA4K_OK;
}

int segment_offsets_impl(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* offsets,
                         int32_t* status, void* workspace, size_t workspace_bytes, hipStream_t stream,
                         int32_t* host_flags) {
  if (int s = check_sizes(n_edges, n_nodes, "segment offsets")) return s;
  if (offsets == nullptr || (n_edges > 0 && keys == nullptr)) return fail(DPA4K_EINVAL, "segment offsets: null pointer");
  Scratch scratch;
  if (int s = prepare(n_edges, n_nodes, workspace, workspace_bytes, "segment offsets", scratch)) return s;
  int32_t* flags = status != nullptr ? status : scratch.flags;
  if (int s = enqueue_build(keys, Plan(n_edges, n_nodes), offsets, nullptr, flags, nullptr, 0, 0, scratch, stream))
    return s;
  if (host_flags == nullptr) return DPA4K_OK;
  if (int s = read_flags(flags, *host_flags, stream)) return s;
  if (*host_flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "destination values must be within the node range");
  return DPA4K_OK;
}

int group_by_key_impl(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* order, int64_t* offsets,
                      int32_t* status, void* workspace, size_t workspace_bytes, hipStream_t stream,
                      int32_t* host_flags) {
  if (int s = check_sizes(n_edges, n_nodes, "group_by_source")) return s;
  if (offsets == nullptr || (n_edges > 0 && (keys == nullptr || order == nullptr)))
    return fail(DPA4K_EINVAL, "group_by_source: null pointer");
  Scratch scratch;
  if (int s = prepare(n_edges, n_nodes, workspace, workspace_bytes, "group_by_source", scratch)) return s;
  int32_t* flags = status != nullptr ? status : scratch.flags;
  if (int s = enqueue_build(keys, Plan(n_edges, n_nodes), offsets, order, flags, nullptr, 0, 0, scratch, stream))
    return s;
  if (host_flags == nullptr) return DPA4K_OK;
  if (int s = read_flags(flags, *host_flags, stream)) return s;
  if (*host_flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "source values must be within the node range");
  return DPA4K_OK;
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" size_t dpa4k_segment_offsets_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return n_nodes > 0 && n_edges >= 0 ? scratch_bytes(Plan(n_edges, n_nodes)) : 0;
}

extern "C" int dpa4k_segment_offsets(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* offsets,
                                     void* workspace, size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  clear_error();
  int32_t flags = 0;
  return segment_offsets_impl(keys, n_edges, n_nodes, offsets, nullptr, workspace, workspace_bytes,
                              as_stream(stream_handle), &flags);
}

extern "C" int dpa4k_segment_offsets_async(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* offsets,
                                           int32_t* status, void* workspace, size_t workspace_bytes,
                                           dpa4k_stream_t stream_handle) {
  clear_error();
  if (status == nullptr) return fail(DPA4K_EINVAL, "segment offsets: the asynchronous form needs a status word");
  return segment_offsets_impl(keys, n_edges, n_nodes, offsets, status, workspace, workspace_bytes,
                              as_stream(stream_handle), nullptr);
}

extern "C" size_t dpa4k_group_by_key_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return n_nodes > 0 && n_edges >= 0 ? scratch_bytes(Plan(n_edges, n_nodes)) : 0;
}

extern "C" int dpa4k_group_by_key(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* order,
                                  int64_t* offsets, void* workspace, size_t workspace_bytes,
                                  dpa4k_stream_t stream_handle) {
  clear_error();
  int32_t flags = 0;
  return group_by_key_impl(keys, n_edges, n_nodes, order, offsets, nullptr, workspace, workspace_bytes,
                           as_stream(stream_handle), &flags);
}

extern "C" int dpa4k_group_by_key_async(const int64_t* keys, int64_t n_edges, int64_t n_nodes, int64_t* order,
                                        int64_t* offsets, int32_t* status, void* workspace, size_t workspace_bytes,
                                        dpa4k_stream_t stream_handle) {
  clear_error();
  if (status == nullptr) return fail(DPA4K_EINVAL, "group_by_source: the asynchronous form needs a status word");
  return group_by_key_impl(keys, n_edges, n_nodes, order, offsets, status, workspace, workspace_bytes,
                           as_stream(stream_handle), nullptr);
}

extern "C" size_t dpa4k_gie_group_workspace_size(int64_t n_edges, int64_t n_nodes) {
  return dpa4k_group_by_key_workspace_size(n_edges, n_nodes);
}

extern "C" int dpa4k_gie_group(const int64_t* dst, const int64_t* radial_slot, int64_t n_edges, int64_t n_nodes,
                               int64_t n_rows, int64_t n_radial, int64_t* offsets, int64_t* order,
                               int32_t* host_info, void* workspace, size_t workspace_bytes,
                               dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_sizes(n_edges, n_nodes, "GIE grouping")) return s;
  if (n_rows < 0 || n_radial < 0) return fail(DPA4K_EINVAL, "GIE grouping: negative sizes");
  if (offsets == nullptr || (n_edges > 0 && (dst == nullptr || order == nullptr)) ||
      (n_rows > 0 && radial_slot == nullptr))
    return fail(DPA4K_EINVAL, "GIE grouping: null pointer");
  Scratch scratch;
  if (int s = prepare(n_edges, n_nodes, workspace, workspace_bytes, "GIE grouping", scratch)) return s;
  hipStream_t stream = as_stream(stream_handle);
  // the order buffer receives the identity when dst is already sorted; the
  // host then passes no order to the kernels (bit 1 of host_info)
  if (int s = enqueue_build(dst, Plan(n_edges, n_nodes), offsets, order, scratch.flags, radial_slot, n_rows,
                            n_radial, scratch, stream))
    return s;
  int32_t flags = 0;
  if (int s = read_flags(scratch.flags, flags, stream)) return s;
  if (flags & kFlagOutOfRange) return fail(DPA4K_EINVAL, "GIE dst values must be within the node range");
  if (flags & kFlagSlotRange) return fail(DPA4K_EINVAL, "GIE radial_slot values must be within the radial range");
  const bool sorted = !(flags & kFlagUnsorted);
  if (host_info != nullptr)
    *host_info = (sorted ? 1 : 0) | ((flags & kFlagSlotShared) ? 0 : 2) | (flags & (0xff << kSlotRowsShift));
  return DPA4K_OK;
}

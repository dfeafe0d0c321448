// CSR construction on the device: offsets, stable grouping order and the GIE
// grouping step.
//
// Restates python/kernels/segment.py:46-71 of the reference
// (segment_offsets = [0] ++ cumsum(bincount(keys)), group_by_source = stable
// argsort + offsets) as a bounded-key counting sort, written for wave64.
// Keys of up to 20 bits take two levels: a coarse digit (the key's high bits,
// at most 1024 buckets) and a fine digit (its low bits).
//
// Packed 32-bit elements with fine digits of at most 7 bits and at most 2048
// tiles (N <= 2^17 and E <= 2^24) take two launches: tile_group_kernel groups
// each tile by the coarse digit in place and writes its row of runs, and
// bucket_gather_kernel gathers each bucket's runs and ranks them by the fine
// digit (the section "grouped two-level path" below).  Other shapes take four:
//
//   count     one pass over the int64 keys in tiles of 8192: the range and
//             sortedness checks (the reference's dst.min()/dst.max() test),
//             and each tile's histogram of the coarse digit (the key's high
//             bits, at most 1024 buckets) with one LDS atomic per run of
//             equal digits in a wave;
//   scan      one workgroup per bucket scans the bucket's counts over the
//             tiles: every tile learns where its run of each bucket starts;
//   scatter   each wave of a tile's workgroup ranks its contiguous share of
//             the tile stably by digit (a wave-level multisplit: one ballot
//             per digit bit finds the lanes with equal digits, mbcnt counts
//             the lower ones, and the group's leader advances the wave's LDS
//             counter of the digit); the counts, scanned over the waves and
//             the digits, place every element in the tile sorted by digit in
//             LDS, and each bucket's run leaves contiguously, packed as
//             (index << fine_bits | fine digit) in 32 bits when it fits.
//             Tiles are dealt to XCDs in contiguous ranges, so the counts of
//             neighbouring tiles share their L2;
//   finish    one workgroup per bucket: the same multisplit by the fine digit
//             (the key's low bits), chunk by chunk, gives the offsets of the
//             bucket's keys and places its edge indices in `order`.  When
//             the keys were already sorted (DeepMD's layout) the same launch
//             instead takes the offsets from the boundaries of the sorted
//             list and writes the identity order, and the count is the only
//             pass.
//
// Keys of more than 20 bits take least-significant-digit passes of the same
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

constexpr int kThreads = 512;
constexpr int kGroupWaves = kThreads / 64;
constexpr int kItems = 16;                             // elements per thread in a tile
constexpr int kTile = kThreads * kItems;               // 8192 elements per count/scatter tile
constexpr int kDigitBits = 10;                         // at most 1024 buckets per scatter pass
constexpr int kMaxBuckets = 1 << kDigitBits;
constexpr int kFineBitsMax = 10;                       // the two-level path: keys of up to 20 bits
constexpr int kMaxFine = 1 << kFineBitsMax;
constexpr int kLocalItems = 16;
constexpr int kLocalChunk = kThreads * kLocalItems;    // 8192 elements per bucket-local round
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

// Loads of data read once (cache policy nt: streamed rather than kept in L2).
__device__ __forceinline__ int64_t load_i64_streamed(BufferView view, uint32_t offset) {
  const u32x2 raw = __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(offset), 0, kNonTemporal);
  return __builtin_bit_cast(int64_t, raw);
}


// A DPP move of `value` (control kCtrl, rows kRowMask); lanes whose source
// lies outside their row, and rows outside the mask, read 0.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t value) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(value), kCtrl, kRowMask, 0xf, true));
}

// Inclusive scan of one value per lane over the wave on the VALU: row_shr 1,
// 2, 4, 8 scan each row of 16 lanes; row_bcast:15 adds lane 15's total to row
// 1 (and lane 47's to row 3), row_bcast:31 adds lane 31's to rows 2 and 3.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t value) {
  uint32_t inclusive = value;
  inclusive += dpp_or_zero<0x111, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x112, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x114, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x118, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x142, 0xa>(inclusive);
  inclusive += dpp_or_zero<0x143, 0xc>(inclusive);
  return inclusive;
}

// Exclusive scan of one value per thread over a workgroup of kT threads;
// `total` gets the sum.  Every thread must call it.
template <int kT = kThreads>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t value, uint32_t* wave_totals, uint32_t& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // inclusive scan of the wave on the VALU: row_shr 1, 2, 4, 8 scan each row
  // of 16 lanes; row_bcast:15 adds lane 15's total to row 1 (and lane 47's
  // to row 3), row_bcast:31 adds lane 31's to rows 2 and 3
  uint32_t inclusive = value;
  inclusive += dpp_or_zero<0x111, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x112, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x114, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x118, 0xf>(inclusive);
  inclusive += dpp_or_zero<0x142, 0xa>(inclusive);
  inclusive += dpp_or_zero<0x143, 0xc>(inclusive);
  if (lane == 63) wave_totals[wave] = inclusive;
  __syncthreads();
  uint32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kT / 64; ++w) {
    const uint32_t part = wave_totals[w];
    before += w < wave ? part : 0u;
    sum += part;
  }
  __syncthreads();
  total = sum;
  return before + inclusive - value;
}

// block_exclusive_scan of two values per thread at once (one pair of
// barriers): returns the exclusive scan of `first`; `totals` gets both sums.
// `wave_totals` holds 2 kT / 64 words.  Every thread must call it.
template <int kT = kThreads>
__device__ __forceinline__ uint32_t block_exclusive_scan2(uint32_t first, uint32_t second, uint32_t* wave_totals,
                                                          uint32_t& first_total, uint32_t& second_total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t a = first, b = second;
  a += dpp_or_zero<0x111, 0xf>(a);
  b += dpp_or_zero<0x111, 0xf>(b);
  a += dpp_or_zero<0x112, 0xf>(a);
  b += dpp_or_zero<0x112, 0xf>(b);
  a += dpp_or_zero<0x114, 0xf>(a);
  b += dpp_or_zero<0x114, 0xf>(b);
  a += dpp_or_zero<0x118, 0xf>(a);
  b += dpp_or_zero<0x118, 0xf>(b);
  a += dpp_or_zero<0x142, 0xa>(a);
  b += dpp_or_zero<0x142, 0xa>(b);
  a += dpp_or_zero<0x143, 0xc>(a);
  b += dpp_or_zero<0x143, 0xc>(b);
  if (lane == 63) {
    wave_totals[2 * wave] = a;
    wave_totals[2 * wave + 1] = b;
  }
  __syncthreads();
  uint32_t before = 0, sum_a = 0, sum_b = 0;
#pragma unroll
  for (int w = 0; w < kT / 64; ++w) {
    const uint32_t part = wave_totals[2 * w];
    before += w < wave ? part : 0u;
    sum_a += part;
    sum_b += wave_totals[2 * w + 1];
  }
  __syncthreads();
  first_total = sum_a;
  second_total = sum_b;
  return before + a - first;
}

// In-place exclusive scan of values[0, n) in LDS (plus `base`) by a
// workgroup of kT threads; returns the total.  Every thread must call it.
template <int kT = kThreads>
__device__ __forceinline__ uint32_t lds_exclusive_scan(uint32_t* values, int n, uint32_t base,
                                                       uint32_t* wave_totals) {
  const int per = (n + kT - 1) / kT;
  const int first = threadIdx.x * per;
  uint32_t sum = 0;
  for (int i = 0; i < per; ++i)
    if (first + i < n) sum += values[first + i];
  uint32_t total = 0;
  uint32_t running = base + block_exclusive_scan<kT>(sum, wave_totals, total);
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
// wave-level multisplit
// ---------------------------------------------------------------------------
//
// A wave ranks its 64 elements stably by a digit of up to kDigitBits bits.
// One ballot per digit bit leaves every lane the mask of the active lanes
// that share its digit; its rank among them is the number of lower lanes
// (mbcnt).  The wave's own LDS counter of the digit holds the number of equal
// digits the wave met in its earlier rounds; the lowest lane of the group,
// its leader, advances it by the group's size.  Either every lane reads the
// counter and the leader then stores it (each wave has counters of its own
// and a wave's LDS operations take effect in program order, so no atomic is
// needed), or the leader advances it atomically and broadcasts the old value.
// A lane's rank among the equal digits of the wave's whole range is that
// value plus its rank in the round.

// Per digit bit: m = the bit spread over the word (v_bfe_i32: all ones or
// zero), its ballot (v_cmp of m itself), and per half `differ |= ballot ^ m`
// (the lanes whose bit differs from this lane's) as one v_bitop3: four VALU
// operations a bit.
template <int kBits>
__device__ __forceinline__ uint64_t lanes_with_digit(uint32_t digit, bool active) {
  constexpr uint32_t kOrOfXor = 0xF6;  // v_bitop3 table of a | (b ^ c)
  constexpr int kNotEqual = 33;        // the integer predicate "ne" of the compare builtin
  uint32_t differ_lo = 0u, differ_hi = 0u;
#pragma unroll
  for (int i = 0; i < kBits; ++i) {
    const uint32_t m = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int>(digit), i, 1));
    const uint64_t with = __builtin_amdgcn_uicmp(m, 0u, kNotEqual);
    differ_lo = __builtin_amdgcn_bitop3_b32(differ_lo, static_cast<uint32_t>(with), m, kOrOfXor);
    differ_hi = __builtin_amdgcn_bitop3_b32(differ_hi, static_cast<uint32_t>(with >> 32), m, kOrOfXor);
  }
  const uint64_t same = ~((static_cast<uint64_t>(differ_hi) << 32) | differ_lo) & __ballot(active);
  return active ? same : 0ull;
}

// The same mask for an active lane, without clearing it for inactive ones:
// `active_lanes` is the ballot of the active lanes.
template <int kBits>
__device__ __forceinline__ uint64_t lanes_with_digit_unmasked(uint32_t digit, uint64_t active_lanes) {
  constexpr uint32_t kOrOfXor = 0xF6;  // v_bitop3 table of a | (b ^ c)
  constexpr int kNotEqual = 33;        // the integer predicate "ne" of the compare builtin
  uint32_t differ_lo = 0u, differ_hi = 0u;
#pragma unroll
  for (int i = 0; i < kBits; ++i) {
    const uint32_t m = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int>(digit), i, 1));
    const uint64_t with = __builtin_amdgcn_uicmp(m, 0u, kNotEqual);
    differ_lo = __builtin_amdgcn_bitop3_b32(differ_lo, static_cast<uint32_t>(with), m, kOrOfXor);
    differ_hi = __builtin_amdgcn_bitop3_b32(differ_hi, static_cast<uint32_t>(with >> 32), m, kOrOfXor);
  }
  return ~((static_cast<uint64_t>(differ_hi) << 32) | differ_lo) & active_lanes;
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// rank[r] = the rank of this lane's round-r element among the equal digits
// the wave meets before it (its earlier rounds, then the lower lanes of round
// r); digit(r) has at most kBits bits, `valid` has bit r for an element in
// round r, and `counter` is the wave's [digit] array, advanced by the call.
// Every lane of the wave must call it.
// kLeaderStores: every lane reads the counter and the leader stores it
// advanced; otherwise the leader advances it with an atomic and broadcasts
// the old value (fewer live registers where a kernel is close to spilling).
template <int kBits, int kRounds, bool kLeaderStores, typename DigitOf>
__device__ __forceinline__ void wave_split_ranks(DigitOf digit, uint32_t valid, uint32_t* counter,
                                                 uint32_t (&rank)[kRounds]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const bool active = ((valid >> r) & 1u) != 0u;
    const uint64_t same = lanes_with_digit<kBits>(digit(r), active);
    const uint32_t below = lanes_below(same);
    const uint32_t size = static_cast<uint32_t>(__popcll(same));
    if constexpr (kLeaderStores) {
      // digits are masked, so every lane's read is in range; the leader's
      // store follows the wave's read in LDS order
      const uint32_t before = counter[digit(r)];
      if (active && below == 0u) counter[digit(r)] = before + size;
      rank[r] = before + below;
    } else {
      uint32_t before = 0u;
      if (active && below == 0u) before = atomicAdd(&counter[digit(r)], size);
      const int leader = active ? __builtin_ctzll(same) : lane;
      rank[r] = static_cast<uint32_t>(__shfl(static_cast<int>(before), leader, 64)) + below;
    }
  }
}

// In place over digits [0, digits): the per-wave counts of a workgroup of kT
// threads become the counts of the earlier waves, and `total[d]` gets the
// digit's count over all waves.
template <int kT = kThreads>
__device__ __forceinline__ void wave_prefix(uint32_t* wave_count, int stride, int digits, uint32_t* total) {
  for (int d = threadIdx.x; d < digits; d += kT) {
    uint32_t running = 0u;
#pragma unroll
    for (int w = 0; w < kT / 64; ++w) {
      const uint32_t count = wave_count[w * stride + d];
      wave_count[w * stride + d] = running;
      running += count;
    }
    total[d] = running;
  }
}

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(64) void clear_word_kernel(int32_t* __restrict__ word) {
  if (threadIdx.x == 0) *word = 0;
}

// A tile of the keys (the caller's int64 keys, or the uint32 keys of an
// earlier pass): element q of the tile is q = kThreads r + thread for
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
// Lane l receives lane l - 1's value (wave_shr:1; lane 0 keeps `fill`) or
// lane l + 1's (wave_shl:1; lane 63 keeps `fill`): a DPP move on the VALU,
// where __shfl_up/__shfl_down would each take an LDS round trip.
__device__ __forceinline__ uint32_t from_lane_below(uint32_t value, uint32_t fill) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(fill), static_cast<int>(value), 0x138, 0xf, 0xf, false));
}
__device__ __forceinline__ uint32_t from_lane_above(uint32_t value, uint32_t fill) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(fill), static_cast<int>(value), 0x130, 0xf, 0xf, false));
}

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
      uint32_t next = from_lane_above(tile.key[r], 0u);
      uint32_t next_ok = from_lane_above((tile.ok >> r) & 1u, 0u);
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
  // tiles dealt to XCDs in contiguous ranges: a line of a bucket's counts
  // (consecutive tiles) is written, and later read, within one L2
  const unsigned int tile_index = xcd_block(blockIdx.x, gridDim.x);
  const int64_t tile_base = static_cast<int64_t>(tile_index) * kTile;
  const uint32_t digit_mask = (1u << bits) - 1u;
  TileKeys tile;
  int32_t local = 0;
  if constexpr (kPairs)
    load_keys32(keys32, tile_base, limit, tile);
  else
    load_keys64<kCheck>(keys64, tile_base, limit, n_nodes, tile, local, first_of_wave, first_ok);
  __syncthreads();
  // LDS atomics, one per run of equal digits among a round's 64 consecutive
  // elements (sorted or clustered keys would otherwise queue on one counter)
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const bool valid = ((tile.ok >> r) & 1u) != 0u;
    const uint32_t digit = (tile.key[r] >> shift) & digit_mask;
    const uint32_t previous = from_lane_below(digit, 0u);  // lane 0 is a head whatever it holds
    const bool previous_valid = from_lane_below(valid ? 1u : 0u, 0u) != 0u;
    const bool head = valid && (lane == 0 || !previous_valid || previous != digit);
    // a run ends at the next head or invalid element
    const uint64_t stops = __ballot(head || !valid);
    const uint64_t after = stops & ~((2ull << lane) - 1ull);
    const int next = after == 0ull ? 64 : __builtin_ctzll(after);
    if (head) atomicAdd(&histogram[digit], static_cast<uint32_t>(next - lane));
  }
  if constexpr (kCheck) {
    const int32_t found = (__syncthreads_or(local & kFlagOutOfRange) ? kFlagOutOfRange : 0) |
                          (__syncthreads_or(local & kFlagUnsorted) ? kFlagUnsorted : 0);
    if (threadIdx.x == 0 && found != 0 &&
        (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & found) != found)
      atomicOr(status, found);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < buckets; b += kThreads)
    counts[static_cast<int64_t>(b) * tiles + tile_index] = histogram[b];
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

// Elements of the scatter's sorted tile in LDS.  32-bit: key in bits
// [0, 19), position in the tile in [19, 32) (keys of at most 19 bits);
// 64-bit: key in the high word, the position (or, for pairs, the edge index)
// in the low word.
template <typename E>
struct ElementCodec;

template <>
struct ElementCodec<uint32_t> {
  __device__ static uint32_t make(uint32_t key, uint32_t low) { return key | (low << 19); }
  __device__ static uint32_t key(uint32_t e) { return e & ((1u << 19) - 1u); }
  __device__ static uint32_t low(uint32_t e) { return e >> 19; }
};

template <>
struct ElementCodec<uint64_t> {
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

constexpr int kScatterSpan = kTile / kGroupWaves;  // elements of a tile per wave
constexpr int kScatterRounds = kScatterSpan / 64;

// Stable scatter of one tile by digit: each element goes to
//   bucket_start[b] + (elements of b in earlier tiles) + (its rank within b in this tile).
// Wave w takes the tile's elements [w S, (w + 1) S) (S = kScatterSpan), 64
// consecutive ones a round, and ranks them with the wave-level multisplit.
// The per-wave digit counts, scanned over the waves and then over the
// digits, give every element its place in the tile sorted stably by digit;
// it takes that place in LDS, and the sorted tile leaves in order, each
// bucket's run as one contiguous write.  Out-of-range keys take no place.
// Every block scans the bucket totals for itself; block 0 also publishes the
// bucket starts (and the count of in-range elements) for the next launch.
template <typename E, bool kPairs, typename Out>
__global__ __launch_bounds__(kThreads, 4) void tile_scatter_kernel(
    const int64_t* __restrict__ keys64, const uint32_t* __restrict__ keys32, const uint32_t* __restrict__ index32,
    int64_t n, const uint32_t* count_limit, uint64_t n_nodes, int shift, int bits, int buckets, int64_t tiles,
    const uint32_t* __restrict__ counts, const uint32_t* __restrict__ bucket_total,
    uint32_t* __restrict__ bucket_start, uint32_t* __restrict__ valid_count, int64_t* __restrict__ offsets_last,
    Out out, const int32_t* __restrict__ status, int gate) {
  using Codec = ElementCodec<E>;
  static_assert(kGroupWaves * kMaxBuckets * 4 <= kTile * sizeof(E), "the wave counters fit the tile's space");
  // the wave counters, then (once every place is known) the sorted tile
  __shared__ E sorted[kTile];
  uint32_t* wave_count = reinterpret_cast<uint32_t*>(sorted);
  __shared__ uint32_t tile_start[kMaxBuckets];
  __shared__ uint32_t shift_to_target[kMaxBuckets];
  __shared__ uint32_t wave_totals[kGroupWaves];
  if (gate_closed(status, gate)) return;
  const int64_t limit = element_limit(n, count_limit);
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const uint32_t digit_mask = (1u << bits) - 1u;
  const unsigned int tile_index = xcd_block(blockIdx.x, gridDim.x);  // as in the count pass
  const int64_t tile_base = static_cast<int64_t>(tile_index) * kTile;
  const int n_tile = tile_elements(tile_base, limit);
  for (int i = t; i < kGroupWaves * kMaxBuckets; i += kThreads) wave_count[i] = 0u;
  const int first = wave * kScatterSpan + lane;  // the lane's element of round 0
  // the tile's column of counts and the bucket totals, loaded early (used after the ranking)
  constexpr int kPerThread = kMaxBuckets / kThreads;
  uint32_t earlier[kPerThread], total[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int b = t + j * kThreads;
    earlier[j] = b < buckets ? counts[static_cast<int64_t>(b) * tiles + tile_index] : 0u;
    total[j] = b < buckets ? bucket_total[b] : 0u;
  }

  uint32_t key[kScatterRounds];
  uint32_t low[kPairs ? kScatterRounds : 1];
  uint32_t ok = 0u;  // bit r: the round-r element exists and is in range
  if constexpr (kPairs) {
    const BufferView key_view = buffer_view(keys32 + (n_tile > 0 ? tile_base : 0), static_cast<int64_t>(n_tile) * 4);
    const BufferView index_view = buffer_view(index32 + (n_tile > 0 ? tile_base : 0), static_cast<int64_t>(n_tile) * 4);
#pragma unroll
    for (int r = 0; r < kScatterRounds; ++r) {
      const int q = first + 64 * r;
      key[r] = load_u32(key_view, static_cast<uint32_t>(q) * 4u);
      low[r] = load_u32(index_view, static_cast<uint32_t>(q) * 4u);
      ok |= q < n_tile ? (1u << r) : 0u;
    }
  } else {
    const BufferView view = buffer_view(keys64 + (n_tile > 0 ? tile_base : 0), static_cast<int64_t>(n_tile) * 8);
#pragma unroll
    for (int r = 0; r < kScatterRounds; ++r) {
      const int q = first + 64 * r;
      const int64_t raw = load_i64(view, static_cast<uint32_t>(q) * 8u);
      key[r] = static_cast<uint32_t>(raw);
      ok |= q < n_tile && static_cast<uint64_t>(raw) < n_nodes ? (1u << r) : 0u;
    }
  }
  __syncthreads();  // the wave counters are zero

  const auto digit = [&](int r) { return (key[r] >> shift) & digit_mask; };
  uint32_t rank[kScatterRounds];
  uint32_t* counter = wave_count + wave * kMaxBuckets;
  wave_split_ranks<kDigitBits, kScatterRounds, sizeof(E) == 4>(digit, ok, counter, rank);
  __syncthreads();
  wave_prefix(wave_count, kMaxBuckets, buckets, tile_start);

  // bucket starts: every block scans the bucket totals (block 0 publishes them)
#pragma unroll
  for (int j = 0; j < kPerThread; ++j)
    if (t + j * kThreads < buckets) shift_to_target[t + j * kThreads] = total[j];
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
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int b = t + j * kThreads;
    if (b < buckets) shift_to_target[b] += earlier[j] - tile_start[b];
  }
  // places in the sorted tile, then (the counters read) the elements move there
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r)
    rank[r] += ((ok >> r) & 1u) ? tile_start[digit(r)] + counter[digit(r)] : 0u;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r) {
    if ((ok >> r) & 1u) {
      if constexpr (kPairs)
        sorted[rank[r]] = Codec::make(key[r], low[r]);
      else
        sorted[rank[r]] = Codec::make(key[r], static_cast<uint32_t>(first + 64 * r));
    }
  }
  __syncthreads();
  // each bucket's run: sorted position p goes to shift_to_target[b] + p
  for (int p = t; p < static_cast<int>(in_tile); p += kThreads) {
    const E e = sorted[p];
    const uint32_t k = Codec::key(e);
    const uint32_t target = shift_to_target[(k >> shift) & digit_mask] + static_cast<uint32_t>(p);
    const uint32_t index = kPairs ? Codec::low(e) : static_cast<uint32_t>(tile_base) + Codec::low(e);
    // unreachable past the element count: the count pass saw the same elements
    if (static_cast<int64_t>(target) < limit) out.store(target, k, index);
  }
}

// offsets[k] = first position e with key[e] >= k, for k in [0, N], of the
// non-decreasing keys[0, limit): position e writes offsets[k] = e for every k
// in (key[e-1], key[e]] (key[-1] = -1, key[limit] = N), so each entry is
// written once.  Gaps of up to kShortGap entries are filled by their thread;
// longer ones (sparse keys) are listed in LDS and filled by the whole
// workgroup.  With `identity`, also identity[e] = e.  Workgroups `block` of
// `blocks` stride over the list.
template <int kT>
struct GapListOf {
  int64_t low[kT];
  int64_t high[kT];
  int64_t edge[kT];
  int count;
};
using GapList = GapListOf<kThreads>;

template <typename K, int kT = kThreads>
__device__ __forceinline__ void boundary_offsets(const K* __restrict__ keys, int64_t limit, int64_t n_nodes,
                                                 int64_t* __restrict__ offsets, int64_t* __restrict__ identity,
                                                 int64_t block, int64_t blocks, GapListOf<kT>& gaps) {
  const int64_t stride = blocks * kT;
  for (int64_t first = block * kT; first <= limit; first += stride) {
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
      for (int64_t k = gaps.low[g] + threadIdx.x; k <= gaps.high[g]; k += kT) offsets[k] = gaps.edge[g];
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
// of 2^fine_bits keys.  The fine-digit histogram gives the offsets of the
// bucket's keys, and each chunk of the bucket, ranked by the fine digit with
// the wave-level multisplit (wave w takes the chunk's elements
// [w S, (w + 1) S), S = kLocalChunk / 4) and sorted stably in LDS, places its
// edge indices in `order`.  A bucket of one chunk takes its histogram from the
// ranking's counts; a longer one counts first in a pass of its own.  Sorted
// keys: every workgroup strides over the keys themselves for the offsets and
// the identity order.
template <typename P, int kFineMatch>
__global__ __launch_bounds__(kThreads, sizeof(P) == 4 ? 4 : 2) void finish_kernel(const P* __restrict__ packed,
                                                          const uint32_t* __restrict__ bucket_start, int buckets,
                                                          int fine_bits, const int64_t* __restrict__ keys,
                                                          int64_t n_edges, int64_t n_nodes,
                                                          int64_t* __restrict__ order,
                                                          int64_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ status) {
  constexpr int kSpan = kLocalChunk / kGroupWaves;
  constexpr int kRounds = kSpan / 64;
  static_assert(kGroupWaves * kMaxFine * 4 <= kLocalChunk * sizeof(P), "the wave counters fit the chunk's space");
  // the wave counters, then (once every place is known) the sorted chunk
  __shared__ P sorted[kLocalChunk];
  uint32_t* wave_count = reinterpret_cast<uint32_t*>(sorted);
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
  const int lane = t & 63;
  const int wave = t >> 6;
  const int64_t start = bucket_start[b];
  const int64_t end = bucket_start[b + 1];
  const int64_t count = end - start;
  const int fines = 1 << fine_bits;
  const P fine_mask = static_cast<P>(fines - 1);
  const bool one_chunk = count <= kLocalChunk;
  for (int i = t; i < kGroupWaves * kMaxFine; i += kThreads) wave_count[i] = 0u;
  for (int f = t; f < fines; f += kThreads) fine_base[f] = 0u;
  __syncthreads();

  const auto load_chunk = [&](int64_t first, int in_chunk, P (&values)[kRounds]) {
    // a view per chunk keeps every offset small, however long the bucket
    const BufferView view = buffer_view(packed + start + first, static_cast<int64_t>(in_chunk) * sizeof(P));
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const uint32_t offset = static_cast<uint32_t>(wave * kSpan + 64 * r + lane) * sizeof(P);
      if constexpr (sizeof(P) == 8)
        values[r] = static_cast<P>(load_i64(view, offset));
      else
        values[r] = load_u32(view, offset);
    }
  };
  const auto write_offsets = [&]() {
    for (int f = t; f < fines; f += kThreads) {
      const int64_t key = (static_cast<int64_t>(b) << fine_bits) + f;
      if (key < n_nodes) offsets[key] = fine_base[f];
    }
  };

  if (!one_chunk) {
    // the bucket's fine-digit histogram -> offsets of its keys
    for (int64_t first = 0; first < count; first += kLocalChunk) {
      const int in_chunk = static_cast<int>(count - first < kLocalChunk ? count - first : kLocalChunk);
      P values[kRounds];
      load_chunk(first, in_chunk, values);
#pragma unroll
      for (int r = 0; r < kRounds; ++r)
        if (wave * kSpan + 64 * r + lane < in_chunk)
          atomicAdd(&fine_base[static_cast<uint32_t>(values[r] & fine_mask)], 1u);
    }
    __syncthreads();
    lds_exclusive_scan(fine_base, fines, static_cast<uint32_t>(start), wave_totals);
    write_offsets();
    if (order == nullptr) return;
  }

  // an empty bucket takes one (empty) round too: it still writes its keys' offsets
  for (int64_t first = 0; first < count || first == 0; first += kLocalChunk) {
    const int in_chunk = static_cast<int>(count - first < kLocalChunk ? count - first : kLocalChunk);
    P values[kRounds];
    uint32_t rank[kRounds];
    load_chunk(first, in_chunk, values);
    const auto fine = [&](int r) { return static_cast<uint32_t>(values[r] & fine_mask); };
    uint32_t valid = 0u;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) valid |= wave * kSpan + 64 * r + lane < in_chunk ? (1u << r) : 0u;
    uint32_t* counter = wave_count + wave * kMaxFine;
    wave_split_ranks<kFineMatch, kRounds, false>(fine, valid, counter, rank);
    __syncthreads();
    wave_prefix(wave_count, kMaxFine, fines, chunk_start);
    __syncthreads();
    lds_exclusive_scan(chunk_start, fines, 0u, wave_totals);
    if (one_chunk) {
      // the chunk is the bucket: its digit counts are the histogram
      for (int f = t; f < fines; f += kThreads) fine_base[f] = static_cast<uint32_t>(start) + chunk_start[f];
      __syncthreads();
      write_offsets();
      if (order == nullptr) return;
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) rank[r] += ((valid >> r) & 1u) ? chunk_start[fine(r)] + counter[fine(r)] : 0u;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRounds; ++r)
      if ((valid >> r) & 1u) sorted[rank[r]] = values[r];
    __syncthreads();
    for (int p = t; p < in_chunk; p += kThreads) {
      const P e = sorted[p];
      const uint32_t f = static_cast<uint32_t>(e & fine_mask);
      const int64_t target = static_cast<int64_t>(fine_base[f]) + (p - static_cast<int64_t>(chunk_start[f]));
      // unreachable outside the bucket: its fine digits were counted from the same elements
      if (target >= start && target < end) order[target] = static_cast<int64_t>(e >> fine_bits);
    }
    __syncthreads();
    // the next chunk's elements of digit f follow this chunk's; the wave counters restart
    for (int f = t; f < fines; f += kThreads) {
      const uint32_t next = f + 1 < fines ? chunk_start[f + 1] : static_cast<uint32_t>(in_chunk);
      fine_base[f] += next - chunk_start[f];
    }
    for (int i = t; i < kGroupWaves * kMaxFine; i += kThreads) wave_count[i] = 0u;
    __syncthreads();
  }
}

// Last launch of the two-level path for fine digits of at most 6 bits and
// 32-bit packed elements (index << fine_bits | fine digit): the same outputs
// as finish_kernel, ranked without ballots.  Thread t takes a contiguous run
// of kPrivateItems elements of the chunk and counts its digits in its own
// row of LDS counters (no other thread touches the row).  Lane d of each
// wave then turns column d of its wave's 64 rows into exclusive prefixes,
// the waves' digit totals are scanned over the waves and the digits, and
// every thread walks its run again in order, placing each element at the
// next position of its digit: a stable rank (run order within a thread,
// thread order within a wave, wave order within the chunk); the chunk is
// then sorted in LDS and written out in order.  Longer buckets take a
// histogram pass first, then chunk after chunk as above.
constexpr int kPrivateItems = kLocalChunk / kThreads;  // 16 elements per thread and chunk
constexpr int kPrivateDigits = 64;
constexpr int kPrivateRow = kPrivateDigits + 2;         // padded row: lanes of one digit fall in 32 banks
static_assert(sizeof(uint16_t) * kThreads * kPrivateRow >= kLocalChunk * sizeof(uint32_t),
              "a sorted chunk fits over the counters");

__global__ __launch_bounds__(kThreads, 2) void finish_private_kernel(
    const uint32_t* __restrict__ packed, const uint32_t* __restrict__ bucket_start, int buckets, int fine_bits,
    const int64_t* __restrict__ keys, int64_t n_edges, int64_t n_nodes, int64_t* __restrict__ order,
    int64_t* __restrict__ offsets, const int32_t* __restrict__ status) {
  constexpr size_t kRankBytes = sizeof(uint16_t) * kThreads * kPrivateRow;
  constexpr size_t kShared = kRankBytes > sizeof(GapList) ? kRankBytes : sizeof(GapList);
  __shared__ __align__(16) unsigned char shared[kShared];
  __shared__ uint32_t wave_digit[kGroupWaves][kPrivateDigits];
  __shared__ uint32_t fine_base[kPrivateDigits];
  __shared__ uint32_t chunk_base[kPrivateDigits];
  __shared__ uint32_t wave_totals[kGroupWaves];
  if (!(status_of(status) & kFlagUnsorted)) {
    boundary_offsets(keys, n_edges, n_nodes, offsets, order, blockIdx.x, gridDim.x,
                     *reinterpret_cast<GapList*>(shared));
    return;
  }
  const int b = blockIdx.x;
  if (b >= buckets) return;
  uint16_t* rank = reinterpret_cast<uint16_t*>(shared);
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int64_t start = bucket_start[b];
  const int64_t end = bucket_start[b + 1];
  const int64_t count = end - start;
  const int fines = 1 << fine_bits;
  const uint32_t fine_mask = static_cast<uint32_t>(fines - 1);
  uint16_t* mine = rank + t * kPrivateRow;

  const auto write_offsets = [&]() {
    for (int f = t; f < fines; f += kThreads) {
      const int64_t key = (static_cast<int64_t>(b) << fine_bits) + f;
      if (key < n_nodes) offsets[key] = fine_base[f];
    }
  };
  if (count > kLocalChunk) {
    // the bucket's fine-digit histogram -> offsets of its keys
    for (int f = t; f < kPrivateDigits; f += kThreads) fine_base[f] = 0u;
    __syncthreads();
    for (int64_t i = t; i < count; i += kThreads) atomicAdd(&fine_base[packed[start + i] & fine_mask], 1u);
    __syncthreads();
    lds_exclusive_scan(fine_base, fines, static_cast<uint32_t>(start), wave_totals);
    write_offsets();
    if (order == nullptr) return;
  }

  // an empty bucket takes one (empty) round too: it still writes its keys' offsets
  for (int64_t first = 0; first < count || first == 0; first += kLocalChunk) {
    const int in_chunk = static_cast<int>(count - first < kLocalChunk ? count - first : kLocalChunk);
    // this thread's run: elements [t * kPrivateItems, (t + 1) * kPrivateItems) of the chunk
    const BufferView view = buffer_view(packed + start + first, static_cast<int64_t>(in_chunk) * 4);
    uint32_t value[kPrivateItems];
#pragma unroll
    for (int q = 0; q < kPrivateItems / 4; ++q) {  // 16-byte loads (zeros past the chunk, dword by dword)
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 four = __builtin_amdgcn_raw_buffer_load_b128(
          view, static_cast<int>((t * kPrivateItems + 4 * q) * 4), 0, 0);
      value[4 * q] = four.x;
      value[4 * q + 1] = four.y;
      value[4 * q + 2] = four.z;
      value[4 * q + 3] = four.w;
    }
    const int here = in_chunk - t * kPrivateItems;  // elements of the run inside the chunk (may be <= 0)
#pragma unroll
    for (int d = 0; d < kPrivateDigits; ++d) mine[d] = 0;
#pragma unroll
    for (int i = 0; i < kPrivateItems; ++i)
      if (i < here) ++mine[value[i] & fine_mask];
    __syncthreads();
    // column `lane` of this wave's rows -> exclusive prefixes over the wave's lanes
    if (lane < fines) {
      uint32_t running = 0;
      uint16_t* column = rank + (wave * 64) * kPrivateRow + lane;
      for (int l0 = 0; l0 < 64; l0 += 16) {  // sixteen rows' reads in flight
        uint32_t c[16];
#pragma unroll
        for (int l = 0; l < 16; ++l) c[l] = column[(l0 + l) * kPrivateRow];
#pragma unroll
        for (int l = 0; l < 16; ++l) {
          column[(l0 + l) * kPrivateRow] = static_cast<uint16_t>(running);
          running += c[l];
        }
      }
      wave_digit[wave][lane] = running;
    }
    __syncthreads();
    // digit totals of the chunk -> chunk_base (exclusive over digits); each wave's
    // base per digit = chunk_base + the digit's elements in earlier waves
    if (t < kPrivateDigits) {
      uint32_t total = 0;
      for (int w = 0; w < kGroupWaves; ++w) total += t < fines ? wave_digit[w][t] : 0u;
      chunk_base[t] = total;
    }
    __syncthreads();
    lds_exclusive_scan(chunk_base, kPrivateDigits, 0u, wave_totals);
    if (t < fines) {
      uint32_t running = chunk_base[t];
      for (int w = 0; w < kGroupWaves; ++w) {
        const uint32_t c = wave_digit[w][t];
        wave_digit[w][t] = running;
        running += c;
      }
    }
    if (count <= kLocalChunk) {
      // the chunk is the bucket: its digit starts are the offsets of its keys
      for (int f = t; f < fines; f += kThreads) fine_base[f] = static_cast<uint32_t>(start) + chunk_base[f];
      __syncthreads();
      write_offsets();
      if (order == nullptr) return;
    }
    __syncthreads();
    uint32_t place[kPrivateItems];
#pragma unroll
    for (int i = 0; i < kPrivateItems; ++i) {
      const uint32_t d = value[i] & fine_mask;
      place[i] = wave_digit[wave][d] + mine[d];
      if (i < here) mine[d] = static_cast<uint16_t>(mine[d] + 1);
    }
    __syncthreads();
    // the chunk sorted by digit in LDS (over the counters), then written out in order
    uint32_t* sorted = reinterpret_cast<uint32_t*>(shared);
#pragma unroll
    for (int i = 0; i < kPrivateItems; ++i)
      if (i < here) sorted[place[i]] = value[i];
    __syncthreads();
    for (int p = t; p < in_chunk; p += kThreads) {
      const uint32_t e = sorted[p];
      const uint32_t d = e & fine_mask;
      const int64_t target = static_cast<int64_t>(fine_base[d]) + (p - static_cast<int64_t>(chunk_base[d]));
      // unreachable outside the bucket: its digits were counted from the same elements
      if (target >= start && target < end) order[target] = static_cast<int64_t>(e >> fine_bits);
    }
    __syncthreads();
    // the next chunk's elements of digit d follow this chunk's
    for (int f = t; f < fines; f += kThreads) {
      const uint32_t next = f + 1 < fines ? chunk_base[f + 1] : static_cast<uint32_t>(in_chunk);
      fine_base[f] += next - chunk_base[f];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// grouped two-level path: tile-local grouping, then bucket gathers
// ---------------------------------------------------------------------------
//
// For packed 32-bit elements, fine digits of at most kGroupedFineBits (7) bits
// and at most kMaxRunTiles (2048) tiles the two-level sort takes two launches
// instead of four:
//
//   group   one workgroup per tile: the range and sortedness checks, then the
//           tile's in-range elements grouped stably by the coarse digit and
//           written back over the tile's own span of the packed buffer (one
//           contiguous write), with the tile's row of the buckets' runs (the
//           run's first and end position in the tile, 16 bits each, in one
//           word, so that a gather reads one word per tile) and its flags.
//           No count pass and no scan over the tiles: nothing in a tile's
//           output depends on another tile.
//   gather  one workgroup per bucket: its run in every tile (two row
//           entries), scanned over the tiles, places the runs one after the
//           other; the bucket's elements, gathered chunk by chunk in tile
//           order (consecutive lanes read consecutive elements of a run), are
//           ranked by the fine digit and their edge indices placed in `order`.
//           Every workgroup ORs the tiles' flags, so the sorted case takes the
//           boundary path without a host round trip, and workgroup 0 writes
//           the status word.
//
// The group ranks with wave_match_ranks (the lanes of equal coarse digits
// found through LDS words instead of one ballot per digit bit), the gather
// with wave_ballot_ranks (one ballot per fine digit bit).  The gather is
// instantiated for 64 or 128 fine digits and 1024 or 2048 tiles; the wider
// instances hold more per thread and spill a few registers, still well ahead
// of the four launches (a config-4R source list, N = 131,072 and 11.9M
// edges: 116 against 155 us).

constexpr int kMaxRunTiles = 2048;                    // tiles a gather holds (edges up to 2^24)
constexpr int kFineMatchBits = 6;                     // digits that name their own LDS mask word
constexpr int kGroupedFineBits = 7;                   // fine digits a gather ranks (at most)
// A gather's workgroup and the elements it ranks at once: 6144 at eight waves
// per SIMD (four gathers per CU, so 1024 buckets run in one round) when the
// buckets average at most 95% of that, else 8192 at six (three per CU).  A
// bucket longer than its chunk takes the multi-chunk path: slower, not wrong.
constexpr int kGatherThreads = 512;
constexpr int kGatherSmallChunk = 6144;
constexpr int kGatherLargeChunk = 8192;

// The same ranks as wave_split_ranks, with the lanes of equal digits found
// through LDS instead of one ballot per digit bit.  Every lane first clears
// the mask word its lane id names; each active lane then ORs its bit into the
// word of its group and reads the word back: the lanes of its group.  Digits
// of at most 6 bits name the word themselves.  A wider digit first names a
// leader: every active lane writes its lane id into the byte of its digit
// (one of the writes remains) and reads the byte back, so the lanes of one
// digit, and only they, read the same lane id.  A wave's LDS operations take
// effect in program order; the signal fences (compiler barriers, no
// instruction) keep the compiler from reordering them or forwarding the
// written byte to the read.  `leader` is the wave's [1 << kBits] bytes (unused
// for kBits <= 6), `masks` its 65 words, `counter` its [digit] array, advanced
// as in wave_split_ranks; the ranks of inactive lanes are unspecified.  Only
// rounds [0, rounds) are ranked.  Every lane of the wave must call it.
template <int kBits, int kRounds, typename DigitOf>
__device__ __forceinline__ void wave_match_ranks(DigitOf digit, uint32_t valid, uint32_t* counter,
                                                 uint8_t* leader, uint64_t* masks, uint32_t (&rank)[kRounds],
                                                 int rounds = kRounds) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (r >= rounds) continue;  // wave-uniform: the rounds the wave's span holds
    const bool active = ((valid >> r) & 1u) != 0u;
    const uint32_t d = digit(r);
    // read first: it follows the previous round's addition in LDS order
    const uint32_t before = counter[d];
    masks[lane] = 0ull;
    uint32_t group = d;
    if constexpr (kBits > kFineMatchBits) {
      // inactive lanes write too: a byte one of them keeps names only that lane's digit
      leader[d] = static_cast<uint8_t>(lane);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      group = leader[d];
    }
    group = active ? group : 64u;  // inactive lanes OR into word 64, which no active lane reads
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    atomicOr(reinterpret_cast<unsigned long long*>(masks + group), static_cast<unsigned long long>(1ull << lane));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint64_t same = masks[group];
    const uint32_t below = lanes_below(same);
    rank[r] = before + below;
    asm volatile("" : "+v"(rank[r]));  // summed before the addition is issued, which then needs no wait
    // digits are masked, so every lane's read above was in range
    if (active && below == 0u) atomicAdd(&counter[d], static_cast<uint32_t>(__popcll(same)));
  }
}

// The same ranks as wave_split_ranks with one ballot per digit bit, arranged
// so that no LDS round trip stalls a round: every lane reads its digit's
// counter first, the ballots run while the read is in flight, and the
// group's leader then adds the group's size to the counter without waiting
// for the old value (a wave's LDS operations take effect in program order, so
// the next round's reads see the addition).  Only rounds [0, rounds) are
// ranked; ranks of inactive lanes are unspecified.  Every lane of the wave
// must call it.
template <int kBits, int kRounds, typename DigitOf>
__device__ __forceinline__ void wave_ballot_ranks(DigitOf digit, uint32_t valid, uint32_t* counter,
                                                  uint32_t (&rank)[kRounds], int rounds = kRounds) {
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (r >= rounds) continue;  // wave-uniform: the rounds the wave's span holds
    const bool active = ((valid >> r) & 1u) != 0u;
    const uint32_t d = digit(r);
    const uint32_t before = counter[d];
    // (an inactive lane's mask is garbage; only active lanes use theirs)
    const uint64_t same = lanes_with_digit_unmasked<kBits>(d, __ballot(active));
    const uint32_t below = lanes_below(same);
    rank[r] = before + below;
    asm volatile("" : "+v"(rank[r]));  // summed before the addition is issued, which then needs no wait
    if (active && below == 0u) atomicAdd(&counter[d], static_cast<uint32_t>(__popcll(same)));
  }
}

// Lane l receives lane l + 1's value and lane 63 lane 0's (DPP wave_rol:1).
__device__ __forceinline__ uint32_t rotate_from_lane_above(uint32_t value) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(value), 0x134, 0xf, 0xf, false));
}

// Exclusive running maximum over a workgroup of kT threads of one value per
// thread (0 for thread 0).  Every thread must call it.
template <int kT = kThreads>
__device__ __forceinline__ uint32_t block_exclusive_max(uint32_t value, uint32_t* wave_totals) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t inclusive = value;
  inclusive = max(inclusive, dpp_or_zero<0x111, 0xf>(inclusive));
  inclusive = max(inclusive, dpp_or_zero<0x112, 0xf>(inclusive));
  inclusive = max(inclusive, dpp_or_zero<0x114, 0xf>(inclusive));
  inclusive = max(inclusive, dpp_or_zero<0x118, 0xf>(inclusive));
  inclusive = max(inclusive, dpp_or_zero<0x142, 0xa>(inclusive));
  inclusive = max(inclusive, dpp_or_zero<0x143, 0xc>(inclusive));
  if (lane == 63) wave_totals[wave] = inclusive;
  __syncthreads();
  uint32_t before = 0u;
#pragma unroll
  for (int w = 0; w < kT / 64; ++w) before = w < wave ? max(before, wave_totals[w]) : before;
  __syncthreads();
  return max(before, from_lane_below(inclusive, 0u));
}

// The wave's OR of the range and sortedness flags into wave_flags[wave]
// (lane 0 writes); after a barrier, wave_or_read gives the workgroup's.
__device__ __forceinline__ void wave_or_flags(int32_t flags, int32_t* wave_flags) {
  const int32_t wave_flags_or = (__ballot(flags & kFlagOutOfRange) ? kFlagOutOfRange : 0) |
                                (__ballot(flags & kFlagUnsorted) ? kFlagUnsorted : 0);
  if ((threadIdx.x & 63) == 0) wave_flags[threadIdx.x >> 6] = wave_flags_or;
}
template <int kT>
__device__ __forceinline__ int32_t wave_or_read(const int32_t* wave_flags) {
  int32_t all = 0;
#pragma unroll
  for (int w = 0; w < kT / 64; ++w) all |= wave_flags[w];
  return all;
}

// One tile: checks, stable grouping by the coarse digit (key >> fine_bits),
// the grouped packed elements over packed[tile_base, tile_base + in-range
// count), the row rows[tile][0, buckets) of the buckets' runs in the tile
// (first | end << 16), and tile_flags[tile].  Wave w takes the tile's elements
// [w S, (w + 1) S) (S = kScatterSpan), 64 consecutive ones a round.
__global__ __launch_bounds__(kThreads, 6) void tile_group_kernel(const int64_t* __restrict__ keys, int64_t n,
                                                                 uint64_t n_nodes, int fine_bits, int buckets,
                                                                 uint32_t* __restrict__ packed,
                                                                 uint32_t* __restrict__ rows, int64_t row_stride,
                                                                 uint32_t* __restrict__ tile_flags) {
  // the wave counters, then (once every place is known) the grouped tile
  __shared__ __align__(16) uint32_t sorted[kTile];
  uint32_t* wave_count = sorted;
  // the match tables while the waves rank
  struct MatchTables {
    uint8_t leader[kGroupWaves][kMaxBuckets];
    uint64_t masks[kGroupWaves][64 + 1];
  };
  __shared__ struct {
    MatchTables match;
  } tables;
  __shared__ uint32_t wave_totals[kGroupWaves];
  __shared__ int32_t wave_flags[kGroupWaves];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  // tiles in launch order, dealt round-robin over the XCDs: the key stream ran 1 us faster at config 4
  // than with each XCD taking a contiguous range of tiles
  const unsigned int tile = blockIdx.x;
  const int64_t tile_base = static_cast<int64_t>(tile) * kTile;
  const int64_t rest = n - tile_base;
  const int n_tile = static_cast<int>(rest > kTile ? kTile : rest);
  const int extent = static_cast<int>(rest > kTile + 1 ? kTile + 1 : rest);  // one element past the tile
  const uint32_t digit_mask = static_cast<uint32_t>(kMaxBuckets - 1);
  const uint32_t fine_mask = (1u << fine_bits) - 1u;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int i = t; i < kGroupWaves * kMaxBuckets / 4; i += kThreads) reinterpret_cast<u32x4*>(wave_count)[i] = zero;

  const BufferView view = buffer_view(keys + tile_base, static_cast<int64_t>(extent) * 8);
  const int first = wave * kScatterSpan + lane;  // the lane's element of round 0
  int64_t raw[kScatterRounds];
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r) raw[r] = load_i64_streamed(view, static_cast<uint32_t>(first + 64 * r) * 8u);
  // the element after the wave's span: the next wave's first, or the one after the tile
  const int after_q = (wave + 1) * kScatterSpan;
  const int64_t after = load_i64(view, static_cast<uint32_t>(after_q) * 8u);
  uint32_t key[kScatterRounds];
  uint32_t ok = 0u;  // bit r: the round-r element exists and is in range
  int32_t flags = 0;
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r) {
    const bool valid = first + 64 * r < n_tile;
    const bool in = valid && static_cast<uint64_t>(raw[r]) < n_nodes;
    key[r] = static_cast<uint32_t>(raw[r]);
    ok |= in ? (1u << r) : 0u;
    if (valid && !in) flags |= kFlagOutOfRange;
  }
  // element q against q + 1 (both in range): the next lane of the round, lane
  // 0 of the next round for lane 63, and `after` past the wave's last round.
  // A wave rotation (lane l reads lane l + 1, lane 63 reads lane 0) of round
  // r + 1 holds lane 63's successor.
  const uint32_t after_ok = after_q < extent && static_cast<uint64_t>(after) < n_nodes ? 1u : 0u;
  const uint32_t ok_above = rotate_from_lane_above(ok);
  uint32_t key_above = rotate_from_lane_above(key[0]);
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r) {
    uint32_t next = key_above;
    uint32_t next_ok = (ok_above >> r) & 1u;
    if (r + 1 < kScatterRounds) {
      key_above = rotate_from_lane_above(key[r + 1 < kScatterRounds ? r + 1 : r]);
      if (lane == 63) {
        next = key_above;
        next_ok = (ok_above >> (r + 1)) & 1u;
      }
    } else if (lane == 63) {
      next = static_cast<uint32_t>(after);
      next_ok = after_ok;
    }
    if (((ok >> r) & 1u) && next_ok && next < key[r]) flags |= kFlagUnsorted;
  }
  asm volatile("" : "+v"(flags));  // the checks finish here, before the ranking
  __syncthreads();  // the wave counters are zero

  // (empty asm: the compiler rebuilds per-round conditions and digits from these
  // registers where they are used instead of holding them across the phases)
  asm volatile("" : "+v"(ok));
  const auto digit = [&](int r) { return (key[r] >> fine_bits) & digit_mask; };
  uint32_t rank[kScatterRounds];
  uint32_t* counter = wave_count + wave * kMaxBuckets;
  wave_match_ranks<kDigitBits, kScatterRounds>(digit, ok, counter, tables.match.leader[wave],
                                               tables.match.masks[wave], rank);
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r) asm volatile("" : "+v"(key[r]));
  asm volatile("" : "+v"(ok));
  __syncthreads();
  // Thread t takes digits 2t and 2t + 1 (digits past `buckets` count nothing):
  // their counts in every wave, scanned over the digits and then the waves,
  // become in place the place of each wave's first element of the digit in
  // the grouped tile, and the digits' runs go to the tile's row.
  static_assert(kMaxBuckets == 2 * kThreads, "two digits a thread");
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  u32x2v* pairs = reinterpret_cast<u32x2v*>(wave_count);
  u32x2v counts[kGroupWaves];
  uint32_t total0 = 0u, total1 = 0u;
#pragma unroll
  for (int w = 0; w < kGroupWaves; ++w) {
    counts[w] = pairs[w * (kMaxBuckets / 2) + t];
    total0 += counts[w].x;
    total1 += counts[w].y;
  }
  uint32_t in_tile = 0u;
  const uint32_t start0 = block_exclusive_scan(total0 + total1, wave_totals, in_tile);
  const uint32_t start1 = start0 + total0;
  uint32_t run0 = start0, run1 = start1;
#pragma unroll
  for (int w = 0; w < kGroupWaves; ++w) {
    const u32x2v place = {run0, run1};
    pairs[w * (kMaxBuckets / 2) + t] = place;
    run0 += counts[w].x;
    run1 += counts[w].y;
  }
  uint32_t* row = rows + static_cast<int64_t>(tile) * row_stride;
  if (2 * t < buckets) row[2 * t] = start0 | (start1 << 16);
  if (2 * t + 1 < buckets) row[2 * t + 1] = start1 | ((start1 + total1) << 16);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r) rank[r] += ((ok >> r) & 1u) ? counter[digit(r)] : 0u;
  wave_or_flags(flags, wave_flags);
  __syncthreads();  // every counter is read before the grouped tile overwrites them
#pragma unroll
  for (int r = 0; r < kScatterRounds; ++r)
    if ((ok >> r) & 1u)
      sorted[rank[r]] = (static_cast<uint32_t>(tile_base + first + 64 * r) << fine_bits) | (key[r] & fine_mask);
  if (t == 0) tile_flags[tile] = static_cast<uint32_t>(wave_or_read<kThreads>(wave_flags));
  __syncthreads();
  // the grouped tile, four elements a thread and store while they lie inside the tile
  // (cached stores: the gathers read them next, from the Infinity Cache)
  uint32_t* out = packed + tile_base;
  for (int p = 4 * t; p < static_cast<int>(in_tile); p += 4 * kThreads) {
    if (p + 4 <= n_tile) {
      *reinterpret_cast<u32x4*>(out + p) = *reinterpret_cast<const u32x4*>(sorted + p);
    } else {
      for (int i = p; i < static_cast<int>(in_tile); ++i) out[i] = sorted[i];
    }
  }
}

// One bucket: see the section comment.  A run's elements sit at packed[delta
// + position in the bucket], with delta = (tile * kTile + the run's start in
// the tile) - (the run's first position in the bucket); delta never decreases
// from one tile to the next (a run ends inside its tile), so a running maximum
// over the run starts, each marked with delta + 1, gives every position of the
// chunk its source.  Buckets of more than one chunk count their fine digits in
// a gather pass of their own first.
template <int kGT, int kChunk, int kMinWaves, int kFB, int kTiles>
__global__ __launch_bounds__(kGT, kMinWaves) void bucket_gather_kernel(
    const uint32_t* __restrict__ packed, const uint32_t* __restrict__ rows, int64_t row_stride,
    const uint32_t* __restrict__ tile_flags, int tiles, int buckets, int fine_bits,
    const int64_t* __restrict__ keys, int64_t n_edges, int64_t n_nodes, int64_t* __restrict__ order,
    int64_t* __restrict__ offsets, int32_t* __restrict__ status, int or_status) {
  constexpr int kGW = kGT / 64;                            // waves of the workgroup
  constexpr int kRounds = kChunk / kGW / 64;          // rounds of the longest span
  constexpr int kMarks = kChunk / kGT;                // positions a thread scans
  constexpr int kRunsPerThread = kTiles / kGT;
  constexpr int kFineDigits = 1 << kFB;               // fine digits of the instance (64 or 128)
  static_assert(kFineDigits % 64 == 0 && kTiles <= kMaxRunTiles, "whole waves of digits; tiles held");
  using Gaps = GapListOf<kGT>;
  constexpr size_t kRegion = kChunk * sizeof(uint32_t) > sizeof(Gaps) ? kChunk * sizeof(uint32_t)
                                                                              : sizeof(Gaps);
  // the chunk's marks while it is gathered, then the sorted chunk; the gap list on the sorted path
  __shared__ __align__(16) unsigned char region[kRegion];
  // per wave and fine digit: the counters while the wave ranks, then the
  // digit's first place in the chunk for the wave's elements
  __shared__ uint32_t wave_base[kGW * kFineDigits];
  __shared__ uint32_t fine_base[kFineDigits];
  __shared__ uint32_t chunk_start[kFineDigits];
  __shared__ uint32_t target_shift[kFineDigits];
  __shared__ uint32_t wave_totals[2 * kGW];
  __shared__ int32_t wave_flags[kGW];
  // (not const: the chunk loop rebuilds them, so that nothing derived from the
  // thread index is hoisted out of the loop and held in registers across it)
  int t = threadIdx.x;
  int lane = t & 63;
  int wave = t >> 6;

  // buckets dealt to XCDs in contiguous ranges: neighbouring buckets read the same lines of runs and rows
  const bool has_bucket = static_cast<int>(blockIdx.x) < buckets;
  const int b = has_bucket ? static_cast<int>(xcd_block(blockIdx.x, static_cast<unsigned int>(buckets))) : 0;
  const int fines = 1 << fine_bits;
  const uint32_t fine_mask = static_cast<uint32_t>(fines - 1);

  // the bucket's run in each of this thread's tiles (consecutive tiles),
  // loaded while the tiles' flags are reduced
  const int per = (tiles + kGT - 1) / kGT;
  const int first_tile = t * per;
  uint32_t run_first[kRunsPerThread], run_length[kRunsPerThread];
  uint32_t sum_start = 0u, sum_length = 0u;
#pragma unroll
  for (int i = 0; i < kRunsPerThread; ++i) {
    const int tile = first_tile + i;
    run_first[i] = 0u;
    run_length[i] = 0u;
    if (has_bucket && i < per && tile < tiles) {
      const uint32_t run = rows[static_cast<int64_t>(tile) * row_stride + b];  // first | end << 16
      run_first[i] = run & 0xffffu;
      run_length[i] = (run >> 16) - run_first[i];
    }
    sum_start += run_first[i];
    sum_length += run_length[i];
  }
  // the tiles' flags
  uint32_t local = 0u;
  for (int i = t; i < tiles; i += kGT) local |= tile_flags[i];
  wave_or_flags(static_cast<int32_t>(local), wave_flags);
  __syncthreads();
  const int32_t found = wave_or_read<kGT>(wave_flags);
  if (blockIdx.x == 0 && t == 0) {
    if (or_status)
      atomicOr(status, found);
    else
      *status = found;
  }
  if (!(found & kFlagUnsorted)) {
    boundary_offsets<int64_t, kGT>(keys, n_edges, n_nodes, offsets, order, blockIdx.x, gridDim.x,
                                   *reinterpret_cast<Gaps*>(region));
    return;
  }
  if (!has_bucket) return;
  uint32_t count = 0u, bucket_start = 0u;
  uint32_t placed = block_exclusive_scan2<kGT>(sum_length, sum_start, wave_totals, count, bucket_start);
  uint32_t run_delta[kRunsPerThread];
#pragma unroll
  for (int i = 0; i < kRunsPerThread; ++i) {
    run_delta[i] = static_cast<uint32_t>(first_tile + i) * kTile + run_first[i] - placed;
    run_first[i] = placed;  // from here: the run's first position in the bucket
    placed += run_length[i];
  }
  for (int i = t; i < kGW * kFineDigits; i += kGT) wave_base[i] = 0u;
  for (int f = t; f < kFineDigits; f += kGT) fine_base[f] = 0u;

  const BufferView packed_view = buffer_view(packed, n_edges * 4);
  uint32_t* mark = reinterpret_cast<uint32_t*>(region);
  // The chunk's elements in equal spans of whole rounds, one span a wave in
  // order: value[r] of element j = wave * span + 64 r + lane for r < rounds
  // (bit r of the result: j < in_chunk; zero elsewhere).
  const auto span_rounds = [](int in_chunk) {
    return (in_chunk + kGW * 64 - 1) / (kGW * 64);
  };
  const auto gather = [&](uint32_t c0, int in_chunk, uint32_t (&value)[kRounds]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int rounds = span_rounds(in_chunk);
    const int first = wave * 64 * rounds + lane;
    u32x4* mark4 = reinterpret_cast<u32x4*>(mark);
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < kMarks / 4; ++k) mark4[t * (kMarks / 4) + k] = zero;
    __syncthreads();
    // the first position of every run that meets the chunk gets delta + 1
#pragma unroll
    for (int i = 0; i < kRunsPerThread; ++i) {
      const uint32_t rs = run_first[i], re = run_first[i] + run_length[i];
      if (run_length[i] > 0u && re > c0 && rs < c0 + static_cast<uint32_t>(in_chunk))
        mark[(rs > c0 ? rs : c0) - c0] = run_delta[i] + 1u;
    }
    __syncthreads();
    // running maximum over the chunk
    uint32_t m[kMarks];
#pragma unroll
    for (int k = 0; k < kMarks / 4; ++k) {
      const u32x4 four = mark4[t * (kMarks / 4) + k];
      m[4 * k] = four.x;
      m[4 * k + 1] = four.y;
      m[4 * k + 2] = four.z;
      m[4 * k + 3] = four.w;
    }
    uint32_t running = 0u;
#pragma unroll
    for (int k = 0; k < kMarks; ++k) running = max(running, m[k]);
    running = block_exclusive_max<kGT>(running, wave_totals);
#pragma unroll
    for (int k = 0; k < kMarks; ++k) m[k] = running = max(running, m[k]);
#pragma unroll
    for (int k = 0; k < kMarks / 4; ++k) {
      const u32x4 four = {m[4 * k], m[4 * k + 1], m[4 * k + 2], m[4 * k + 3]};
      mark4[t * (kMarks / 4) + k] = four;
    }
    __syncthreads();
    uint32_t valid = 0u;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      value[r] = 0u;
      if (r >= rounds) continue;
      const int j = first + 64 * r;
      // every position carries a mark (position 0 lies in a run); past the chunk the view reads zero
      const uint32_t source = mark[j] - 1u + c0 + static_cast<uint32_t>(j);
      const bool inside = j < in_chunk;
      valid |= inside ? (1u << r) : 0u;
      // (cached: the neighbouring buckets gathered beside this one read the same lines)
      value[r] = load_u32(packed_view, inside ? source * 4u : kNoRow);
    }
    return valid;
  };
  const auto write_offsets = [&]() {
    for (int f = t; f < fines; f += kGT) {
      const int64_t key = (static_cast<int64_t>(b) << fine_bits) + f;
      if (key < n_nodes) offsets[key] = fine_base[f];
    }
    if (b == buckets - 1 && t == 0) offsets[n_nodes] = static_cast<int64_t>(bucket_start) + count;
  };
  const bool one_chunk = count <= static_cast<uint32_t>(kChunk);

  if (!one_chunk) {
    // the bucket's fine-digit histogram -> offsets of its keys
    for (uint32_t c0 = 0u; c0 < count; c0 += kChunk) {
      const int in_chunk = static_cast<int>(count - c0 < static_cast<uint32_t>(kChunk) ? count - c0 : kChunk);
      uint32_t value[kRounds];
      const uint32_t valid = gather(c0, in_chunk, value);
#pragma unroll
      for (int r = 0; r < kRounds; ++r)
        if ((valid >> r) & 1u) atomicAdd(&fine_base[value[r] & fine_mask], 1u);
      __syncthreads();  // the marks are read before the next chunk clears them
    }
    lds_exclusive_scan<kGT>(fine_base, fines, bucket_start, wave_totals);
    write_offsets();
    if (order == nullptr) return;
  }

  // an empty bucket takes one (empty) round too: it still writes its keys' offsets
  for (uint32_t c0 = 0u; c0 < count || c0 == 0u; c0 += kChunk) {
    asm volatile("" : "+v"(t));
    lane = t & 63;
    wave = t >> 6;
    const int in_chunk = static_cast<int>(count - c0 < static_cast<uint32_t>(kChunk) ? count - c0 : kChunk);
    uint32_t value[kRounds], rank[kRounds];
    const uint32_t valid = gather(c0, in_chunk, value);
    const auto fine = [&](int r) { return value[r] & fine_mask; };
    uint32_t* counter = wave_base + wave * kFineDigits;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) rank[r] = 0u;
    wave_ballot_ranks<kFB, kRounds>(fine, valid, counter, rank, span_rounds(in_chunk));
#pragma unroll
    for (int r = 0; r < kRounds; ++r) asm volatile("" : "+v"(value[r]));
    __syncthreads();
    if (wave == 0) {
      // lane l: fine digits f = l + 64 h (digits past `fines` count nothing).
      // Their counts in every wave, scanned over the digits (within the wave,
      // then after the previous group of 64) and then over the waves, become
      // the place of each wave's first element of the digit.
      uint32_t carry = 0u;
#pragma unroll
      for (int h = 0; h < kFineDigits / 64; ++h) {
        const int f = 64 * h + lane;
        uint32_t counts[kGW], total = 0u;
#pragma unroll
        for (int w = 0; w < kGW; ++w) {
          counts[w] = wave_base[w * kFineDigits + f];
          total += counts[w];
        }
        const uint32_t inclusive = wave_inclusive_scan(total);
        const uint32_t start = carry + inclusive - total;
        carry += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(inclusive), 63));
        uint32_t running = start;
#pragma unroll
        for (int w = 0; w < kGW; ++w) {
          wave_base[w * kFineDigits + f] = running;
          running += counts[w];
        }
        chunk_start[f] = start;
        // a bucket of one chunk: its digit counts are the histogram
        const uint32_t base = one_chunk ? bucket_start + start : fine_base[f];
        fine_base[f] = base;
        target_shift[f] = base - start;
      }
    }
    __syncthreads();
    if (one_chunk) {
      write_offsets();
      if (order == nullptr) return;
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) rank[r] += ((valid >> r) & 1u) ? counter[fine(r)] : 0u;
    // (the marks were all read before the ranking's barriers: the sorted chunk may overwrite them)
    uint32_t* sorted = mark;
#pragma unroll
    for (int r = 0; r < kRounds; ++r)
      if ((valid >> r) & 1u) sorted[rank[r]] = value[r];
    __syncthreads();
    const uint32_t end = bucket_start + count;
    for (int p = t; p < in_chunk; p += kGT) {
      const uint32_t e = sorted[p];
      const uint32_t target = target_shift[e & fine_mask] + static_cast<uint32_t>(p);
      // unreachable outside the bucket: its fine digits were counted from the same elements
      // (non-temporal: the order is not read again by this build, so it streams past L2)
      if (target >= bucket_start && target < end)
        __builtin_nontemporal_store(static_cast<int64_t>(e >> fine_bits), order + target);
    }
    if (c0 + kChunk >= count) break;  // the last chunk: nothing follows it
    __syncthreads();
    // the next chunk's elements of digit f follow this chunk's; the wave counters restart
    for (int f = t; f < fines; f += kGT) {
      const uint32_t next = f + 1 < fines ? chunk_start[f + 1] : static_cast<uint32_t>(in_chunk);
      fine_base[f] += next - chunk_start[f];
    }
    for (int i = t; i < kGW * kFineDigits; i += kGT) wave_base[i] = 0u;
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
  bool grouped = false;  // the two-launch form: tile grouping, then bucket gathers
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
      grouped = !wide && fine_bits <= kGroupedFineBits && tiles <= kMaxRunTiles;
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
  uint32_t* tile_flags = nullptr;  // grouped path: per tile
  void* packed = nullptr;         // two-level path
  uint32_t* keys[2] = {nullptr, nullptr};   // LSD ping-pong
  uint32_t* index[2] = {nullptr, nullptr};
};

size_t scratch_bytes(const Plan& plan) {
  const size_t edges = static_cast<size_t>(plan.n_edges > 0 ? plan.n_edges : 1);
  const size_t tiles = static_cast<size_t>(plan.tiles > 0 ? plan.tiles : 1);
  size_t bytes = 256 + 256 + round_up_256(tiles * kMaxBuckets * 4) + round_up_256(kMaxBuckets * 4) +
                 round_up_256((kMaxBuckets + 1) * 4) + round_up_256(kMaxRunTiles * 4);
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
  out.tile_flags = carver.take<uint32_t>(kMaxRunTiles);
  if (plan.two_level) {
    out.packed = carver.take<char>(edges * (plan.wide ? 8 : 4));
    return out.flags && out.valid_count && out.counts && out.bucket_total && out.bucket_start && out.tile_flags &&
           out.packed;
  }
  for (int k = 0; k < 2; ++k) {
    out.keys[k] = carver.take<uint32_t>(edges);
    out.index[k] = carver.take<uint32_t>(edges);
  }
  return out.flags && out.valid_count && out.counts && out.bucket_total && out.bucket_start && out.tile_flags &&
         out.keys[0] && out.keys[1] && out.index[0] && out.index[1];
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
  // the grouped path's gather writes the status word itself (ORs into it after the slot checks)
  if (!plan.grouped || n_rows > 0 || plan.n_edges == 0) {
    clear_word_kernel<<<1, 64, 0, stream>>>(status);
    if (int code = launched("clear_word_kernel")) return code;
  }
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
  if (plan.grouped) {
    const int64_t row_stride = plan.buckets;
    uint32_t* rows = s.counts;
    uint32_t* packed = static_cast<uint32_t*>(s.packed);
    tile_group_kernel<<<tiles, kThreads, 0, stream>>>(keys, plan.n_edges, nodes, plan.fine_bits, plan.buckets, packed,
                                                      rows, row_stride, s.tile_flags);
    if (int code = launched("tile_group_kernel")) return code;
    // one workgroup per bucket; at least 512 for the boundary path of sorted keys
    const unsigned int blocks =
        static_cast<unsigned int>(std::max<int64_t>(plan.buckets, std::min<int64_t>(boundary_blocks, 512)));
    const auto gather = [&](auto kernel) {
      kernel<<<blocks, kGatherThreads, 0, stream>>>(packed, rows, row_stride, s.tile_flags,
                                                     static_cast<int>(plan.tiles), plan.buckets, plan.fine_bits, keys,
                                                     plan.n_edges, plan.n_nodes, order, offsets, status,
                                                     n_rows > 0 ? 1 : 0);
      return launched("bucket_gather_kernel");
    };
    // instances by the fine digits (6 or 7 bits) and the tiles (1024 or 2048) they hold
    const bool small = plan.n_edges * 20 <= static_cast<int64_t>(plan.buckets) * kGatherSmallChunk * 19;
    const bool fine7 = plan.fine_bits > kFineMatchBits, tiles2k = plan.tiles > kMaxRunTiles / 2;
#define DPA4K_GATHER(FB, TILES)                                                                    \
  return small ? gather(bucket_gather_kernel<kGatherThreads, kGatherSmallChunk, 8, FB, TILES>)      \
               : gather(bucket_gather_kernel<kGatherThreads, kGatherLargeChunk, 6, FB, TILES>)
    if (fine7) {
      if (tiles2k) DPA4K_GATHER(7, 2048);
      DPA4K_GATHER(7, 1024);
    }
    if (tiles2k) DPA4K_GATHER(6, 2048);
    DPA4K_GATHER(6, 1024);
#undef DPA4K_GATHER
  }
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
    // the fine digits are matched over 6 bits when they fit, else over all kFineBitsMax
    const auto finish = [&](auto element) {
      using P = decltype(element);
      const P* packed = static_cast<const P*>(s.packed);
      if constexpr (sizeof(P) == 4) {
        if (plan.fine_bits <= 6) {
          finish_private_kernel<<<finish_blocks, kThreads, 0, stream>>>(
              packed, s.bucket_start, buckets, plan.fine_bits, keys, plan.n_edges, plan.n_nodes, order, offsets,
              status);
          return launched("finish_private_kernel");
        }
      }
      if (plan.fine_bits <= 6)
        finish_kernel<P, 6><<<finish_blocks, kThreads, 0, stream>>>(packed, s.bucket_start, buckets, plan.fine_bits,
                                                                    keys, plan.n_edges, plan.n_nodes, order, offsets,
                                                                    status);
      else
        finish_kernel<P, kFineBitsMax><<<finish_blocks, kThreads, 0, stream>>>(
            packed, s.bucket_start, buckets, plan.fine_bits, keys, plan.n_edges, plan.n_nodes, order, offsets,
            status);
      return launched("finish_kernel");
    };
    if (plan.wide) {
      const PackedOut<uint64_t> packed{static_cast<uint64_t*>(s.packed), plan.fine_bits};
      if (int code = plan.narrow_elements ? scatter(packed, uint32_t(0)) : scatter(packed, uint64_t(0))) return code;
      return finish(uint64_t(0));
    }
    const PackedOut<uint32_t> packed{static_cast<uint32_t*>(s.packed), plan.fine_bits};
    if (int code = plan.narrow_elements ? scatter(packed, uint32_t(0)) : scatter(packed, uint64_t(0))) return code;
    return finish(uint32_t(0));
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

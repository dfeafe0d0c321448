// segment_softmax forward and backward (python/kernels/segment.py:233-280,
// csrc/segment_softmax.cpp:235-343 of the reference; the arithmetic follows
// the oracle chain python/reference/segment.py:63-118).
//
// Per segment and channel, in the base-2 domain:
//   y_e = logit_e * log2(e) + 2 log2(max(env_e, 1e-30))   (env_e > 0; else no mass)
//   m = max(null * log2(e), max_e y_e),  w_e = 2^(y_e - m),  D = 2^(null log2 e - m) + sum_e w_e
//   alpha_e = w_e * (1 / D),  null_alpha = 2^(null log2 e - m) * (1 / D)
// which is the natural-base softmax of the reference with the exponent
// rescaled once; v_exp_f32 / v_log_f32 / v_rcp_f32 evaluate it (relative error
// a few 1e-7, inside the 1e-5 parity bar).
//
// Work decomposition (rows of up to 64 vector chunks, C <= 256):
//   * LC lanes cover one edge row (LC = next power of two >= C / V).
//   * Short segments (degree <= CAP) belong to G-lane groups (G = 32, or 64
//     when LC = 64): the group issues all of its segment's loads at once into
//     RMAX register tiles of PG = G / LC rows, so one memory round trip
//     brings the whole segment in; max, sum and normalisation run on the
//     registers and alpha is written once.
//   * Long segments (degree > CAP) belong to a whole 256-thread workgroup:
//     up to RMAXB tiles of PB = 256 / LC rows are staged in registers (one
//     read); longer segments stream twice (an online max/sum pass, then the
//     write pass).  Partial results of the four waves meet in LDS in a fixed
//     order.
//   * With a plan (dpa4k_segment_softmax_plan: the list of long segments of
//     the CSR, built once per graph), workgroups [0, n_long) take one long
//     segment each and the remaining workgroups take SPB consecutive
//     segments and skip the long ones, so no workgroup runs a long segment
//     after its short ones.  This is the degree-binned schedule.  Without a
//     plan, a workgroup handles its own long segments after its short ones.
// All reductions are DPP / ds_swizzle / ds_bpermute butterflies or fixed LDS
// orders: results are reproducible bit for bit from run to run.
// Rows wider than 64 chunks use a channel-major kernel (one lane per chunk).
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr float kLog2e = 1.4426950408889634f;
// Plan layout (int64 words): [0] short-path capacity the plan was built for,
// [1] n_long, [2, 2 + n_long) ascending ids of the long segments, then
// scratch (one count per tile of segments).
constexpr int64_t kPlanHeader = 2;

// ---------------------------------------------------------------------------
// arithmetic
// ---------------------------------------------------------------------------

// y = logit * log2(e) + 2 log2(max(env, 1e-30)) for env > 0, else -inf.
__device__ __forceinline__ float log2_weight(float logit, float env) {
  return env > 0.0f ? logit * kLog2e + 2.0f * __builtin_amdgcn_logf(fmaxf(env, 1e-30f)) : -INFINITY;
}

__device__ __forceinline__ float exp2_of(float x) { return __builtin_amdgcn_exp2f(x); }

// 2^(y - peak), zero when the segment has no mass (peak = -inf).
__device__ __forceinline__ float weight_of(float y, float peak) {
  return peak > -INFINITY ? exp2_of(y - peak) : 0.0f;
}

// The per-row part of y: 2 log2(max(env, 1e-30)) for env > 0, -inf otherwise.
__device__ __forceinline__ float row_term(float env) {
  return env > 0.0f ? 2.0f * __builtin_amdgcn_logf(fmaxf(env, 1e-30f)) : -INFINITY;
}

// y of one value from its row's term: -inf for a row without mass, whatever
// the logit.
__device__ __forceinline__ float log2_weight_of_row(float logit, float term) {
  return term > -INFINITY ? __builtin_fmaf(logit, kLog2e, term) : -INFINITY;
}

// The exponent shift of a column: its peak, or 0 when it has no mass (every
// y is then -inf and 2^(y - 0) = 0).
__device__ __forceinline__ float shift_of(float peak) { return peak > -INFINITY ? peak : 0.0f; }

// 1 / D, with D = 1 for a segment without mass.
__device__ __forceinline__ float inverse_total(float total) {
  return __builtin_amdgcn_rcpf(total > 0.0f ? total : 1.0f);
}

// d l_e / d env = 2 / env where the clamp of the oracle is inactive, 0 elsewhere.
__device__ __forceinline__ float env_gradient(float row_sum, float env) {
  return env >= 1e-30f ? row_sum * 2.0f / env : 0.0f;
}

// Online (max, sum) state of a base-2 softmax: sum = sum_i 2^(y_i - max).
__device__ __forceinline__ void online_add(float& peak, float& sum, float y) {
  if (y == -INFINITY) return;
  if (y > peak) {
    sum = (peak == -INFINITY ? 0.0f : sum * exp2_of(peak - y)) + 1.0f;
    peak = y;
  } else {
    sum += exp2_of(y - peak);
  }
}

// Compensated accumulation (Neumaier's variant of Kahan summation) for the
// loops that run over a whole long segment in one lane.  Over millions of
// rows a plain fp32 running sum drops the many terms far below its own
// magnitude (each rounds away) and comes out biased low: about 5e-4 for a
// 67M-row segment of N(0, 4) logits.  `carry` keeps what each addition
// rounded off; the caller folds it in once, with sum + carry.
__device__ __forceinline__ void compensated_add(float& sum, float& carry, float x) {
  const float t = sum + x;
  carry += fabsf(sum) >= fabsf(x) ? (sum - t) + x : (x - t) + sum;
  sum = t;
}

// online_add with a compensated sum; a new maximum rescales both parts.
__device__ __forceinline__ void online_add(float& peak, float& sum, float& carry, float y) {
  if (y == -INFINITY) return;
  if (y > peak) {
    const float scale = peak == -INFINITY ? 0.0f : exp2_of(peak - y);
    sum *= scale;
    carry *= scale;
    compensated_add(sum, carry, 1.0f);
    peak = y;
  } else {
    compensated_add(sum, carry, exp2_of(y - peak));
  }
}

// Merges (peak_b, sum_b) into (peak, sum); symmetric in its operands.
__device__ __forceinline__ void online_merge(float& peak, float& sum, float peak_b, float sum_b) {
  const float top = fmaxf(peak, peak_b);
  const float a = peak == -INFINITY ? 0.0f : sum * exp2_of(peak - top);
  const float b = peak_b == -INFINITY ? 0.0f : sum_b * exp2_of(peak_b - top);
  peak = top;
  sum = a + b;
}

// Butterflies over the lane bits [FROM, TO) of the wave.
template <int FROM, int TO>
__device__ __forceinline__ float span_max(float v) {
  if constexpr (FROM <= 1 && TO > 1) v = fmaxf(v, xor_lane<1>(v));
  if constexpr (FROM <= 2 && TO > 2) v = fmaxf(v, xor_lane<2>(v));
  if constexpr (FROM <= 4 && TO > 4) v = fmaxf(v, xor_lane<4>(v));
  if constexpr (FROM <= 8 && TO > 8) v = fmaxf(v, xor_lane<8>(v));
  if constexpr (FROM <= 16 && TO > 16) v = fmaxf(v, xor_lane<16>(v));
  if constexpr (FROM <= 32 && TO > 32) v = fmaxf(v, xor_lane<32>(v));
  return v;
}

template <int FROM, int TO>
__device__ __forceinline__ float span_sum(float v) {
  if constexpr (FROM <= 1 && TO > 1) v += xor_lane<1>(v);
  if constexpr (FROM <= 2 && TO > 2) v += xor_lane<2>(v);
  if constexpr (FROM <= 4 && TO > 4) v += xor_lane<4>(v);
  if constexpr (FROM <= 8 && TO > 8) v += xor_lane<8>(v);
  if constexpr (FROM <= 16 && TO > 16) v += xor_lane<16>(v);
  if constexpr (FROM <= 32 && TO > 32) v += xor_lane<32>(v);
  return v;
}

template <int MASK>
__device__ __forceinline__ void merge_lane(float& peak, float& sum) {
  const float peak_b = xor_lane<MASK>(peak);
  const float sum_b = xor_lane<MASK>(sum);
  online_merge(peak, sum, peak_b, sum_b);
}

template <int FROM, int TO>
__device__ __forceinline__ void span_merge(float& peak, float& sum) {
  if constexpr (FROM <= 1 && TO > 1) merge_lane<1>(peak, sum);
  if constexpr (FROM <= 2 && TO > 2) merge_lane<2>(peak, sum);
  if constexpr (FROM <= 4 && TO > 4) merge_lane<4>(peak, sum);
  if constexpr (FROM <= 8 && TO > 8) merge_lane<8>(peak, sum);
  if constexpr (FROM <= 16 && TO > 16) merge_lane<16>(peak, sum);
  if constexpr (FROM <= 32 && TO > 32) merge_lane<32>(peak, sum);
}

// ---------------------------------------------------------------------------
// geometry
// ---------------------------------------------------------------------------

// Short-path capacity (rows) for rows of LC lanes: 24 / V tiles of a
// 32-lane group.  Forward and backward share it, so one plan serves both.
constexpr int short_capacity(int v, int lc) { return (24 / v) * ((lc > 32 ? lc : 32) / lc); }

// Lanes per short group: 32, or LC when a row is wider.  (16-lane groups
// with twice the tiles fit a config-2-like graph into one dispatch round
// but need over 96 VGPRs, which halves the occupancy, and ran slower.)
constexpr int short_group_log(int v, int log_lc, bool backward) {
  (void)v;
  (void)backward;
  return log_lc > 5 ? log_lc : 5;
}

template <int V, int LOG_LC, bool kBackward = false>
struct Geo {
  static constexpr int LC = 1 << LOG_LC;               // lanes per edge row
  static constexpr int LOG_G = short_group_log(V, LOG_LC, kBackward);
  static constexpr int G = 1 << LOG_G;                 // lanes per short segment
  static constexpr int GPW = 64 / G;                   // short segments per wave
  static constexpr int PG = G / LC;                    // rows per group load
  static constexpr int SPB = kBlock / G;               // segments per short workgroup
  static constexpr int PB = kBlock / LC;               // rows per workgroup load
  static constexpr int CAP = short_capacity(V, LC);    // longest short segment
  static constexpr int RMAX = CAP / PG;                // register tiles, short path
  static constexpr int RMAXB = 16 / V;                 // register tiles, staged long path
  static constexpr int UNROLL = 2;                     // loads in flight per thread, streaming path
};

// Register tiles of rows: tile i holds, for this lane, the row of CSR slot
// first + i * STEP + row_lane when that slot is below `end` and the lane is
// live (its column lies inside the row).
//
// Natural order (slot = edge): rows are read and written through buffer
// views rebased at `base` (wave-uniform, at most the lowest slot of the
// active lanes), and a lane without a row uses kNoRow; callers keep every
// slot of the window within 2^31 bytes of `base`.  No load sits in a branch.
// With an order: the order entries of every tile are loaded first (at slot 0
// for lanes without a row), then the rows they name at a clamped index; `e`
// keeps the edge id, or -1 where there is no row.  Callers guard the ordered
// loads with n_edges > 0, so index 0 exists.  A lane that is not live reads
// column 0 instead of its own (null rows included); its results are neither
// stored nor reduced into the live lanes' results.
template <int R, int STEP, bool kOrdered>
struct Tiles {
  int64_t first, base;
  int32_t rows_left;  // min(end - first, 2^31 - 1)
  int row_lane;
  bool live;
  uint32_t row_bytes, col_bytes;
  int64_t e[kOrdered ? R : 1];

  __device__ __forceinline__ Tiles(int64_t first_, int64_t end, int64_t base_, int row_lane_, bool live_,
                                   int64_t column, int64_t channels)
      : first(first_), base(kOrdered ? 0 : base_), row_lane(row_lane_), live(live_) {
    const int64_t left = end - first_;
    rows_left = static_cast<int32_t>(left < 0 ? 0 : (left > 0x7fffffff ? 0x7fffffff : left));
    row_bytes = static_cast<uint32_t>(channels) * 4u;
    col_bytes = static_cast<uint32_t>(column) * 4u;
  }
  __device__ __forceinline__ bool row(int i) const { return live & (i * STEP + row_lane < rows_left); }
  // kNoRow without a row, 0 with one; folded into offsets by an OR, which keeps
  // the offset arithmetic free of selects (a select here becomes a branch).
  __device__ __forceinline__ uint32_t miss(int i) const { return (static_cast<uint32_t>(row(i)) - 1u) & kNoRow; }
  __device__ __forceinline__ int64_t slot(int i) const { return first + static_cast<int64_t>(i) * STEP + row_lane; }
  // natural order: byte offsets of this lane's chunk and of its row's scalar
  __device__ __forceinline__ uint32_t rel(int i) const {
    return static_cast<uint32_t>(first - base) + static_cast<uint32_t>(i * STEP + row_lane);
  }
  __device__ __forceinline__ uint32_t at(int i) const { return (rel(i) * row_bytes + col_bytes) | miss(i); }
  __device__ __forceinline__ uint32_t scalar_at(int i) const { return (rel(i) * 4u) | miss(i); }
  // ordered: edge ids of every tile
  __device__ __forceinline__ void gather_ids(const int64_t* __restrict__ order, int64_t n_edges) {
    if constexpr (kOrdered) {
#pragma unroll
      for (int i = 0; i < R; ++i) e[i] = order[row(i) ? slot(i) : 0];
#pragma unroll
      for (int i = 0; i < R; ++i) e[i] = row(i) && e[i] >= 0 && e[i] < n_edges ? e[i] : -1;
    }
  }
  __device__ __forceinline__ void clear_ids() {
    if constexpr (kOrdered)
#pragma unroll
      for (int i = 0; i < R; ++i) e[i] = -1;
  }
};

// Lane roles inside a workgroup for rows of LC lanes (short groups of the
// forward or the backward geometry).
template <int V, int LOG_LC, bool kBackward = false>
struct Lanes {
  using S = Geo<V, LOG_LC, kBackward>;
  int lane, wave, k, p, pb, gidx;
  bool live;
  int64_t column;
  __device__ Lanes(int64_t chunks) {
    lane = threadIdx.x & 63;
    wave = threadIdx.x >> 6;
    k = lane & (S::LC - 1);
    p = (threadIdx.x & (S::G - 1)) >> LOG_LC;
    pb = threadIdx.x >> LOG_LC;
    gidx = threadIdx.x >> S::LOG_G;
    live = k < chunks;
    column = static_cast<int64_t>(k) * V;
  }
};

// Segment bounds of the SPB segments [first, first + SPB) held by lanes
// 0..SPB of every wave (one vector load); lane i gets segment first + i.
struct BlockBounds {
  int64_t lo, hi;
};

template <int SPB>
__device__ __forceinline__ BlockBounds block_bounds(const int64_t* __restrict__ offsets, int64_t first,
                                                    int64_t n_nodes, int64_t n_edges) {
  const int lane = threadIdx.x & 63;
  const int64_t last = first + SPB < n_nodes ? first + SPB : n_nodes;
  const int64_t index = first + lane < last ? first + lane : last;
  int64_t lo = offsets[index];
  lo = lo < 0 ? 0 : (lo > n_edges ? n_edges : lo);
  int64_t hi = __shfl_down(lo, 1);
  if (hi < lo || first + lane >= last) hi = lo;
  return {lo, hi};
}

// Bounds of this lane's group among the 64 / G consecutive segments of its
// wave (segments first + wave * 64 / G + j), read with scalar loads: the
// addresses are wave-uniform, so no vector load and no lane shuffle stands
// between the kernel's start and the first row loads.
template <int LOG_G>
__device__ __forceinline__ void group_bounds(const int64_t* __restrict__ offsets, int64_t first, int64_t n_nodes,
                                             int64_t n_edges, int64_t& begin, int64_t& end) {
  constexpr int GPW = 64 >> LOG_G;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t s0 = first + static_cast<int64_t>(wave) * GPW;
  int64_t o[GPW + 1];
#pragma unroll
  for (int j = 0; j <= GPW; ++j) o[j] = offsets[s0 + j < n_nodes ? s0 + j : n_nodes];
  __builtin_amdgcn_sched_barrier(0);  // the loads above overlap; clamps follow
#pragma unroll
  for (int j = 0; j <= GPW; ++j) o[j] = o[j] < 0 ? 0 : (o[j] > n_edges ? n_edges : o[j]);
  const int g = static_cast<int>(threadIdx.x & 63) >> LOG_G;
  begin = o[0];
  end = o[1];
#pragma unroll
  for (int j = 1; j < GPW; ++j)
    if (g == j) {
      begin = o[j];
      end = o[j + 1];
    }
  if (end < begin) end = begin;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------

struct ForwardArgs {
  const float* logit;
  const float* env;
  const int64_t* offsets;
  const float* null_logit;
  const int64_t* order;
  float* alpha;
  float* null_alpha;
  int64_t n_edges, n_nodes, channels;
};

// Loads tile i of the forward input for this lane: the logit chunk and the
// envelope (0, hence no mass, where the lane has no row).  Natural order
// reads through the views; with an order the caller has gathered the ids.
template <int V, int R, int STEP, bool kOrdered>
__device__ __forceinline__ void forward_loads(const ForwardArgs& a, const Tiles<R, STEP, kOrdered>& t,
                                              int64_t column, float (&value)[R][V], float (&envelope)[R]) {
  if constexpr (!kOrdered) {
    const BufferView logit = row_view(a.logit, t.base, a.n_edges, a.channels);
    const BufferView env = row_view(a.env, t.base, a.n_edges, 1);
    // Logit rows are read once and loaded non-temporally (config 2: 14.3 ->
    // 13.7 us, 2R: 138 -> 127 us); the envelope loads keep the default
    // policy, which was faster for them.
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const fvec<V> x = buffer_load_vec<V, kNonTemporal>(logit, t.at(i));
      envelope[i] = buffer_load_f32(env, t.scalar_at(i));
#pragma unroll
      for (int v = 0; v < V; ++v) value[i][v] = x.v[v];
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any use
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t e = t.e[i] >= 0 ? t.e[i] : 0;
      const fvec<V> x = load_vec_stream<V>(a.logit + e * a.channels + column);
      const float env = a.env[e];
      envelope[i] = t.e[i] >= 0 ? env : 0.0f;
#pragma unroll
      for (int v = 0; v < V; ++v) value[i][v] = x.v[v];
    }
  }
}

// Stores alpha of tile i where the lane has a row (tiles [0, tiles) hold
// every row of the lane).
template <int V, int R, int STEP, bool kOrdered>
__device__ __forceinline__ void forward_stores(const ForwardArgs& a, const Tiles<R, STEP, kOrdered>& t,
                                               int64_t column, const float (&alpha)[R][V], int tiles = R) {
  if constexpr (!kOrdered) {
    const BufferView out = row_view(a.alpha, t.base, a.n_edges, a.channels);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (i >= tiles) continue;
      fvec<V> row;
#pragma unroll
      for (int v = 0; v < V; ++v) row.v[v] = alpha[i][v];
      buffer_store_vec_stream<V>(out, t.at(i), row);
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (t.e[i] >= 0) {
        fvec<V> row;
#pragma unroll
        for (int v = 0; v < V; ++v) row.v[v] = alpha[i][v];
        store_vec_stream<V>(a.alpha + t.e[i] * a.channels + column, row);
      }
    }
  }
}

// Tiles of [first, end) with every load issued before any arithmetic.
template <int V, int R, int STEP, bool kOrdered>
__device__ __forceinline__ Tiles<R, STEP, kOrdered> forward_tiles(const ForwardArgs& a, int64_t first, int64_t end,
                                                                  int64_t base, int row_lane, bool live,
                                                                  int64_t column, float (&value)[R][V],
                                                                  float (&envelope)[R]) {
  Tiles<R, STEP, kOrdered> t(first, end, base, row_lane, live, column, a.channels);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    envelope[i] = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) value[i][v] = 0.0f;
  }
  if constexpr (kOrdered) {
    t.clear_ids();
    if (a.n_edges > 0) {
      t.gather_ids(a.order, a.n_edges);
      forward_loads<V>(a, t, column, value, envelope);
    }
  } else {
    forward_loads<V>(a, t, column, value, envelope);
  }
  return t;
}

// One long segment [begin, end) of `segment`, processed by the whole workgroup.
template <int V, int LOG_LC, bool kNull, bool kOrdered>
__device__ void forward_long(const ForwardArgs& a, int64_t segment, int64_t begin, int64_t end,
                             float (*partial)[2][Geo<V, LOG_LC>::LC * V]) {
  using S = Geo<V, LOG_LC>;
  begin = uniform_i64(begin);  // one segment per workgroup
  end = uniform_i64(end);
  constexpr int LC = S::LC, PB = S::PB, RMAXB = S::RMAXB;
  const Lanes<V, LOG_LC> L(a.channels / V);
  const int64_t column = L.live ? L.column : 0;
  const int64_t degree = end - begin;
  fvec<V> n0;
#pragma unroll
  for (int v = 0; v < V; ++v) n0.v[v] = -INFINITY;
  if constexpr (kNull) n0 = load_vec<V>(a.null_logit + segment * a.channels + column);
  float nv[V];
#pragma unroll
  for (int v = 0; v < V; ++v) nv[v] = n0.v[v] * kLog2e;
  float peak[V], total[V];
  if (degree <= RMAXB * PB) {
    // staged: every row of the segment in registers, one read
    float value[RMAXB][V], envelope[RMAXB];
    const auto t = forward_tiles<V, RMAXB, PB, kOrdered>(a, begin, end, begin, L.pb, L.live, column, value, envelope);
#pragma unroll
    for (int v = 0; v < V; ++v) peak[v] = -INFINITY;
#pragma unroll
    for (int i = 0; i < RMAXB; ++i)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        value[i][v] = log2_weight(value[i][v], envelope[i]);
        peak[v] = fmaxf(peak[v], value[i][v]);
      }
#pragma unroll
    for (int v = 0; v < V; ++v) peak[v] = span_max<LC, 64>(peak[v]);
    if ((L.lane >> LOG_LC) == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[L.wave][0][L.k * V + v] = peak[v];
    __syncthreads();
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float m = partial[0][0][L.k * V + v];
      for (int q = 1; q < kWaves; ++q) m = fmaxf(m, partial[q][0][L.k * V + v]);
      peak[v] = kNull ? fmaxf(m, nv[v]) : m;
      total[v] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < RMAXB; ++i)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float w = weight_of(value[i][v], peak[v]);
        value[i][v] = w;
        total[v] += w;
      }
#pragma unroll
    for (int v = 0; v < V; ++v) total[v] = span_sum<LC, 64>(total[v]);
    if ((L.lane >> LOG_LC) == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[L.wave][1][L.k * V + v] = total[v];
    __syncthreads();
    float nw[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float sum = partial[0][1][L.k * V + v];
      for (int q = 1; q < kWaves; ++q) sum = sum + partial[q][1][L.k * V + v];
      nw[v] = kNull ? weight_of(nv[v], peak[v]) : 0.0f;
      total[v] = inverse_total(sum + nw[v]);
    }
#pragma unroll
    for (int i = 0; i < RMAXB; ++i)
#pragma unroll
      for (int v = 0; v < V; ++v) value[i][v] *= total[v];
    forward_stores<V>(a, t, column, value);
    if (kNull && threadIdx.x < LC && L.live) {
      fvec<V> out;
#pragma unroll
      for (int v = 0; v < V; ++v) out.v[v] = nw[v] * total[v];
      store_vec<V>(a.null_alpha + segment * a.channels + L.column, out);
    }
    __syncthreads();  // partial[] is reused by the next long segment
    return;
  }

  // streaming: online max/sum pass, then the write pass
  float run_sum[V], carry[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    peak[v] = -INFINITY;
    run_sum[v] = 0.0f;
    carry[v] = 0.0f;
  }
  for (int64_t base = begin; base < end; base += S::UNROLL * PB) {
    float value[S::UNROLL][V], envelope[S::UNROLL];
    forward_tiles<V, S::UNROLL, PB, kOrdered>(a, base, end, base, L.pb, L.live, column, value, envelope);
#pragma unroll
    for (int u = 0; u < S::UNROLL; ++u)
#pragma unroll
      for (int v = 0; v < V; ++v) online_add(peak[v], run_sum[v], carry[v], log2_weight(value[u][v], envelope[u]));
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    run_sum[v] = run_sum[v] + carry[v];
    span_merge<LC, 64>(peak[v], run_sum[v]);
  }
  if ((L.lane >> LOG_LC) == 0)
#pragma unroll
    for (int v = 0; v < V; ++v) {
      partial[L.wave][0][L.k * V + v] = peak[v];
      partial[L.wave][1][L.k * V + v] = run_sum[v];
    }
  __syncthreads();
  float nw[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    float m = partial[0][0][L.k * V + v];
    float s = partial[0][1][L.k * V + v];
    for (int q = 1; q < kWaves; ++q) online_merge(m, s, partial[q][0][L.k * V + v], partial[q][1][L.k * V + v]);
    if (kNull) online_add(m, s, nv[v]);
    peak[v] = m;
    nw[v] = kNull ? weight_of(nv[v], m) : 0.0f;
    total[v] = inverse_total(s);
  }
  for (int64_t base = begin; base < end; base += S::UNROLL * PB) {
    float value[S::UNROLL][V], envelope[S::UNROLL];
    const auto t = forward_tiles<V, S::UNROLL, PB, kOrdered>(a, base, end, base, L.pb, L.live, column, value, envelope);
#pragma unroll
    for (int u = 0; u < S::UNROLL; ++u)
#pragma unroll
      for (int v = 0; v < V; ++v) value[u][v] = weight_of(log2_weight(value[u][v], envelope[u]), peak[v]) * total[v];
    forward_stores<V>(a, t, column, value);
  }
  if (kNull && threadIdx.x < LC && L.live) {
    fvec<V> out;
#pragma unroll
    for (int v = 0; v < V; ++v) out.v[v] = nw[v] * total[v];
    store_vec<V>(a.null_alpha + segment * a.channels + L.column, out);
  }
  __syncthreads();
}

// Short segment of this lane's group (degree <= CAP), all in registers; rows
// are addressed from `base` (see Tiles).
template <int V, int LOG_LC, bool kNull, bool kOrdered>
__device__ __forceinline__ void forward_short(const ForwardArgs& a, int64_t segment, int64_t begin, int64_t end,
                                              int64_t base) {
  using S = Geo<V, LOG_LC>;
  constexpr int LC = S::LC, G = S::G, PG = S::PG, RMAX = S::RMAX;
  const Lanes<V, LOG_LC> L(a.channels / V);
  const int64_t column = L.live ? L.column : 0;
  const int64_t degree = end - begin;
  fvec<V> n0;
#pragma unroll
  for (int v = 0; v < V; ++v) n0.v[v] = -INFINITY;
  if constexpr (kNull) n0 = load_vec<V>(a.null_logit + segment * a.channels + column);
  float value[RMAX][V], envelope[RMAX];
  const auto t = forward_tiles<V, RMAX, PG, kOrdered>(a, begin, end, base, L.p, L.live, column, value, envelope);
  // Only the tiles that hold rows of the group are computed (the wave runs
  // the larger count of its groups).
  const int tiles = static_cast<int>((degree + PG - 1) / PG);
  float nv[V], peak[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    nv[v] = n0.v[v] * kLog2e;
    peak[v] = -INFINITY;
  }
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    if (i < tiles) {
      const float term = row_term(envelope[i]);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        value[i][v] = log2_weight_of_row(value[i][v], term);
        peak[v] = fmaxf(peak[v], value[i][v]);
      }
    }
  }
  float total[V], nw[V], shift[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    peak[v] = span_max<LC, G>(peak[v]);
    if (kNull) peak[v] = fmaxf(peak[v], nv[v]);
    shift[v] = shift_of(peak[v]);
    total[v] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    if (i < tiles) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float w = exp2_of(value[i][v] - shift[v]);
        value[i][v] = w;
        total[v] += w;
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    total[v] = span_sum<LC, G>(total[v]);
    nw[v] = kNull ? exp2_of(nv[v] - shift[v]) : 0.0f;
    total[v] = inverse_total(total[v] + nw[v]);
  }
#pragma unroll
  for (int i = 0; i < RMAX; ++i)
    if (i < tiles)
#pragma unroll
      for (int v = 0; v < V; ++v) value[i][v] *= total[v];
  forward_stores<V>(a, t, column, value, tiles);
  if (kNull && L.p == 0 && L.live) {
    fvec<V> out;
#pragma unroll
    for (int v = 0; v < V; ++v) out.v[v] = nw[v] * total[v];
    store_vec<V>(a.null_alpha + segment * a.channels + L.column, out);
  }
}

// Planned: workgroups [0, n_long) take the listed long segments, the others
// SPB consecutive segments each, skipping the long ones.  Unplanned: every
// workgroup takes SPB consecutive segments and runs its own long segments
// after its short ones.
template <int V, int LOG_LC, bool kNull, bool kOrdered, bool kPlanned>
__global__ __launch_bounds__(kBlock) void softmax_forward_kernel(ForwardArgs a, const int64_t* __restrict__ plan,
                                                                 int64_t n_long) {
  using S = Geo<V, LOG_LC>;
  __shared__ float partial[kWaves][2][S::LC * V];
  constexpr bool planned = kPlanned;
  const int64_t block = block_index();
  if (planned && block < n_long) {
    const int64_t segment = plan[kPlanHeader + block];
    if (static_cast<uint64_t>(segment) >= static_cast<uint64_t>(a.n_nodes)) return;
    int64_t begin, end;
    segment_bounds(a.offsets, segment, a.n_edges, begin, end);
    forward_long<V, LOG_LC, kNull, kOrdered>(a, segment, begin, end, partial);
    return;
  }
  const int64_t first = (block - (planned ? n_long : 0)) * S::SPB;
  const int gidx = threadIdx.x >> S::LOG_G;
  const int64_t segment = first + gidx;
  {
    int64_t begin, end;
    group_bounds<S::LOG_G>(a.offsets, first, a.n_nodes, a.n_edges, begin, end);
    // The rows of a wave's short groups (at most two) lie within 2 CAP slots
    // of the lowest short group's begin: one buffer window serves the wave.
    static_assert(S::GPW <= 2, "one row window per wave needs at most two short groups per wave");
    if (segment < a.n_nodes && end - begin <= S::CAP)
      forward_short<V, LOG_LC, kNull, kOrdered>(a, segment, begin, end, uniform_i64(begin));
  }
  if constexpr (planned) return;
  const BlockBounds bb = block_bounds<S::SPB>(a.offsets, first, a.n_nodes, a.n_edges);
  // no plan: this workgroup's long segments, one at a time
  const int lane = threadIdx.x & 63;
  unsigned long long longs =
      __ballot(lane < S::SPB && first + lane < a.n_nodes && bb.hi - bb.lo > S::CAP);
  while (longs != 0ull) {
    const int s = __ffsll(static_cast<long long>(longs)) - 1;
    longs &= longs - 1ull;
    forward_long<V, LOG_LC, kNull, kOrdered>(a, first + s, __shfl(bb.lo, s), __shfl(bb.hi, s), partial);
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------

struct BackwardArgs {
  const float* alpha;
  const float* grad_alpha;
  const float* env;
  const int64_t* offsets;
  const float* null_alpha;
  const float* grad_null_alpha;
  const int64_t* order;
  float* grad_logit;
  float* grad_null_logit;
  float* grad_env;
  int64_t n_edges, n_nodes, channels;
};

// Tiles of [first, end) for the backward: alpha, grad_alpha and the envelope
// of every row (zeros without a row), every load issued before any arithmetic.
template <int V, int R, int STEP, bool kOrdered>
__device__ __forceinline__ Tiles<R, STEP, kOrdered> backward_tiles(const BackwardArgs& a, int64_t first, int64_t end,
                                                                   int64_t base, int row_lane, bool live,
                                                                   int64_t column, float (&x)[R][V],
                                                                   float (&g)[R][V], float (&envelope)[R]) {
  Tiles<R, STEP, kOrdered> t(first, end, base, row_lane, live, column, a.channels);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    envelope[i] = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) x[i][v] = g[i][v] = 0.0f;
  }
  if constexpr (!kOrdered) {
    const BufferView alpha = row_view(a.alpha, t.base, a.n_edges, a.channels);
    const BufferView grad = row_view(a.grad_alpha, t.base, a.n_edges, a.channels);
    const BufferView env = row_view(a.env, t.base, a.n_edges, 1);
    // envelopes first: they are consumed last, after the row sums.  The rows
    // are read once and loaded non-temporally (config 2R: 222 -> 200 us).
#pragma unroll
    for (int i = 0; i < R; ++i) envelope[i] = buffer_load_f32(env, t.scalar_at(i));
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const fvec<V> xv = buffer_load_vec<V, kNonTemporal>(alpha, t.at(i));
      const fvec<V> gv = buffer_load_vec<V, kNonTemporal>(grad, t.at(i));
#pragma unroll
      for (int v = 0; v < V; ++v) {
        x[i][v] = xv.v[v];
        g[i][v] = gv.v[v];
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any use
  } else {
    t.clear_ids();
    if (a.n_edges > 0) {
      t.gather_ids(a.order, a.n_edges);
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int64_t e = t.e[i] >= 0 ? t.e[i] : 0;
        const fvec<V> xv = load_vec_stream<V>(a.alpha + e * a.channels + column);
        const fvec<V> gv = load_vec_stream<V>(a.grad_alpha + e * a.channels + column);
        const float env = a.env[e];
        const bool has = t.e[i] >= 0;
        envelope[i] = has ? env : 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          x[i][v] = has ? xv.v[v] : 0.0f;
          g[i][v] = has ? gv.v[v] : 0.0f;
        }
      }
    }
  }
  return t;
}

// grad_logit rows of the tiles from alpha, grad_alpha and the segment's S;
// grad_env of each row from the row sum over the LC lanes of the row.
template <int V, int LOG_LC, int R, int STEP, bool kOrdered>
__device__ __forceinline__ void backward_rows(const BackwardArgs& a, const Lanes<V, LOG_LC, true>& L,
                                              const Tiles<R, STEP, kOrdered>& t, int64_t column,
                                              const float (&x)[R][V], const float (&g)[R][V],
                                              const float (&expect)[V], const float (&envelope)[R],
                                              int tiles = R) {
  // natural order only (unused, and dropped by the compiler, with an order)
  const BufferView grad_logit = row_view(a.grad_logit, t.base, a.n_edges, a.channels);
  const BufferView grad_env = row_view(a.grad_env, t.base, a.n_edges, 1);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (i >= tiles) continue;  // no row of the lane's group in this tile or later ones
    const bool has = kOrdered ? t.e[i] >= 0 : t.row(i);
    fvec<V> out;
    float row = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      out.v[v] = x[i][v] * (g[i][v] - expect[v]);
      row += out.v[v];
    }
    row = span_sum<1, Geo<V, LOG_LC>::LC>(has ? row : 0.0f);
    const float d_env = env_gradient(row, envelope[i]);
    if constexpr (!kOrdered) {
      buffer_store_vec_stream<V>(grad_logit, t.at(i), out);
      buffer_store_f32(grad_env, L.k == 0 ? t.scalar_at(i) : kNoRow, d_env);
    } else {
      if (has) {
        store_vec_stream<V>(a.grad_logit + t.e[i] * a.channels + column, out);
        if (L.k == 0) a.grad_env[t.e[i]] = d_env;
      }
    }
  }
}

template <int V, int LOG_LC, bool kNull, bool kOrdered>
__device__ void backward_long(const BackwardArgs& a, int64_t segment, int64_t begin, int64_t end,
                              float (*partial)[2][Geo<V, LOG_LC>::LC * V]) {
  using S = Geo<V, LOG_LC>;
  begin = uniform_i64(begin);  // one segment per workgroup
  end = uniform_i64(end);
  constexpr int LC = S::LC, PB = S::PB, RMAXB = S::RMAXB;
  const Lanes<V, LOG_LC, true> L(a.channels / V);
  const int64_t column = L.live ? L.column : 0;
  const int64_t degree = end - begin;
  float a0[V], g0[V], expect[V];
#pragma unroll
  for (int v = 0; v < V; ++v) a0[v] = g0[v] = expect[v] = 0.0f;
  if constexpr (kNull) {
    const fvec<V> x = load_vec<V>(a.null_alpha + segment * a.channels + column);
    const fvec<V> g = load_vec<V>(a.grad_null_alpha + segment * a.channels + column);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      a0[v] = x.v[v];
      g0[v] = g.v[v];
    }
  }
  if (degree <= RMAXB * PB) {
    // staged: every row of the segment in registers, one read
    float xs[RMAXB][V], gs[RMAXB][V], envs[RMAXB];
    const auto t = backward_tiles<V, RMAXB, PB, kOrdered>(a, begin, end, begin, L.pb, L.live, column, xs, gs, envs);
#pragma unroll
    for (int i = 0; i < RMAXB; ++i)
#pragma unroll
      for (int v = 0; v < V; ++v) expect[v] = expect[v] + xs[i][v] * gs[i][v];
#pragma unroll
    for (int v = 0; v < V; ++v) expect[v] = span_sum<LC, 64>(expect[v]);
    if ((L.lane >> LOG_LC) == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[L.wave][0][L.k * V + v] = expect[v];
    __syncthreads();
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float sum = partial[0][0][L.k * V + v];
      for (int q = 1; q < kWaves; ++q) sum = sum + partial[q][0][L.k * V + v];
      expect[v] = kNull ? sum + a0[v] * g0[v] : sum;
    }
    backward_rows<V, LOG_LC>(a, L, t, column, xs, gs, expect, envs);
  } else {
    // streaming: the dot-product pass (compensated), then the gradient pass
    float carry[V];
#pragma unroll
    for (int v = 0; v < V; ++v) carry[v] = 0.0f;
    for (int64_t base = begin; base < end; base += S::UNROLL * PB) {
      float x[S::UNROLL][V], g[S::UNROLL][V], envs[S::UNROLL];
      backward_tiles<V, S::UNROLL, PB, kOrdered>(a, base, end, base, L.pb, L.live, column, x, g, envs);
#pragma unroll
      for (int u = 0; u < S::UNROLL; ++u)
#pragma unroll
        for (int v = 0; v < V; ++v) compensated_add(expect[v], carry[v], x[u][v] * g[u][v]);
    }
#pragma unroll
    for (int v = 0; v < V; ++v) expect[v] = span_sum<LC, 64>(expect[v] + carry[v]);
    if ((L.lane >> LOG_LC) == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[L.wave][0][L.k * V + v] = expect[v];
    __syncthreads();
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float sum = partial[0][0][L.k * V + v];
      for (int q = 1; q < kWaves; ++q) sum = sum + partial[q][0][L.k * V + v];
      expect[v] = kNull ? sum + a0[v] * g0[v] : sum;
    }
    for (int64_t base = begin; base < end; base += S::UNROLL * PB) {
      float x[S::UNROLL][V], g[S::UNROLL][V], envs[S::UNROLL];
      const auto t = backward_tiles<V, S::UNROLL, PB, kOrdered>(a, base, end, base, L.pb, L.live, column, x, g, envs);
      backward_rows<V, LOG_LC>(a, L, t, column, x, g, expect, envs);
    }
  }
  if (kNull && threadIdx.x < LC && L.live) {
    fvec<V> out;
#pragma unroll
    for (int v = 0; v < V; ++v) out.v[v] = a0[v] * (g0[v] - expect[v]);
    store_vec<V>(a.grad_null_logit + segment * a.channels + L.column, out);
  }
  __syncthreads();
}

template <int V, int LOG_LC, bool kNull, bool kOrdered>
__device__ __forceinline__ void backward_short(const BackwardArgs& a, int64_t segment, int64_t begin, int64_t end,
                                               int64_t base) {
  using S = Geo<V, LOG_LC, true>;
  constexpr int LC = S::LC, G = S::G, PG = S::PG, RMAX = S::RMAX;
  const Lanes<V, LOG_LC, true> L(a.channels / V);
  const int64_t column = L.live ? L.column : 0;
  float a0[V], g0[V], expect[V];
#pragma unroll
  for (int v = 0; v < V; ++v) a0[v] = g0[v] = expect[v] = 0.0f;
  if constexpr (kNull) {
    const fvec<V> x = load_vec<V>(a.null_alpha + segment * a.channels + column);
    const fvec<V> g = load_vec<V>(a.grad_null_alpha + segment * a.channels + column);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      a0[v] = x.v[v];
      g0[v] = g.v[v];
    }
  }
  float xs[RMAX][V], gs[RMAX][V], envs[RMAX];
  const auto t = backward_tiles<V, RMAX, PG, kOrdered>(a, begin, end, base, L.p, L.live, column, xs, gs, envs);
  const int tiles = static_cast<int>((end - begin + PG - 1) / PG);
#pragma unroll
  for (int i = 0; i < RMAX; ++i)
    if (i < tiles)
#pragma unroll
      for (int v = 0; v < V; ++v) expect[v] = expect[v] + xs[i][v] * gs[i][v];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    expect[v] = span_sum<LC, G>(expect[v]);
    if (kNull) expect[v] = expect[v] + a0[v] * g0[v];
  }
  backward_rows<V, LOG_LC>(a, L, t, column, xs, gs, expect, envs, tiles);
  if (kNull && L.p == 0 && L.live) {
    fvec<V> out;
#pragma unroll
    for (int v = 0; v < V; ++v) out.v[v] = a0[v] * (g0[v] - expect[v]);
    store_vec<V>(a.grad_null_logit + segment * a.channels + L.column, out);
  }
}

template <int V, int LOG_LC, bool kNull, bool kOrdered, bool kPlanned>
__global__ __launch_bounds__(kBlock) void softmax_backward_kernel(BackwardArgs a, const int64_t* __restrict__ plan,
                                                                  int64_t n_long) {
  using S = Geo<V, LOG_LC, true>;
  __shared__ float partial[kWaves][2][S::LC * V];
  constexpr bool planned = kPlanned;
  const int64_t block = block_index();
  if (planned && block < n_long) {
    const int64_t segment = plan[kPlanHeader + block];
    if (static_cast<uint64_t>(segment) >= static_cast<uint64_t>(a.n_nodes)) return;
    int64_t begin, end;
    segment_bounds(a.offsets, segment, a.n_edges, begin, end);
    backward_long<V, LOG_LC, kNull, kOrdered>(a, segment, begin, end, partial);
    return;
  }
  const int64_t first = (block - (planned ? n_long : 0)) * S::SPB;
  const int gidx = threadIdx.x >> S::LOG_G;
  const int64_t segment = first + gidx;
  {
    int64_t begin, end;
    group_bounds<S::LOG_G>(a.offsets, first, a.n_nodes, a.n_edges, begin, end);
    // The rows of a wave's short groups (at most two) lie within 2 CAP slots
    // of the lowest short group's begin: one buffer window serves the wave.
    static_assert(S::GPW <= 2, "one row window per wave needs at most two short groups per wave");
    if (segment < a.n_nodes && end - begin <= S::CAP)
      backward_short<V, LOG_LC, kNull, kOrdered>(a, segment, begin, end, uniform_i64(begin));
  }
  if constexpr (planned) return;
  const BlockBounds bb = block_bounds<S::SPB>(a.offsets, first, a.n_nodes, a.n_edges);
  const int lane = threadIdx.x & 63;
  unsigned long long longs =
      __ballot(lane < S::SPB && first + lane < a.n_nodes && bb.hi - bb.lo > S::CAP);
  while (longs != 0ull) {
    const int s = __ffsll(static_cast<long long>(longs)) - 1;
    longs &= longs - 1ull;
    backward_long<V, LOG_LC, kNull, kOrdered>(a, first + s, __shfl(bb.lo, s), __shfl(bb.hi, s), partial);
  }
}

// ---------------------------------------------------------------------------
// rows wider than 64 chunks: one wave per segment, lane per channel
// ---------------------------------------------------------------------------

template <bool kOrdered>
__global__ __launch_bounds__(kBlock) void softmax_forward_wide_kernel(ForwardArgs a) {
  const int64_t segment = block_index() * kWaves + (threadIdx.x >> 6);
  if (segment >= a.n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int64_t channels = a.channels;
  int64_t begin, end;
  segment_bounds(a.offsets, segment, a.n_edges, begin, end);
  for (int64_t c = lane; c < channels; c += 64) {
    float peak = -INFINITY, sum = 0.0f, carry = 0.0f;
    for (int64_t slot = begin; slot < end; ++slot) {
      const int64_t e = edge_of<kOrdered>(a.order, slot, a.n_edges);
      if (e >= 0) online_add(peak, sum, carry, log2_weight(a.logit[e * channels + c], a.env[e]));
    }
    float null_value = -INFINITY;
    if (a.null_logit != nullptr) {
      null_value = a.null_logit[segment * channels + c] * kLog2e;
      online_add(peak, sum, carry, null_value);
    }
    const float inverse = inverse_total(sum + carry);
    for (int64_t slot = begin; slot < end; ++slot) {
      const int64_t e = edge_of<kOrdered>(a.order, slot, a.n_edges);
      if (e < 0) continue;
      a.alpha[e * channels + c] = weight_of(log2_weight(a.logit[e * channels + c], a.env[e]), peak) * inverse;
    }
    if (a.null_logit != nullptr) a.null_alpha[segment * channels + c] = weight_of(null_value, peak) * inverse;
  }
}

template <bool kOrdered>
__global__ __launch_bounds__(kBlock) void softmax_backward_wide_kernel(BackwardArgs a) {
  const int64_t segment = block_index() * kWaves + (threadIdx.x >> 6);
  if (segment >= a.n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int64_t channels = a.channels;
  int64_t begin, end;
  segment_bounds(a.offsets, segment, a.n_edges, begin, end);
  const bool has_null = a.null_alpha != nullptr;
  // Channel windows of 64 lanes; grad_env keeps the raw channel sum until the
  // last window, which applies the 2 / env factor.
  for (int64_t base = 0; base < channels; base += 64) {
    const int64_t c = base + lane;
    const bool live = c < channels;
    const bool last = base + 64 >= channels;
    float expect = 0.0f, carry = 0.0f;
    if (live)
      for (int64_t slot = begin; slot < end; ++slot) {
        const int64_t e = edge_of<kOrdered>(a.order, slot, a.n_edges);
        if (e >= 0) compensated_add(expect, carry, a.alpha[e * channels + c] * a.grad_alpha[e * channels + c]);
      }
    if (has_null && live)
      compensated_add(expect, carry, a.null_alpha[segment * channels + c] * a.grad_null_alpha[segment * channels + c]);
    expect = expect + carry;
    for (int64_t slot = begin; slot < end; ++slot) {
      const int64_t e = edge_of<kOrdered>(a.order, slot, a.n_edges);
      if (e < 0) continue;
      float out = 0.0f;
      if (live) {
        out = a.alpha[e * channels + c] * (a.grad_alpha[e * channels + c] - expect);
        a.grad_logit[e * channels + c] = out;
      }
      float row = group_sum<64>(out);
      if (lane == 0) {
        if (base > 0) row = a.grad_env[e] + row;
        a.grad_env[e] = last ? env_gradient(row, a.env[e]) : row;
      }
    }
    if (has_null && live)
      a.grad_null_logit[segment * channels + c] =
          a.null_alpha[segment * channels + c] * (a.grad_null_alpha[segment * channels + c] - expect);
  }
}

// ---------------------------------------------------------------------------
// plan: ascending list of the segments longer than the short-path capacity
// ---------------------------------------------------------------------------

constexpr int kPlanThreads = 256;
constexpr int kPlanItems = 16;
constexpr int64_t kPlanTile = kPlanThreads * kPlanItems;

__device__ __forceinline__ bool is_long(const int64_t* __restrict__ offsets, int64_t segment, int64_t n_edges,
                                        int64_t capacity) {
  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  return end - begin > capacity;
}

__device__ int64_t plan_block_scan(int64_t value, int64_t* lds) {
  const int t = threadIdx.x;
  lds[t] = value;
  __syncthreads();
  for (int offset = 1; offset < kPlanThreads; offset <<= 1) {
    const int64_t add = t >= offset ? lds[t - offset] : 0;
    __syncthreads();
    lds[t] += add;
    __syncthreads();
  }
  const int64_t result = lds[t];
  __syncthreads();
  return result;
}

__global__ __launch_bounds__(kPlanThreads) void plan_count_kernel(const int64_t* __restrict__ offsets,
                                                                  int64_t n_nodes, int64_t n_edges,
                                                                  int64_t capacity, int64_t* __restrict__ counts) {
  __shared__ int64_t lds[kPlanThreads];
  const int64_t tile = block_index();
  if (tile * kPlanTile >= n_nodes) return;
  const int64_t base = tile * kPlanTile + static_cast<int64_t>(threadIdx.x) * kPlanItems;
  int64_t count = 0;
  for (int i = 0; i < kPlanItems; ++i)
    if (base + i < n_nodes && is_long(offsets, base + i, n_edges, capacity)) ++count;
  const int64_t inclusive = plan_block_scan(count, lds);
  if (threadIdx.x == kPlanThreads - 1) counts[tile] = inclusive;
}

// Exclusive scan of the tile counts in place (one workgroup); writes the
// header of the plan.
__global__ __launch_bounds__(kPlanThreads) void plan_scan_kernel(int64_t* __restrict__ counts, int64_t tiles,
                                                                 int64_t capacity, int64_t* __restrict__ plan) {
  __shared__ int64_t lds[kPlanThreads];
  const int64_t per_thread = (tiles + kPlanThreads - 1) / kPlanThreads;
  const int64_t begin = static_cast<int64_t>(threadIdx.x) * per_thread;
  const int64_t end = begin + per_thread < tiles ? begin + per_thread : tiles;
  int64_t sum = 0;
  for (int64_t i = begin; i < end; ++i) sum += counts[i];
  const int64_t inclusive = plan_block_scan(sum, lds);
  int64_t running = inclusive - sum;
  for (int64_t i = begin; i < end; ++i) {
    const int64_t value = counts[i];
    counts[i] = running;
    running += value;
  }
  if (threadIdx.x == kPlanThreads - 1) {
    plan[0] = capacity;
    plan[1] = inclusive;
  }
}

__global__ __launch_bounds__(kPlanThreads) void plan_write_kernel(const int64_t* __restrict__ offsets,
                                                                  int64_t n_nodes, int64_t n_edges,
                                                                  int64_t capacity,
                                                                  const int64_t* __restrict__ tile_prefix,
                                                                  int64_t* __restrict__ list) {
  __shared__ int64_t lds[kPlanThreads];
  const int64_t tile = block_index();
  if (tile * kPlanTile >= n_nodes) return;
  const int64_t base = tile * kPlanTile + static_cast<int64_t>(threadIdx.x) * kPlanItems;
  bool flag[kPlanItems];
  int64_t count = 0;
#pragma unroll
  for (int i = 0; i < kPlanItems; ++i) {
    flag[i] = base + i < n_nodes && is_long(offsets, base + i, n_edges, capacity);
    count += flag[i] ? 1 : 0;
  }
  const int64_t inclusive = plan_block_scan(count, lds);
  int64_t position = tile_prefix[tile] + inclusive - count;
#pragma unroll
  for (int i = 0; i < kPlanItems; ++i)
    if (flag[i]) list[position++] = base + i;
}

int64_t plan_tiles(int64_t n_nodes) { return (n_nodes + kPlanTile - 1) / kPlanTile; }

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int lanes_log_for(int64_t chunks) {
  int log = 0;
  while ((int64_t(1) << log) < chunks) ++log;
  return log;
}

// Short-path capacity of the kernel that runs `channels` with (vec4) or
// without 128-bit rows; 0 for the channel-major kernel (no plan use).
int64_t capacity_for(int64_t channels, bool vec4) {
  const int64_t chunks = vec4 ? channels / 4 : channels;
  if (chunks > 64) return 0;
  return short_capacity(vec4 ? 4 : 1, 1 << lanes_log_for(chunks));
}

int64_t short_blocks(int64_t n_nodes, int v, int log_lc, bool backward) {
  const int64_t per_block = kBlock >> short_group_log(v, log_lc, backward);
  return (n_nodes + per_block - 1) / per_block;
}

template <int V, int LOG_LC>
int launch_forward(const ForwardArgs& a, const int64_t* plan, int64_t n_long, hipStream_t stream) {
  const dim3 grid = launch_grid((plan != nullptr ? n_long : 0) + short_blocks(a.n_nodes, V, LOG_LC, false), kBlock);
#define DPA4K_SOFTMAX_FWD(NULLV, ORD)                                                                      \
  (plan != nullptr                                                                                        \
       ? softmax_forward_kernel<V, LOG_LC, NULLV, ORD, true>                                               \
       : softmax_forward_kernel<V, LOG_LC, NULLV, ORD, false>)<<<grid, kBlock, 0, \
                                                                 stream>>>(a, plan, n_long)
  if (a.null_logit != nullptr) {
    if (a.order != nullptr) DPA4K_SOFTMAX_FWD(true, true); else DPA4K_SOFTMAX_FWD(true, false);
  } else {
    if (a.order != nullptr) DPA4K_SOFTMAX_FWD(false, true); else DPA4K_SOFTMAX_FWD(false, false);
  }
#undef DPA4K_SOFTMAX_FWD
  return launched("softmax_forward_kernel");
}

template <int V, int LOG_LC>
int launch_backward(const BackwardArgs& a, const int64_t* plan, int64_t n_long, hipStream_t stream) {
  const dim3 grid = launch_grid((plan != nullptr ? n_long : 0) + short_blocks(a.n_nodes, V, LOG_LC, true), kBlock);
#define DPA4K_SOFTMAX_BWD(NULLV, ORD)                                                                       \
  (plan != nullptr                                                                                         \
       ? softmax_backward_kernel<V, LOG_LC, NULLV, ORD, true>                                               \
       : softmax_backward_kernel<V, LOG_LC, NULLV, ORD, false>)<<<grid, kBlock, 0, \
                                                                  stream>>>(a, plan, n_long)
  if (a.null_alpha != nullptr) {
    if (a.order != nullptr) DPA4K_SOFTMAX_BWD(true, true); else DPA4K_SOFTMAX_BWD(true, false);
  } else {
    if (a.order != nullptr) DPA4K_SOFTMAX_BWD(false, true); else DPA4K_SOFTMAX_BWD(false, false);
  }
#undef DPA4K_SOFTMAX_BWD
  return launched("softmax_backward_kernel");
}

template <int V, typename Args>
int dispatch_forward(int log_lc, const Args& a, const int64_t* list, int64_t n_long, hipStream_t stream) {
  switch (log_lc) {
    case 0: return launch_forward<V, 0>(a, list, n_long, stream);
    case 1: return launch_forward<V, 1>(a, list, n_long, stream);
    case 2: return launch_forward<V, 2>(a, list, n_long, stream);
    case 3: return launch_forward<V, 3>(a, list, n_long, stream);
    case 4: return launch_forward<V, 4>(a, list, n_long, stream);
    case 5: return launch_forward<V, 5>(a, list, n_long, stream);
    default: return launch_forward<V, 6>(a, list, n_long, stream);
  }
}

template <int V, typename Args>
int dispatch_backward(int log_lc, const Args& a, const int64_t* list, int64_t n_long, hipStream_t stream) {
  switch (log_lc) {
    case 0: return launch_backward<V, 0>(a, list, n_long, stream);
    case 1: return launch_backward<V, 1>(a, list, n_long, stream);
    case 2: return launch_backward<V, 2>(a, list, n_long, stream);
    case 3: return launch_backward<V, 3>(a, list, n_long, stream);
    case 4: return launch_backward<V, 4>(a, list, n_long, stream);
    case 5: return launch_backward<V, 5>(a, list, n_long, stream);
    default: return launch_backward<V, 6>(a, list, n_long, stream);
  }
}

int check_common(int64_t n_edges, int64_t n_nodes, int64_t channels, const char* what) {
  if (n_edges < 0 || n_nodes < 0) return fail(DPA4K_EINVAL, "%s: negative sizes", what);
  if (channels <= 0) return fail(DPA4K_EINVAL, "%s requires at least one channel", what);
  if (!grid_fits(n_nodes, kBlock)) return fail(DPA4K_EINVAL, "%s: segment count too large", what);
  return DPA4K_OK;
}

int softmax_forward(const float* logit, const float* env, const int64_t* offsets, const float* null_logit,
                    const int64_t* order, float* alpha, float* null_alpha, int64_t n_edges, int64_t n_nodes,
                    int64_t channels, const void* plan, int64_t n_long, int64_t plan_capacity,
                    dpa4k_stream_t stream_handle) {
  if (int s = check_common(n_edges, n_nodes, channels, "segment softmax")) return s;
  if (plan != nullptr && (n_long < 0 || n_long > n_nodes))
    return fail(DPA4K_EINVAL, "segment softmax: n_long outside [0, n_nodes]");
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr || (n_edges > 0 && (logit == nullptr || env == nullptr || alpha == nullptr)))
    return fail(DPA4K_EINVAL, "segment softmax: null pointer");
  if ((null_logit == nullptr) != (null_alpha == nullptr))
    return fail(DPA4K_EINVAL, "segment softmax: null_logit and null_alpha go together");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(logit) && aligned16(alpha) &&
                    (null_logit == nullptr || (aligned16(null_logit) && aligned16(null_alpha)));
  const int64_t chunks = vec4 ? channels / 4 : channels;
  const ForwardArgs a{logit, env, offsets, null_logit, order, alpha, null_alpha, n_edges, n_nodes, channels};
  if (chunks > 64) {
    const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
    if (order != nullptr) softmax_forward_wide_kernel<true><<<grid, kBlock, 0, stream>>>(a);
    else softmax_forward_wide_kernel<false><<<grid, kBlock, 0, stream>>>(a);
    return launched("softmax_forward_wide_kernel");
  }
  // a plan applies only to the geometry it was built for; otherwise run unplanned
  const bool use_plan = plan != nullptr && plan_capacity == capacity_for(channels, vec4);
  const int64_t* words = use_plan ? static_cast<const int64_t*>(plan) : nullptr;
  const int log_lc = lanes_log_for(chunks);
  return vec4 ? dispatch_forward<4>(log_lc, a, words, use_plan ? n_long : 0, stream)
              : dispatch_forward<1>(log_lc, a, words, use_plan ? n_long : 0, stream);
}

int softmax_backward(const float* alpha, const float* grad_alpha, const float* env, const int64_t* offsets,
                     const float* null_alpha, const float* grad_null_alpha, const int64_t* order,
                     float* grad_logit, float* grad_null_logit, float* grad_env, int64_t n_edges,
                     int64_t n_nodes, int64_t channels, const void* plan, int64_t n_long,
                     int64_t plan_capacity, dpa4k_stream_t stream_handle) {
  if (int s = check_common(n_edges, n_nodes, channels, "segment softmax backward")) return s;
  if (plan != nullptr && (n_long < 0 || n_long > n_nodes))
    return fail(DPA4K_EINVAL, "segment softmax backward: n_long outside [0, n_nodes]");
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr ||
      (n_edges > 0 && (alpha == nullptr || grad_alpha == nullptr || env == nullptr ||
                       grad_logit == nullptr || grad_env == nullptr)))
    return fail(DPA4K_EINVAL, "segment softmax backward: null pointer");
  const bool has_null = null_alpha != nullptr;
  if (has_null != (grad_null_alpha != nullptr) || has_null != (grad_null_logit != nullptr))
    return fail(DPA4K_EINVAL, "segment softmax requires null_alpha and grad_null_alpha together");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(alpha) && aligned16(grad_alpha) && aligned16(grad_logit) &&
                    (!has_null || (aligned16(null_alpha) && aligned16(grad_null_alpha) &&
                                   aligned16(grad_null_logit)));
  const int64_t chunks = vec4 ? channels / 4 : channels;
  const BackwardArgs a{alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order,
                       grad_logit, grad_null_logit, grad_env, n_edges, n_nodes, channels};
  if (chunks > 64) {
    const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
    if (order != nullptr) softmax_backward_wide_kernel<true><<<grid, kBlock, 0, stream>>>(a);
    else softmax_backward_wide_kernel<false><<<grid, kBlock, 0, stream>>>(a);
    return launched("softmax_backward_wide_kernel");
  }
  const bool use_plan = plan != nullptr && plan_capacity == capacity_for(channels, vec4);
  const int64_t* words = use_plan ? static_cast<const int64_t*>(plan) : nullptr;
  const int log_lc = lanes_log_for(chunks);
  return vec4 ? dispatch_backward<4>(log_lc, a, words, use_plan ? n_long : 0, stream)
              : dispatch_backward<1>(log_lc, a, words, use_plan ? n_long : 0, stream);
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" int dpa4k_segment_softmax_forward(const float* logit, const float* env, const int64_t* offsets,
                                             const float* null_logit, const int64_t* order, float* alpha,
                                             float* null_alpha, int64_t n_edges, int64_t n_nodes,
                                             int64_t channels, dpa4k_stream_t stream) {
  clear_error();
  return softmax_forward(logit, env, offsets, null_logit, order, alpha, null_alpha, n_edges, n_nodes, channels,
                         nullptr, 0, 0, stream);
}

extern "C" int dpa4k_segment_softmax_backward(const float* alpha, const float* grad_alpha, const float* env,
                                              const int64_t* offsets, const float* null_alpha,
                                              const float* grad_null_alpha, const int64_t* order,
                                              float* grad_logit, float* grad_null_logit, float* grad_env,
                                              int64_t n_edges, int64_t n_nodes, int64_t channels,
                                              dpa4k_stream_t stream) {
  clear_error();
  return softmax_backward(alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order, grad_logit,
                          grad_null_logit, grad_env, n_edges, n_nodes, channels, nullptr, 0, 0, stream);
}

extern "C" size_t dpa4k_segment_softmax_plan_size(int64_t n_nodes) {
  if (n_nodes < 0) return 0;
  return round_up_256(static_cast<size_t>(kPlanHeader + n_nodes + plan_tiles(n_nodes)) * sizeof(int64_t));
}

extern "C" int dpa4k_segment_softmax_plan(const int64_t* offsets, int64_t n_edges, int64_t n_nodes,
                                          int64_t channels, void* plan, size_t plan_bytes, int64_t* n_long,
                                          int64_t* plan_capacity, dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_common(n_edges, n_nodes, channels, "segment softmax plan")) return s;
  if (offsets == nullptr || plan == nullptr || n_long == nullptr || plan_capacity == nullptr)
    return fail(DPA4K_EINVAL, "segment softmax plan: null pointer");
  if (plan_bytes < dpa4k_segment_softmax_plan_size(n_nodes))
    return fail(DPA4K_EWORKSPACE, "segment softmax plan: %zu bytes given, %zu needed", plan_bytes,
                dpa4k_segment_softmax_plan_size(n_nodes));
  hipStream_t stream = as_stream(stream_handle);
  // The plan is for the 128-bit row kernel when C % 4 == 0 (operands from
  // torch's allocator are 16-byte aligned), for the scalar one otherwise.
  const int64_t capacity = capacity_for(channels, channels % 4 == 0);
  int64_t* words = static_cast<int64_t*>(plan);
  const int64_t tiles = plan_tiles(n_nodes);
  int64_t* counts = words + kPlanHeader + n_nodes;
  if (tiles > 0) {
    plan_count_kernel<<<launch_grid(tiles, kPlanThreads), kPlanThreads, 0, stream>>>(offsets, n_nodes, n_edges,
                                                                                     capacity, counts);
    if (int s = launched("plan_count_kernel")) return s;
  }
  plan_scan_kernel<<<1, kPlanThreads, 0, stream>>>(counts, tiles, capacity, words);
  if (int s = launched("plan_scan_kernel")) return s;
  if (tiles > 0) {
    plan_write_kernel<<<launch_grid(tiles, kPlanThreads), kPlanThreads, 0, stream>>>(
        offsets, n_nodes, n_edges, capacity, counts, words + kPlanHeader);
    if (int s = launched("plan_write_kernel")) return s;
  }
  int64_t header[2] = {0, 0};
  if (int s = hip_status(hipMemcpyAsync(header, words, sizeof(header), hipMemcpyDeviceToHost, stream),
                         "hipMemcpyAsync(plan header)"))
    return s;
  if (int s = hip_status(hipStreamSynchronize(stream), "hipStreamSynchronize")) return s;
  *n_long = header[1];
  *plan_capacity = header[0];
  return DPA4K_OK;
}

extern "C" int dpa4k_segment_softmax_forward_planned(const float* logit, const float* env, const int64_t* offsets,
                                                     const float* null_logit, const int64_t* order, float* alpha,
                                                     float* null_alpha, int64_t n_edges, int64_t n_nodes,
                                                     int64_t channels, const void* plan, int64_t n_long,
                                                     int64_t plan_capacity, dpa4k_stream_t stream) {
  clear_error();
  return softmax_forward(logit, env, offsets, null_logit, order, alpha, null_alpha, n_edges, n_nodes, channels,
                         plan, n_long, plan_capacity, stream);
}

extern "C" int dpa4k_segment_softmax_backward_planned(const float* alpha, const float* grad_alpha, const float* env,
                                                      const int64_t* offsets, const float* null_alpha,
                                                      const float* grad_null_alpha, const int64_t* order,
                                                      float* grad_logit, float* grad_null_logit, float* grad_env,
                                                      int64_t n_edges, int64_t n_nodes, int64_t channels,
                                                      const void* plan, int64_t n_long, int64_t plan_capacity,
                                                      dpa4k_stream_t stream) {
  clear_error();
  return softmax_backward(alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order, grad_logit,
                          grad_null_logit, grad_env, n_edges, n_nodes, channels, plan, n_long, plan_capacity,
                          stream);
}

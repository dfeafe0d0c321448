// segment_sum forward and backward (python/kernels/segment.py:196-230,
// csrc/segment_sum.cpp:214-317 of the reference).
//
// Layout: a lane group of G lanes owns one destination segment; lane l of
// the group owns the float4 (or float) channel chunks l, l + G, ... of the
// row.  The group walks the segment's CSR slots in order, so every output
// element is accumulated sequentially in slot order with the product rounded
// before the add -- the same arithmetic as `index_add_` on the CPU, hence a
// bit-exact match with the sequential fp32 chain (the library is built with
// -ffp-contract=off).  256-thread blocks hold 256 / G segments; rows of
// C = 128 floats give G = 32 (two segments per wave, one 512-byte row per
// half wave per load), C >= 256 gives one segment per wave with several
// chunks per lane.
//
// Backward is segment-parallel too: a workgroup (rows of 64 to 256 floats)
// or a lane group loads grad_out[n] once, writes grad_src for every edge of
// the segment, and reduces the per-edge channel dot product (grad_edge_scale,
// and summed over the segment grad_node_scale) with a fixed butterfly.  The reference's edge-parallel grad_src kernel
// needs `dst`; here the CSR names each edge's segment, which the grouping
// contract makes identical.  Grids too small to fill the chip (few segments)
// keep up to 32 rows per lane in flight.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;

template <int V, int G, int CPL, int U, bool kScaleEdge, bool kOrdered>
__global__ __launch_bounds__(kBlock) void segment_sum_forward_kernel(
    const float* __restrict__ src, const int64_t* __restrict__ offsets,
    const float* __restrict__ edge_scale, const float* __restrict__ node_scale,
    const int64_t* __restrict__ order, float* __restrict__ out, int64_t n_edges, int64_t n_nodes,
    int64_t channels, int64_t chunk_base) {
  constexpr int kSegments = kBlock / G;
  const int64_t segment = block_index() * kSegments + threadIdx.x / G;
  if (segment >= n_nodes) return;
  const int lane = threadIdx.x % G;
  const int64_t chunks = channels / V;

  int64_t column[CPL];
  bool live[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t chunk = chunk_base + lane + static_cast<int64_t>(G) * j;
    live[j] = chunk < chunks;
    column[j] = chunk * V;
  }

  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);

  fvec<V> acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[j].v[i] = 0.0f;

  // U slots per round, all loads of a round issued before any add; the adds
  // then run in slot order, so each element is a sequential sum.  Rows are
  // read once and loaded non-temporally, which keeps the lines of the order
  // and of the gathered edge scales cached for the neighbouring slots.
  for (int64_t slot = begin; slot < end; slot += U) {
    int64_t edge[U];
    float weight[U];
    fvec<V> x[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
      edge[u] = slot + u < end ? edge_of<kOrdered>(order, slot + u, n_edges) : -1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = edge[u] >= 0;
      weight[u] = kScaleEdge && ok ? edge_scale[edge[u]] : 1.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (live[j] && ok) {
          x[u][j] = load_vec_stream<V>(src + edge[u] * channels + column[j]);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) x[u][j].v[i] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (edge[u] < 0) continue;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i)
          acc[j].v[i] = acc[j].v[i] + (kScaleEdge ? x[u][j].v[i] * weight[u] : x[u][j].v[i]);
    }
  }

  const bool scaled = node_scale != nullptr;
  const float scale = scaled ? node_scale[segment] : 1.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    if (!live[j]) continue;
    fvec<V> result;
#pragma unroll
    for (int i = 0; i < V; ++i) result.v[i] = scaled ? acc[j].v[i] * scale : acc[j].v[i];
    store_vec<V>(out + segment * channels + column[j], result);
  }
}

// With g = grad_out[n], s = node_scale[n], w = edge_scale[e] and the raw
// channel dot d_e = sum_c g[c] * src[e, c]:
//   grad_src[e]        = (g * s) * w
//   grad_edge_scale[e] = s * d_e
//   grad_node_scale[n] = sum_e w * d_e
// (the reference recomputes the prefix sum_e w src[e] for the node-scale
// gradient; the per-edge dots give the same sum without it).  Each edge row
// is read once; U edges per round are loaded before any arithmetic.
// `accumulate` adds the partial dots of this channel window to the values
// written by the previous window (channels wider than one window).
template <int V, int G, int CPL, int U, bool kOrdered>
__global__ __launch_bounds__(kBlock) void segment_sum_backward_kernel(
    const float* __restrict__ grad_out, const float* __restrict__ src,
    const int64_t* __restrict__ offsets, const float* __restrict__ edge_scale,
    const float* __restrict__ node_scale, const int64_t* __restrict__ order,
    float* __restrict__ grad_src, float* __restrict__ grad_edge_scale,
    float* __restrict__ grad_node_scale, int64_t n_edges, int64_t n_nodes, int64_t channels,
    int64_t chunk_base, int accumulate) {
  constexpr int kSegments = kBlock / G;
  const int64_t segment = block_index() * kSegments + threadIdx.x / G;
  if (segment >= n_nodes) return;
  const int lane = threadIdx.x % G;
  const int64_t chunks = channels / V;
  const bool want_edge = grad_edge_scale != nullptr;
  const bool want_node = grad_node_scale != nullptr;
  const bool need_dot = want_edge || want_node;
  const bool has_edge_scale = edge_scale != nullptr;

  int64_t column[CPL];
  bool live[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t chunk = chunk_base + lane + static_cast<int64_t>(G) * j;
    live[j] = chunk < chunks;
    column[j] = chunk * V;
  }

  const float scale = node_scale != nullptr ? node_scale[segment] : 1.0f;
  fvec<V> g[CPL], gs[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    if (live[j]) {
      g[j] = load_vec<V>(grad_out + segment * channels + column[j]);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) g[j].v[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) gs[j].v[i] = node_scale != nullptr ? g[j].v[i] * scale : g[j].v[i];
  }

  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  float node_sum = 0.0f;
  for (int64_t slot = begin; slot < end; slot += U) {
    int64_t edge[U];
    float weight[U], dot[U];
    fvec<V> x[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
      edge[u] = slot + u < end ? edge_of<kOrdered>(order, slot + u, n_edges) : -1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      weight[u] = has_edge_scale && edge[u] >= 0 ? edge_scale[edge[u]] : 1.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (need_dot && live[j] && edge[u] >= 0) {
          x[u][j] = load_vec<V>(src + edge[u] * channels + column[j]);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) x[u][j].v[i] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (edge[u] < 0) continue;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (!live[j]) continue;
        fvec<V> out;
#pragma unroll
        for (int i = 0; i < V; ++i) out.v[i] = has_edge_scale ? gs[j].v[i] * weight[u] : gs[j].v[i];
        store_vec_stream<V>(grad_src + edge[u] * channels + column[j], out);
      }
    }
    if (need_dot) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
          for (int i = 0; i < V; ++i) d = d + g[j].v[i] * x[u][j].v[i];
        dot[u] = group_sum<G>(d);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (edge[u] < 0) continue;
        if (want_edge && lane == 0) {
          const float value = scale * dot[u];
          grad_edge_scale[edge[u]] = accumulate ? grad_edge_scale[edge[u]] + value : value;
        }
        node_sum = node_sum + weight[u] * dot[u];
      }
    }
  }
  if (want_node && lane == 0)
    grad_node_scale[segment] = accumulate ? grad_node_scale[segment] + node_sum : node_sum;
}

// ---------------------------------------------------------------------------
// Small grids: one segment per workgroup
// ---------------------------------------------------------------------------
//
// With few segments (config 1: 1,024 segments of ~40 rows of 128 floats) the
// lane-group kernels above leave the chip mostly empty and walk a segment in
// several dependent memory round trips.  These kernels give each segment a
// whole 256-thread workgroup instead.

constexpr int kStageChunks = 2048;  // float4 chunks of LDS staging (32 KB)
constexpr int kStageItems = kStageChunks / kBlock;

// Forward: the workgroup loads up to kStageChunks / chunks rows of the
// segment into LDS at once (every thread's loads in flight together), then
// thread c < channels sums column c of the staged rows in slot order, eight
// rows of LDS reads ahead of its adds -- the same sequential fp32 sum as the
// lane-group kernel, so the result is bit-identical.  Longer segments repeat
// the load/sum step.  Rows of 16 to 64 chunks (64 to 256 floats).
template <bool kScaleEdge, bool kOrdered>
__global__ __launch_bounds__(kBlock) void segment_sum_staged_kernel(
    const float* __restrict__ src, const int64_t* __restrict__ offsets,
    const float* __restrict__ edge_scale, const float* __restrict__ node_scale,
    const int64_t* __restrict__ order, float* __restrict__ out, int64_t n_edges, int64_t n_nodes,
    int64_t channels) {
  constexpr int kAhead = 8;
  __shared__ fvec<4> stage[kStageChunks];
  __shared__ float weight[kStageChunks / 16 + kAhead];  // rows per batch (chunks >= 16), padded
  __shared__ unsigned char skip[kStageChunks / 16 + kAhead];  // 1: the row's order entry is out of range
  const int64_t segment = block_index();
  if (segment >= n_nodes) return;
  const int chunks = static_cast<int>(channels / 4);
  const int width = chunks * 4;
  const int rows_per_batch = kStageChunks / chunks;
  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  const int t = threadIdx.x;
  const float* staged = reinterpret_cast<const float*>(stage);
  float acc = 0.0f;

  for (int64_t first = begin; first < end; first += rows_per_batch) {
    const int rows = static_cast<int>(end - first < rows_per_batch ? end - first : rows_per_batch);
    const int items = rows * chunks;
    fvec<4> x[kStageItems];
#pragma unroll
    for (int k = 0; k < kStageItems; ++k) {
      const int item = t + k * kBlock;
      const int row = item / chunks;
      const int64_t e = item < items ? edge_of<kOrdered>(order, first + row, n_edges) : -1;
      if (e >= 0) {  // rows are read once: non-temporal (config 1: 7.6 -> 7.25 us)
        x[k] = load_vec_stream<4>(src + e * channels + static_cast<int64_t>(item - row * chunks) * 4);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) x[k].v[i] = 0.0f;
      }
    }
    // weight of each staged row, and whether it is skipped (order entry out of range); the
    // flag lives apart from the weight so that a NaN edge_scale still propagates into the sum
    for (int row = t; row < rows; row += kBlock) {
      const int64_t e = edge_of<kOrdered>(order, first + row, n_edges);
      weight[row] = e < 0 ? 0.0f : (kScaleEdge ? edge_scale[e] : 1.0f);
      skip[row] = e < 0 ? 1 : 0;
    }
#pragma unroll
    for (int k = 0; k < kStageItems; ++k)
      if (t + k * kBlock < items) stage[t + k * kBlock] = x[k];
    __syncthreads();
    if (t < width) {
      for (int row = 0; row < rows; row += kAhead) {
        float v[kAhead], w[kAhead];
        bool dropped[kAhead];
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
          const int r = row + k < rows ? row + k : row;
          v[k] = staged[r * width + t];
          w[k] = weight[r];
          dropped[k] = kOrdered && skip[r] != 0;
        }
#pragma unroll
        for (int k = 0; k < kAhead; ++k) {
          if (row + k >= rows || dropped[k]) continue;
          acc = acc + (kScaleEdge ? v[k] * w[k] : v[k]);
        }
      }
    }
    __syncthreads();
  }
  if (t < width) out[segment * channels + t] = node_scale != nullptr ? acc * node_scale[segment] : acc;
}

// Backward: SG = 256 / G lane groups of G lanes (G >= chunks) take the
// segment's rows round-robin, U rows per group per round with every load of
// a round issued first.  grad_edge_scale is per edge; the groups' partial
// grad_node_scale sums meet in LDS in group order.  Rows of at most 64 chunks.
// kStreamRows loads the rows non-temporally (small grids, see the launcher).
template <int G, int U, bool kOrdered, bool kStreamRows>
__global__ __launch_bounds__(kBlock) void segment_sum_backward_wide_kernel(
    const float* __restrict__ grad_out, const float* __restrict__ src,
    const int64_t* __restrict__ offsets, const float* __restrict__ edge_scale,
    const float* __restrict__ node_scale, const int64_t* __restrict__ order,
    float* __restrict__ grad_src, float* __restrict__ grad_edge_scale,
    float* __restrict__ grad_node_scale, int64_t n_edges, int64_t n_nodes, int64_t channels) {
  constexpr int SG = kBlock / G;
  __shared__ float partial[SG];
  const int64_t segment = block_index();
  if (segment >= n_nodes) return;
  const int lane = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int chunks = static_cast<int>(channels / 4);
  const bool live = lane < chunks;
  const int64_t column = static_cast<int64_t>(live ? lane : 0) * 4;
  const bool want_edge = grad_edge_scale != nullptr;
  const bool want_node = grad_node_scale != nullptr;
  const bool need_dot = want_edge || want_node;
  const bool has_edge_scale = edge_scale != nullptr;

  const float scale = node_scale != nullptr ? node_scale[segment] : 1.0f;
  fvec<4> g, gs;
  if (live) {
    g = load_vec<4>(grad_out + segment * channels + column);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) g.v[i] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) gs.v[i] = node_scale != nullptr ? g.v[i] * scale : g.v[i];

  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  float node_sum = 0.0f;
  for (int64_t base = begin + group; base < end; base += static_cast<int64_t>(SG) * U) {
    int64_t edge[U];
    float weight[U];
    fvec<4> x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t slot = base + static_cast<int64_t>(u) * SG;
      edge[u] = slot < end ? edge_of<kOrdered>(order, slot, n_edges) : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      weight[u] = has_edge_scale && edge[u] >= 0 ? edge_scale[edge[u]] : 1.0f;
      if (need_dot && live && edge[u] >= 0) {
        x[u] = kStreamRows ? load_vec_stream<4>(src + edge[u] * channels + column)
                           : load_vec<4>(src + edge[u] * channels + column);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) x[u].v[i] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (edge[u] < 0 || !live) continue;
      fvec<4> o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o.v[i] = has_edge_scale ? gs.v[i] * weight[u] : gs.v[i];
      store_vec_stream<4>(grad_src + edge[u] * channels + column, o);
    }
    if (need_dot) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) d = d + g.v[i] * x[u].v[i];
        d = group_sum<G>(d);
        if (edge[u] < 0) continue;
        if (want_edge && lane == 0) grad_edge_scale[edge[u]] = scale * d;
        node_sum = node_sum + weight[u] * d;
      }
    }
  }
  if (want_node) {
    if (lane == 0) partial[group] = node_sum;
    __syncthreads();
    if (threadIdx.x == 0) {
      float total = partial[0];
      for (int q = 1; q < SG; ++q) total = total + partial[q];
      grad_node_scale[segment] = total;
    }
  }
}

int launch_staged_forward(const float* src, const int64_t* offsets, const float* edge_scale,
                          const float* node_scale, const int64_t* order, float* out, int64_t n_edges,
                          int64_t n_nodes, int64_t channels, hipStream_t stream) {
  const dim3 grid = launch_grid(n_nodes, kBlock);
#define DPA4K_SUM_STAGED(SCALE, ORD)                                                                  \
  segment_sum_staged_kernel<SCALE, ORD><<<grid, kBlock, 0, stream>>>(src, offsets, edge_scale, node_scale, \
                                                                      order, out, n_edges, n_nodes, channels)
  if (edge_scale != nullptr) {
    if (order != nullptr) DPA4K_SUM_STAGED(true, true); else DPA4K_SUM_STAGED(true, false);
  } else {
    if (order != nullptr) DPA4K_SUM_STAGED(false, true); else DPA4K_SUM_STAGED(false, false);
  }
#undef DPA4K_SUM_STAGED
  return launched("segment_sum_staged_kernel");
}

template <int G>
int launch_wide_backward_g(const float* grad_out, const float* src, const int64_t* offsets,
                           const float* edge_scale, const float* node_scale, const int64_t* order,
                           float* grad_src, float* grad_edge_scale, float* grad_node_scale, int64_t n_edges,
                           int64_t n_nodes, int64_t channels, hipStream_t stream) {
  constexpr int U = 8;
  const dim3 grid = launch_grid(n_nodes, kBlock);
  // Non-temporal row loads pay on small grids (config 1: 11.4 -> 10.6-10.9 us) and not on large ones
  // (config 1R: 1,846 -> 1,886-1,903 us), measured on one box.
  const bool stream_rows = n_nodes < 4096;
#define DPA4K_SUM_BWD_WIDE(ORD, NT)                                                                    \
  segment_sum_backward_wide_kernel<G, U, ORD, NT><<<grid, kBlock, 0, stream>>>(                         \
      grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale, grad_node_scale, \
      n_edges, n_nodes, channels)
  if (order != nullptr) {
    if (stream_rows) DPA4K_SUM_BWD_WIDE(true, true); else DPA4K_SUM_BWD_WIDE(true, false);
  } else {
    if (stream_rows) DPA4K_SUM_BWD_WIDE(false, true); else DPA4K_SUM_BWD_WIDE(false, false);
  }
#undef DPA4K_SUM_BWD_WIDE
  return launched("segment_sum_backward_wide_kernel");
}

int launch_wide_backward(const float* grad_out, const float* src, const int64_t* offsets, const float* edge_scale,
                         const float* node_scale, const int64_t* order, float* grad_src, float* grad_edge_scale,
                         float* grad_node_scale, int64_t n_edges, int64_t n_nodes, int64_t channels,
                         hipStream_t stream) {
  const int64_t chunks = channels / 4;
  if (chunks <= 16)
    return launch_wide_backward_g<16>(grad_out, src, offsets, edge_scale, node_scale, order, grad_src,
                                      grad_edge_scale, grad_node_scale, n_edges, n_nodes, channels, stream);
  if (chunks <= 32)
    return launch_wide_backward_g<32>(grad_out, src, offsets, edge_scale, node_scale, order, grad_src,
                                      grad_edge_scale, grad_node_scale, n_edges, n_nodes, channels, stream);
  return launch_wide_backward_g<64>(grad_out, src, offsets, edge_scale, node_scale, order, grad_src,
                                    grad_edge_scale, grad_node_scale, n_edges, n_nodes, channels, stream);
}

// The workgroup-per-segment kernels take float4 rows of 16 to 64 chunks (64
// to 256 channels).  The forward uses its staged kernel on grids of fewer
// than kWideSegments segments; on larger grids the lane-group kernel's
// several rows in flight per lane stream faster (config 1R: 1.03 ms against
// 1.07-1.17 ms).  The backward uses its workgroup kernel on every grid
// (config 1R: 1.75 ms against 2.15 ms for the lane-group kernel).
constexpr int64_t kWideSegments = 4096;
bool wide_rows(int64_t chunks) { return chunks >= 16 && chunks <= 64; }
bool use_wide_forward(int64_t n_nodes, int64_t chunks) { return n_nodes < kWideSegments && wide_rows(chunks); }
bool use_wide_backward(int64_t chunks) { return wide_rows(chunks); }

// Lane-group geometry for a row of `chunks` vector chunks.
struct Geometry {
  int group;   // lanes per segment (power of two, <= 64)
  int per_lane;  // chunks per lane (1, 2, 4 or 8)
  int64_t window() const { return static_cast<int64_t>(group) * per_lane; }
};

Geometry geometry_for(int64_t chunks) {
  Geometry g{1, 1};
  while (g.group < 64 && g.group < chunks) g.group <<= 1;
  if (g.group == 64) {
    const int64_t need = (chunks + 63) / 64;
    while (g.per_lane < 8 && g.per_lane < need) g.per_lane <<= 1;
  }
  return g;
}

// Slots per round: about 32 loaded floats per lane, or 128 when the grid is
// too small to fill the chip (then each lane must keep more bytes in flight).
template <int V, int CPL>
constexpr int unroll_for(bool small_grid) {
  return small_grid ? (CPL * V >= 8 ? 16 : 32) : (CPL * V >= 16 ? 2 : (CPL * V >= 8 ? 4 : 8));
}

template <int V, int G, int CPL, int U>
int launch_forward_u(const float* src, const int64_t* offsets, const float* edge_scale,
                     const float* node_scale, const int64_t* order, float* out, int64_t n_edges,
                     int64_t n_nodes, int64_t channels, int64_t chunk_base, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kBlock / G - 1) / (kBlock / G), kBlock);
#define DPA4K_SUM_FWD(SCALE, ORD)                                                                     \
  segment_sum_forward_kernel<V, G, CPL, U, SCALE, ORD><<<grid, kBlock, 0, stream>>>(                \
      src, offsets, edge_scale, node_scale, order, out, n_edges, n_nodes, channels, chunk_base)
  if (edge_scale != nullptr) {
    if (order != nullptr) DPA4K_SUM_FWD(true, true); else DPA4K_SUM_FWD(true, false);
  } else {
    if (order != nullptr) DPA4K_SUM_FWD(false, true); else DPA4K_SUM_FWD(false, false);
  }
#undef DPA4K_SUM_FWD
  return launched("segment_sum_forward_kernel");
}

// A grid of fewer waves than the chip holds at once (256 CUs x 8 waves).
bool small_grid(int64_t n_nodes, int group) { return n_nodes * group / 64 < 2048; }

// Forward rounds over segments read in natural order with narrow rows (fewer
// than 8 loaded floats per lane a slot): 32 slots a round, so each lane group
// reads most of its segment in one burst.  Fewer, longer streams run faster
// from HBM than more, shorter ones at the same bytes in flight (config 1R,
// C = 128: 954 us against 1022 us with 8 slots, at 2 waves per SIMD against
// 4); rows named by `order` are scattered, and there the occupancy wins
// (1184 us with 8 slots against 1594 us with 32; 4 slots, below, better still).
template <int V, int CPL>
constexpr int contiguous_unroll_for() {
  return CPL * V >= 8 ? unroll_for<V, CPL>(false) : 32;
}

// Rows gathered through an order, narrow rows: 4 slots a round (config 1R
// with scales through a shuffled order: 1,117 us against 1,135 us with 8 and
// 1,228 us with 16).
template <int V, int CPL>
constexpr int ordered_unroll_for() {
  return CPL * V >= 8 ? unroll_for<V, CPL>(false) : 4;
}

template <int V, int G, int CPL>
int launch_forward(const float* src, const int64_t* offsets, const float* edge_scale,
                   const float* node_scale, const int64_t* order, float* out, int64_t n_edges,
                   int64_t n_nodes, int64_t channels, int64_t chunk_base, hipStream_t stream) {
  if (small_grid(n_nodes, G))
    return launch_forward_u<V, G, CPL, unroll_for<V, CPL>(true)>(src, offsets, edge_scale, node_scale, order,
                                                                 out, n_edges, n_nodes, channels, chunk_base,
                                                                 stream);
  if (order == nullptr)
    return launch_forward_u<V, G, CPL, contiguous_unroll_for<V, CPL>()>(src, offsets, edge_scale, node_scale,
                                                                        order, out, n_edges, n_nodes, channels,
                                                                        chunk_base, stream);
  return launch_forward_u<V, G, CPL, ordered_unroll_for<V, CPL>()>(src, offsets, edge_scale, node_scale, order, out,
                                                                   n_edges, n_nodes, channels, chunk_base, stream);
}

template <int V, int G, int CPL, int U>
int launch_backward_u(const float* grad_out, const float* src, const int64_t* offsets,
                      const float* edge_scale, const float* node_scale, const int64_t* order,
                      float* grad_src, float* grad_edge_scale, float* grad_node_scale,
                      int64_t n_edges, int64_t n_nodes, int64_t channels, int64_t chunk_base,
                      int accumulate, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kBlock / G - 1) / (kBlock / G), kBlock);
  if (order != nullptr)
    segment_sum_backward_kernel<V, G, CPL, U, true><<<grid, kBlock, 0, stream>>>(
        grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale,
        grad_node_scale, n_edges, n_nodes, channels, chunk_base, accumulate);
  else
    segment_sum_backward_kernel<V, G, CPL, U, false><<<grid, kBlock, 0, stream>>>(
        grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale,
        grad_node_scale, n_edges, n_nodes, channels, chunk_base, accumulate);
  return launched("segment_sum_backward_kernel");
}

template <int V, int G, int CPL>
int launch_backward(const float* grad_out, const float* src, const int64_t* offsets,
                    const float* edge_scale, const float* node_scale, const int64_t* order,
                    float* grad_src, float* grad_edge_scale, float* grad_node_scale,
                    int64_t n_edges, int64_t n_nodes, int64_t channels, int64_t chunk_base,
                    int accumulate, hipStream_t stream) {
  // the backward holds its rows for the dot products: half the forward's depth
  if (small_grid(n_nodes, G))
    return launch_backward_u<V, G, CPL, unroll_for<V, CPL>(true) / 2>(
        grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale, grad_node_scale,
        n_edges, n_nodes, channels, chunk_base, accumulate, stream);
  return launch_backward_u<V, G, CPL, (unroll_for<V, CPL>(false) > 2 ? unroll_for<V, CPL>(false) / 2 : 2)>(
      grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale, grad_node_scale, n_edges,
      n_nodes, channels, chunk_base, accumulate, stream);
}

// Dispatches a launcher template over the (V, G, CPL) geometry.
template <int V, template <int, int, int> class Launcher, typename... Args>
int dispatch_geometry(const Geometry& geo, Args... args) {
  switch (geo.group) {
    case 1: return Launcher<V, 1, 1>::run(args...);
    case 2: return Launcher<V, 2, 1>::run(args...);
    case 4: return Launcher<V, 4, 1>::run(args...);
    case 8: return Launcher<V, 8, 1>::run(args...);
    case 16: return Launcher<V, 16, 1>::run(args...);
    case 32: return Launcher<V, 32, 1>::run(args...);
    default: break;
  }
  switch (geo.per_lane) {
    case 1: return Launcher<V, 64, 1>::run(args...);
    case 2: return Launcher<V, 64, 2>::run(args...);
    case 4: return Launcher<V, 64, 4>::run(args...);
    default: return Launcher<V, 64, 8>::run(args...);
  }
}

template <int V, int G, int CPL>
struct ForwardLauncher {
  template <typename... Args>
  static int run(Args... args) { return launch_forward<V, G, CPL>(args...); }
};

template <int V, int G, int CPL>
struct BackwardLauncher {
  template <typename... Args>
  static int run(Args... args) { return launch_backward<V, G, CPL>(args...); }
};

int check_common(int64_t n_edges, int64_t n_nodes, int64_t channels, const char* what) {
  if (n_edges < 0 || n_nodes < 0) return fail(DPA4K_EINVAL, "%s: negative sizes", what);
  if (channels <= 0) return fail(DPA4K_EINVAL, "%s requires at least one channel", what);
  if (!grid_fits(n_nodes, kBlock)) return fail(DPA4K_EINVAL, "%s: segment count too large", what);
  return DPA4K_OK;
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" int dpa4k_segment_sum_forward(const float* src, const int64_t* offsets,
                                         const float* edge_scale, const float* node_scale,
                                         const int64_t* order, float* out, int64_t n_edges,
                                         int64_t n_nodes, int64_t channels,
                                         dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_common(n_edges, n_nodes, channels, "segment sum")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr || out == nullptr || (n_edges > 0 && src == nullptr))
    return fail(DPA4K_EINVAL, "segment sum: null pointer");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(src) && aligned16(out);
  const int64_t chunks = vec4 ? channels / 4 : channels;
  if (vec4 && use_wide_forward(n_nodes, chunks))
    return launch_staged_forward(src, offsets, edge_scale, node_scale, order, out, n_edges, n_nodes, channels,
                                 stream);
  const Geometry geo = geometry_for(chunks);
  for (int64_t base = 0; base < chunks; base += geo.window()) {
    const int status =
        vec4 ? dispatch_geometry<4, ForwardLauncher>(geo, src, offsets, edge_scale, node_scale,
                                                     order, out, n_edges, n_nodes, channels, base,
                                                     stream)
             : dispatch_geometry<1, ForwardLauncher>(geo, src, offsets, edge_scale, node_scale,
                                                     order, out, n_edges, n_nodes, channels, base,
                                                     stream);
    if (status) return status;
  }
  return DPA4K_OK;
}

extern "C" int dpa4k_segment_sum_backward(const float* grad_out, const float* src,
                                          const int64_t* offsets, const float* edge_scale,
                                          const float* node_scale, const int64_t* order,
                                          float* grad_src, float* grad_edge_scale,
                                          float* grad_node_scale, int64_t n_edges, int64_t n_nodes,
                                          int64_t channels, dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_common(n_edges, n_nodes, channels, "segment sum backward")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr || grad_out == nullptr || (n_edges > 0 && grad_src == nullptr))
    return fail(DPA4K_EINVAL, "segment sum backward: null pointer");
  if ((grad_edge_scale != nullptr || grad_node_scale != nullptr) && n_edges > 0 && src == nullptr)
    return fail(DPA4K_EINVAL, "segment sum backward: scale gradients need src");
  if (grad_edge_scale != nullptr && edge_scale == nullptr)
    return fail(DPA4K_EINVAL, "segment sum backward: grad_edge_scale needs edge_scale");
  if (grad_node_scale != nullptr && node_scale == nullptr)
    return fail(DPA4K_EINVAL, "segment sum backward: grad_node_scale needs node_scale");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(grad_out) && aligned16(grad_src) &&
                    (src == nullptr || aligned16(src));
  const int64_t chunks = vec4 ? channels / 4 : channels;
  if (vec4 && use_wide_backward(chunks))
    return launch_wide_backward(grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale,
                                grad_node_scale, n_edges, n_nodes, channels, stream);
  const Geometry geo = geometry_for(chunks);
  int accumulate = 0;
  for (int64_t base = 0; base < chunks; base += geo.window()) {
    const int status =
        vec4 ? dispatch_geometry<4, BackwardLauncher>(
                   geo, grad_out, src, offsets, edge_scale, node_scale, order, grad_src,
                   grad_edge_scale, grad_node_scale, n_edges, n_nodes, channels, base, accumulate,
                   stream)
             : dispatch_geometry<1, BackwardLauncher>(
                   geo, grad_out, src, offsets, edge_scale, node_scale, order, grad_src,
                   grad_edge_scale, grad_node_scale, n_edges, n_nodes, channels, base, accumulate,
                   stream);
    if (status) return status;
    accumulate = 1;
  }
  return DPA4K_OK;
}

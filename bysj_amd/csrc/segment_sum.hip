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
// Backward is segment-parallel too: the group loads grad_out[n] once, writes
// grad_src for every edge of the segment, and reduces the per-edge channel
// dot product for grad_edge_scale with a fixed butterfly.  The reference's
// edge-parallel grad_src kernel needs `dst`; here the CSR names each edge's
// segment, which the grouping contract makes identical.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;

template <int V, int G, int CPL, bool kScaleEdge, bool kOrdered>
__global__ __launch_bounds__(kBlock) void segment_sum_forward_kernel(
    const float* __restrict__ src, const int64_t* __restrict__ offsets,
    const float* __restrict__ edge_scale, const float* __restrict__ node_scale,
    const int64_t* __restrict__ order, float* __restrict__ out, int64_t n_edges, int64_t n_nodes,
    int64_t channels, int64_t chunk_base) {
  constexpr int kSegments = kBlock / G;
  constexpr int U = CPL >= 8 ? 2 : (CPL >= 4 ? 4 : 8);
  const int64_t segment = static_cast<int64_t>(blockIdx.x) * kSegments + threadIdx.x / G;
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

  int64_t slot = begin;
  for (; slot + U <= end; slot += U) {
    int64_t edge[U];
    float weight[U];
    fvec<V> x[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) edge[u] = edge_of<kOrdered>(order, slot + u, n_edges);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = !kOrdered || edge[u] >= 0;
      weight[u] = kScaleEdge && ok ? edge_scale[edge[u]] : 1.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (live[j] && ok) {
          x[u][j] = load_vec<V>(src + edge[u] * channels + column[j]);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) x[u][j].v[i] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kOrdered && edge[u] < 0) continue;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i)
          acc[j].v[i] = acc[j].v[i] + (kScaleEdge ? x[u][j].v[i] * weight[u] : x[u][j].v[i]);
    }
  }
  for (; slot < end; ++slot) {
    const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
    if (kOrdered && e < 0) continue;
    const float w = kScaleEdge ? edge_scale[e] : 1.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (!live[j]) continue;
      const fvec<V> x = load_vec<V>(src + e * channels + column[j]);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[j].v[i] = acc[j].v[i] + (kScaleEdge ? x.v[i] * w : x.v[i]);
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

// grad_src[e] = (grad_out[n] * node_scale[n]) * edge_scale[e];
// grad_edge_scale[e] = sum_c (grad_out[n, c] * node_scale[n]) * src[e, c];
// grad_node_scale[n] = sum_c grad_out[n, c] * prefix[n, c],
// prefix = sum_e edge_scale[e] * src[e] (recomputed in slot order).
// `accumulate` adds the channel partial of this chunk window to the value
// written by the previous window (channels wider than one window).
template <int V, int G, int CPL, bool kOrdered>
__global__ __launch_bounds__(kBlock) void segment_sum_backward_kernel(
    const float* __restrict__ grad_out, const float* __restrict__ src,
    const int64_t* __restrict__ offsets, const float* __restrict__ edge_scale,
    const float* __restrict__ node_scale, const int64_t* __restrict__ order,
    float* __restrict__ grad_src, float* __restrict__ grad_edge_scale,
    float* __restrict__ grad_node_scale, int64_t n_edges, int64_t n_nodes, int64_t channels,
    int64_t chunk_base, int accumulate) {
  constexpr int kSegments = kBlock / G;
  const int64_t segment = static_cast<int64_t>(blockIdx.x) * kSegments + threadIdx.x / G;
  if (segment >= n_nodes) return;
  const int lane = threadIdx.x % G;
  const int64_t chunks = channels / V;
  const bool want_edge = grad_edge_scale != nullptr;
  const bool want_node = grad_node_scale != nullptr;
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
  fvec<V> g[CPL], gs[CPL], prefix[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    if (live[j]) {
      g[j] = load_vec<V>(grad_out + segment * channels + column[j]);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) g[j].v[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
      gs[j].v[i] = node_scale != nullptr ? g[j].v[i] * scale : g[j].v[i];
      prefix[j].v[i] = 0.0f;
    }
  }

  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  for (int64_t slot = begin; slot < end; ++slot) {
    const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
    if (kOrdered && e < 0) continue;
    const float w = has_edge_scale ? edge_scale[e] : 1.0f;
    fvec<V> x[CPL];
    if (want_edge || want_node) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (live[j]) {
          x[j] = load_vec<V>(src + e * channels + column[j]);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) x[j].v[i] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (!live[j]) continue;
      fvec<V> out;
#pragma unroll
      for (int i = 0; i < V; ++i) out.v[i] = has_edge_scale ? gs[j].v[i] * w : gs[j].v[i];
      store_vec_stream<V>(grad_src + e * channels + column[j], out);
    }
    if (want_edge) {
      float dot = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) dot = dot + gs[j].v[i] * x[j].v[i];
      dot = group_sum<G>(dot);
      if (lane == 0) grad_edge_scale[e] = accumulate ? grad_edge_scale[e] + dot : dot;
    }
    if (want_node) {
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i)
          prefix[j].v[i] = prefix[j].v[i] + (has_edge_scale ? x[j].v[i] * w : x[j].v[i]);
    }
  }
  if (want_node) {
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < V; ++i) dot = dot + g[j].v[i] * prefix[j].v[i];
    dot = group_sum<G>(dot);
    if (lane == 0)
      grad_node_scale[segment] = accumulate ? grad_node_scale[segment] + dot : dot;
  }
}

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

template <int V, int G, int CPL>
int launch_forward(const float* src, const int64_t* offsets, const float* edge_scale,
                   const float* node_scale, const int64_t* order, float* out, int64_t n_edges,
                   int64_t n_nodes, int64_t channels, int64_t chunk_base, hipStream_t stream) {
  const unsigned int grid = blocks_for(n_nodes, kBlock / G);
  if (edge_scale != nullptr) {
    if (order != nullptr)
      segment_sum_forward_kernel<V, G, CPL, true, true><<<grid, kBlock, 0, stream>>>(
          src, offsets, edge_scale, node_scale, order, out, n_edges, n_nodes, channels, chunk_base);
    else
      segment_sum_forward_kernel<V, G, CPL, true, false><<<grid, kBlock, 0, stream>>>(
          src, offsets, edge_scale, node_scale, order, out, n_edges, n_nodes, channels, chunk_base);
  } else {
    if (order != nullptr)
      segment_sum_forward_kernel<V, G, CPL, false, true><<<grid, kBlock, 0, stream>>>(
          src, offsets, edge_scale, node_scale, order, out, n_edges, n_nodes, channels, chunk_base);
    else
      segment_sum_forward_kernel<V, G, CPL, false, false><<<grid, kBlock, 0, stream>>>(
          src, offsets, edge_scale, node_scale, order, out, n_edges, n_nodes, channels, chunk_base);
  }
  return launched("segment_sum_forward_kernel");
}

template <int V, int G, int CPL>
int launch_backward(const float* grad_out, const float* src, const int64_t* offsets,
                    const float* edge_scale, const float* node_scale, const int64_t* order,
                    float* grad_src, float* grad_edge_scale, float* grad_node_scale,
                    int64_t n_edges, int64_t n_nodes, int64_t channels, int64_t chunk_base,
                    int accumulate, hipStream_t stream) {
  const unsigned int grid = blocks_for(n_nodes, kBlock / G);
  if (order != nullptr)
    segment_sum_backward_kernel<V, G, CPL, true><<<grid, kBlock, 0, stream>>>(
        grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale,
        grad_node_scale, n_edges, n_nodes, channels, chunk_base, accumulate);
  else
    segment_sum_backward_kernel<V, G, CPL, false><<<grid, kBlock, 0, stream>>>(
        grad_out, src, offsets, edge_scale, node_scale, order, grad_src, grad_edge_scale,
        grad_node_scale, n_edges, n_nodes, channels, chunk_base, accumulate);
  return launched("segment_sum_backward_kernel");
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
  if ((n_nodes + 3) / 4 > kMaxGrid * 64) return fail(DPA4K_EINVAL, "%s: segment count too large", what);
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

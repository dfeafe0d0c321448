// GIE zonal scatter, forward and backward (python/kernels/gie.py:50-93,
// csrc/gie.cpp:148-228 of the reference; arithmetic of the oracle
// python/reference/gie.py:42-65):
//   out[n, 0, :]   = 0 * inv[n]
//   out[n, r+1, c] = inv[n] * sum_{dst(e)=n} zonal[e, r] * radial[e, slot[r], c]
//
// The reference scatters every (edge, row, channel) product with a float
// atomic into a zero-filled output and rescales it in a second pass.  Here
// the edges are grouped by destination first (csr.hip) and one wave owns one
// node: lane l owns the output chunks q = l, l + 64, ... of rows 1..R
// (chunk = 4 channels), walks the node's edges in CSR order and accumulates
// each element sequentially (product rounded, then added), normalising once
// after the sum.  The node's [R, C] accumulator never leaves registers, the
// output is written once, and the result equals the sequential fp32 chain
// `gather -> mul -> index_add_ -> mul` bit for bit.  The forward kernels load
// the radial rows non-temporally: each is read once, and keeping them out of
// the caches' normal replacement made the [E, 16, 64] forward 5% (fused with
// RMSNorm 8%) faster; the backward kernels keep ordinary loads, which were
// equal or faster there.
//
// Backward is node-parallel as well.  It recomputes the unnormalised sum for
// the inverse-degree gradient in the same pass that reads radial/zonal for
// the zonal/radial gradients, so each edge row is read once.  With distinct
// radial slots (each slot feeds at most one row) lanes own (slot, chunk)
// pairs and everything stays in registers; shared slots (several rows
// reading one slot, e.g. one radial channel per degree l) go through a
// one-wave kernel that stages the per-row products in LDS and sums them per
// slot in ascending row order.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

template <int V, int CPL, bool kOrdered>
__global__ __launch_bounds__(kBlock) void gie_forward_kernel(
    const float* __restrict__ zonal, const float* __restrict__ radial,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ order,
    const int64_t* __restrict__ radial_slot, const float* __restrict__ inv,
    float* __restrict__ out, int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
    int64_t channels, int64_t chunk_base) {
  constexpr int U = CPL >= 8 ? 1 : (CPL >= 4 ? 2 : 4);
  const int64_t node = block_index() * kWaves + (threadIdx.x >> 6);
  if (node >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int64_t row_chunks = channels / V;
  const int64_t chunks = n_rows * row_chunks;
  const int64_t edge_stride = n_radial * channels;

  int64_t zonal_col[CPL], radial_col[CPL], out_col[CPL];
  bool live[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t q = chunk_base + lane + 64 * j;
    const int64_t r = q / row_chunks;
    const int64_t c = q - r * row_chunks;
    int64_t slot = q < chunks ? radial_slot[r] : -1;
    live[j] = static_cast<uint64_t>(slot) < static_cast<uint64_t>(n_radial);
    zonal_col[j] = live[j] ? r : 0;
    radial_col[j] = live[j] ? slot * channels + c * V : 0;
    out_col[j] = (r + 1) * channels + c * V;
    if (q >= chunks) out_col[j] = -1;
  }

  fvec<V> acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[j].v[i] = 0.0f;

  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  int64_t slot = begin;
  for (; slot + U <= end; slot += U) {
    int64_t edge[U];
    float z[U][CPL];
    fvec<V> x[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) edge[u] = edge_of<kOrdered>(order, slot + u, n_edges);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (live[j] && (!kOrdered || edge[u] >= 0)) {
          z[u][j] = zonal[edge[u] * n_rows + zonal_col[j]];
          x[u][j] = load_vec_stream<V>(radial + edge[u] * edge_stride + radial_col[j]);
        } else {
          z[u][j] = 0.0f;
#pragma unroll
          for (int i = 0; i < V; ++i) x[u][j].v[i] = 0.0f;
        }
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kOrdered && edge[u] < 0) continue;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) acc[j].v[i] = acc[j].v[i] + z[u][j] * x[u][j].v[i];
    }
  }
  for (; slot < end; ++slot) {
    const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
    if (kOrdered && e < 0) continue;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (!live[j]) continue;
      const float zv = zonal[e * n_rows + zonal_col[j]];
      const fvec<V> xv = load_vec_stream<V>(radial + e * edge_stride + radial_col[j]);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[j].v[i] = acc[j].v[i] + zv * xv.v[i];
    }
  }

  const float scale = inv[node];
  float* node_out = out + node * (n_rows + 1) * channels;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    if (out_col[j] < 0) continue;
    fvec<V> result;
#pragma unroll
    for (int i = 0; i < V; ++i) result.v[i] = acc[j].v[i] * scale;
    store_vec<V>(node_out + out_col[j], result);
  }
  if (chunk_base == 0) {
    fvec<V> zero;
#pragma unroll
    for (int i = 0; i < V; ++i) zero.v[i] = 0.0f * scale;
    for (int64_t c = lane; c < row_chunks; c += 64) store_vec<V>(node_out + c * V, zero);
  }
}

// Shared radial slots (several rows read one slot, e.g. one radial channel
// per degree l).  Each slot's rows are split into groups of at most G rows,
// G the smallest that lets every group have row_chunks = C / 4 lanes of its
// own (a slot with k rows takes ceil(k / G) groups); lane pair p = lane + 64 j
// serves chunk p % row_chunks of group p / row_chunks.  Every radial element
// is then loaded by one lane per group of its slot instead of once per row,
// and the lanes' row counts stay within G of each other (DeepMD's 3 / 5 / 7
// rows at C = 64 become 4 groups of at most 5).  Lane r < R loads zonal[e, r]
// and the lanes fetch the values of their rows with ds_bpermute.  Per output
// element the arithmetic is gie_forward_kernel's (edges in CSR order, product
// rounded, then added, normalised after the sum): the same output bit for
// bit.  Needs C % 4 == 0, 1 <= R <= 64, S <= 64, S * C / 4 <= 64 * PPL, and
// at most MAXR rows per slot.  With kRowBcast (C / 4 a multiple of 16, so a
// group is whole 16-lane rows of the wave), lane k of each row loads the
// zonal value of its group's k-th row instead, and a DPP row broadcast
// (row_newbcast) hands it to the row: a VALU move in place of the
// ds_bpermute, which goes through the LDS pipeline.
// Lane k of each 16-lane row of the wave, to every lane of that row (DPP row_newbcast:k).
template <int K>
__device__ __forceinline__ float row_broadcast_of(float value) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(value), 0x150 + K, 0xf, 0xf, false));
}

// k < 8, a constant once the caller's loop is unrolled (the switch folds away).
__device__ __forceinline__ float row_broadcast(float value, int k) {
  switch (k) {
    case 0: return row_broadcast_of<0>(value);
    case 1: return row_broadcast_of<1>(value);
    case 2: return row_broadcast_of<2>(value);
    case 3: return row_broadcast_of<3>(value);
    case 4: return row_broadcast_of<4>(value);
    case 5: return row_broadcast_of<5>(value);
    case 6: return row_broadcast_of<6>(value);
    default: return row_broadcast_of<7>(value);
  }
}

template <int PPL, int MAXR, bool kRowBcast, bool kOrdered>
__global__ __launch_bounds__(kBlock) void gie_forward_shared_kernel(
    const float* __restrict__ zonal, const float* __restrict__ radial,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ order,
    const int64_t* __restrict__ radial_slot, const float* __restrict__ inv,
    float* __restrict__ out, int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
    int64_t channels) {
  constexpr int U = 4;
  const int64_t node = block_index() * kWaves + (threadIdx.x >> 6);
  if (node >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int row_chunks = static_cast<int>(channels / 4);
  const int slots = static_cast<int>(n_radial);
  const int rows = static_cast<int>(n_rows);
  const int64_t edge_stride = n_radial * channels;

  // the group plan, the same in every lane: lane t < S counts the rows of slot t
  int rows_of_lane_slot = 0;
  for (int r = 0; r < rows; ++r) rows_of_lane_slot += radial_slot[r] == lane ? 1 : 0;
  const int groups_available = 64 * PPL / row_chunks;
  int group_rows = MAXR;
  for (int g = 1; g < MAXR; ++g) {
    int needed = 0;
    for (int t = 0; t < slots; ++t) needed += (__builtin_amdgcn_readlane(rows_of_lane_slot, t) + g - 1) / g;
    if (needed <= groups_available) {
      group_rows = g;
      break;
    }
  }

  // each pair's slot and its rows (ascending); unused entries point at row 0
  int row_of[PPL][MAXR];
  int count[PPL];
  int64_t radial_col[PPL], chunk_col[PPL];
  // (a lambda: the edge loop's row-broadcast path rebuilds the rows after the loop)
  const auto plan_pairs = [&](int who) {
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const int p = who + 64 * j;
      const int group = p / row_chunks;
      const int c = p - group * row_chunks;
      int slot = -1, part = 0, first = 0;
      for (int t = 0; t < slots; ++t) {
        const int groups = (__builtin_amdgcn_readlane(rows_of_lane_slot, t) + group_rows - 1) / group_rows;
        if (group >= first && group < first + groups) {
          slot = t;
          part = group - first;
        }
        first += groups;
      }
      radial_col[j] = slot >= 0 ? static_cast<int64_t>(slot) * channels + c * 4 : 0;
      chunk_col[j] = c * 4;
      count[j] = 0;
#pragma unroll
      for (int k = 0; k < MAXR; ++k) row_of[j][k] = 0;
      int seen = 0;
      for (int r = 0; r < rows; ++r) {
        const bool reads = slot >= 0 && radial_slot[r] == slot;
        const int k = seen - part * group_rows;
        const bool mine = reads && k >= 0 && k < group_rows;
#pragma unroll
        for (int kk = 0; kk < MAXR; ++kk)
          if (mine && k == kk) row_of[j][kk] = r;
        count[j] += mine ? 1 : 0;
        seen += reads ? 1 : 0;
      }
    }
  };
  plan_pairs(lane);

  fvec<4> acc[PPL][MAXR];
#pragma unroll
  for (int j = 0; j < PPL; ++j)
#pragma unroll
    for (int k = 0; k < MAXR; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][k].v[i] = 0.0f;

  // the zonal row this lane loads: its own index (ds_bpermute), or the (lane mod 16)-th row of
  // each pair's group (row broadcast)
  int64_t zonal_row[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    if constexpr (kRowBcast) {
      const int k = lane & 15;
      int row = row_of[j][0];
#pragma unroll
      for (int kk = 1; kk < MAXR; ++kk) row = k == kk && kk < count[j] ? row_of[j][kk] : row;
      zonal_row[j] = row;
    } else {
      zonal_row[j] = lane < rows ? lane : rows - 1;
    }
  }
  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  for (int64_t slot = begin; slot < end; slot += U) {
    int64_t edge[U];
    bool use[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = slot + u < end ? edge_of<kOrdered>(order, slot + u, n_edges) : -1;
      use[u] = e >= 0;
      edge[u] = e >= 0 ? e : begin;  // a valid edge to load from when this one is skipped
    }
    constexpr int ZQ = kRowBcast ? PPL : 1;
    float zq[U][ZQ];
    fvec<4> x[U][PPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < ZQ; ++j) zq[u][j] = zonal[edge[u] * n_rows + zonal_row[j]];
#pragma unroll
      for (int j = 0; j < PPL; ++j) x[u][j] = load_vec_stream<4>(radial + edge[u] * edge_stride + radial_col[j]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!use[u]) continue;  // wave-uniform
#pragma unroll
      for (int k = 0; k < MAXR; ++k) {
        if (k >= group_rows) break;  // wave-uniform
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
          float z;
          if constexpr (kRowBcast)
            z = row_broadcast(zq[u][j], k);
          else
            z = __int_as_float(__builtin_amdgcn_ds_bpermute(row_of[j][k] << 2, __float_as_int(zq[u][0])));
          if (k < count[j])
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[j][k].v[i] = acc[j][k].v[i] + z * x[u][j].v[i];
        }
      }
    }
  }

  if constexpr (kRowBcast) {
    // (the rows of each pair rebuilt here rather than held in registers through the edge loop)
    int again = lane;
    asm volatile("" : "+v"(again));
    plan_pairs(again);
  }
  const float scale = inv[node];
  float* node_out = out + node * (n_rows + 1) * channels;
#pragma unroll
  for (int j = 0; j < PPL; ++j)
#pragma unroll
    for (int k = 0; k < MAXR; ++k) {
      if (k >= count[j]) continue;
      fvec<4> result;
#pragma unroll
      for (int i = 0; i < 4; ++i) result.v[i] = acc[j][k].v[i] * scale;
      store_vec<4>(node_out + (row_of[j][k] + 1) * channels + chunk_col[j], result);
    }
  // row 0, and rows whose slot is out of range (no group serves them): 0 * inv
  fvec<4> zero;
#pragma unroll
  for (int i = 0; i < 4; ++i) zero.v[i] = 0.0f * scale;
  for (int64_t c = lane; c < row_chunks; c += 64) store_vec<4>(node_out + c * 4, zero);
  for (int64_t r = 0; r < n_rows; ++r)
    if (static_cast<uint64_t>(radial_slot[r]) >= static_cast<uint64_t>(n_radial))
      for (int64_t c = lane; c < row_chunks; c += 64) store_vec<4>(node_out + (r + 1) * channels + c * 4, zero);
}

// Fused GIE -> RMSNorm over each node's flattened row of W = (R + 1) * C
// floats (no reference counterpart; the reference runs the two operators
// back to back).  One wave per node, float4 chunks.  Lane l owns the chunks
// q = l + 64 j of the whole row, row 0 included -- the chunk layout of
// rmsnorm_forward_kernel -- and accumulates the GIE sum of the chunks it owns
// exactly as gie_forward_kernel does (slot order, product rounded before the
// add, normalised by inv_sqrt_deg after the sum).  The sum of squares,
// 1 / sqrt(mean + eps) and the scaled output then follow the RMSNorm kernel
// step for step, so y, the pre-norm row x (written only when x_out is
// given) and inverse_rms equal the two kernels run back to back, bit for bit.
__device__ __forceinline__ float fused_inverse_rms(float sum_squares, int64_t width, float eps) {
  return 1.0f / sqrtf(sum_squares / static_cast<float>(width) + eps);
}

template <int CPL, bool kOrdered>
__global__ __launch_bounds__(kBlock) void gie_rmsnorm_forward_kernel(
    const float* __restrict__ zonal, const float* __restrict__ radial,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ order,
    const int64_t* __restrict__ radial_slot, const float* __restrict__ inv,
    const float* __restrict__ scale, float eps, float* __restrict__ y, float* __restrict__ x_out,
    float* __restrict__ inverse_rms, int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
    int64_t channels) {
  constexpr int V = 4;
  constexpr int U = CPL >= 8 ? 1 : (CPL >= 4 ? 2 : 4);
  const int64_t node = block_index() * kWaves + (threadIdx.x >> 6);
  if (node >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int64_t row_chunks = channels / V;
  const int64_t chunks = (n_rows + 1) * row_chunks;  // the whole row, row 0 included
  const int64_t width = (n_rows + 1) * channels;
  const int64_t edge_stride = n_radial * channels;

  int64_t zonal_col[CPL], radial_col[CPL];
  bool live[CPL];
  fvec<V> s[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t q = lane + 64 * j;
    const int64_t gq = q - row_chunks;  // chunk of rows 1..R
    const int64_t r = gq >= 0 ? gq / row_chunks : 0;
    const int64_t c = gq >= 0 ? gq - r * row_chunks : 0;
    const int64_t slot = (gq >= 0 && q < chunks) ? radial_slot[r] : -1;
    live[j] = static_cast<uint64_t>(slot) < static_cast<uint64_t>(n_radial);
    zonal_col[j] = live[j] ? r : 0;
    radial_col[j] = live[j] ? slot * channels + c * V : 0;
#pragma unroll
    for (int i = 0; i < V; ++i) s[j].v[i] = 0.0f;
    if (q < chunks && scale != nullptr) s[j] = load_vec<V>(scale + q * V);
  }

  fvec<V> acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[j].v[i] = 0.0f;

  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  int64_t slot = begin;
  for (; slot + U <= end; slot += U) {
    int64_t edge[U];
    float z[U][CPL];
    fvec<V> x[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) edge[u] = edge_of<kOrdered>(order, slot + u, n_edges);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if (live[j] && (!kOrdered || edge[u] >= 0)) {
          z[u][j] = zonal[edge[u] * n_rows + zonal_col[j]];
          x[u][j] = load_vec_stream<V>(radial + edge[u] * edge_stride + radial_col[j]);
        } else {
          z[u][j] = 0.0f;
#pragma unroll
          for (int i = 0; i < V; ++i) x[u][j].v[i] = 0.0f;
        }
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kOrdered && edge[u] < 0) continue;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) acc[j].v[i] = acc[j].v[i] + z[u][j] * x[u][j].v[i];
    }
  }
  for (; slot < end; ++slot) {
    const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
    if (kOrdered && e < 0) continue;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (!live[j]) continue;
      const float zv = zonal[e * n_rows + zonal_col[j]];
      const fvec<V> xv = load_vec_stream<V>(radial + e * edge_stride + radial_col[j]);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[j].v[i] = acc[j].v[i] + zv * xv.v[i];
    }
  }

  // the GIE output row (row 0 and absent rows: 0 * inv), then RMSNorm over it
  const float degree_scale = inv[node];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const bool in_row = lane + 64 * j < chunks;
#pragma unroll
    for (int i = 0; i < V; ++i) acc[j].v[i] = in_row ? acc[j].v[i] * degree_scale : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int i = 0; i < V; ++i) sum = sum + acc[j].v[i] * acc[j].v[i];
  sum = group_sum<64>(sum);
  const float inv_rms = fused_inverse_rms(sum, width, eps);
  float* y_row = y + node * width;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t q = lane + 64 * j;
    if (q >= chunks) continue;
    fvec<V> out;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      out.v[i] = acc[j].v[i] * inv_rms;
      if (scale != nullptr) out.v[i] = out.v[i] * s[j].v[i];
    }
    store_vec_stream<V>(y_row + q * V, out);
    if (x_out != nullptr) store_vec<V>(x_out + node * width + q * V, acc[j]);
  }
  if (lane == 0) inverse_rms[node] = inv_rms;
}

// Distinct slots: lane owns (slot s, chunk c) pairs q = s * row_chunks + c of
// one edge's radial block; RC = row_chunks lanes share a slot (power of two).
template <int V, int CPL, int RC, bool kOrdered>
__global__ __launch_bounds__(kBlock) void gie_backward_distinct_kernel(
    const float* __restrict__ grad_output, const float* __restrict__ zonal,
    const float* __restrict__ radial, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ order, const int64_t* __restrict__ radial_slot,
    const float* __restrict__ inv, float* __restrict__ grad_zonal, float* __restrict__ grad_radial,
    float* __restrict__ grad_inv, int64_t n_edges, int64_t n_nodes, int64_t n_rows,
    int64_t n_radial, int64_t channels) {
  const int64_t node = block_index() * kWaves + (threadIdx.x >> 6);
  if (node >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int64_t chunks = n_radial * RC;
  const int64_t edge_stride = n_radial * channels;
  const float scale = inv[node];

  // Per-lane 32-bit byte offsets into an edge's radial block and zonal row
  // (kNoRow where the lane has no row), so the edge loop keeps no 64-bit
  // addresses in registers.
  uint32_t col_at[CPL], zon_at[CPL], out_at[CPL], gz_at[CPL];
  fvec<V> g[CPL], pre[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t q = lane + 64 * j;
    const int64_t s = q / RC;
    const int64_t c = q % RC;
    const bool in_range = q < chunks;
    int64_t r = -1;
    if (in_range)
      for (int64_t k = 0; k < n_rows; ++k)
        if (radial_slot[k] == s) r = k;
    const uint32_t col = static_cast<uint32_t>(s * channels + c * V) * 4u;
    col_at[j] = r >= 0 ? col : kNoRow;
    zon_at[j] = r >= 0 ? static_cast<uint32_t>(r) * 4u : kNoRow;
    out_at[j] = in_range ? col : kNoRow;
    gz_at[j] = in_range && r >= 0 && (lane % RC) == 0 ? static_cast<uint32_t>(r) * 4u : kNoRow;
    if (r >= 0) {
      g[j] = load_vec<V>(grad_output + (node * (n_rows + 1) + r + 1) * channels + c * V);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) g[j].v[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) pre[j].v[i] = 0.0f;
  }
  const int64_t radial_bytes = edge_stride * 4, zonal_bytes = n_rows * 4;

  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  for (int64_t slot = begin; slot < end; ++slot) {
    const int64_t e = uniform_i64(edge_of<kOrdered>(order, slot, n_edges));
    if (kOrdered && e < 0) continue;
    const BufferView rv = buffer_view(radial + e * edge_stride, radial_bytes);
    const BufferView zv = buffer_view(zonal + e * n_rows, zonal_bytes);
    fvec<V> x[CPL];
    float z[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      x[j] = buffer_load_vec<V>(rv, col_at[j]);
      z[j] = buffer_load_f32(zv, zon_at[j]);
    }
    float sc = scale;
    asm volatile("" : "+v"(sc));  // keeps g * scale inside the loop
    const BufferView ov = grad_radial != nullptr ? buffer_view(grad_radial + e * edge_stride, radial_bytes)
                                                 : buffer_view(radial, 0);
    const BufferView gv = grad_zonal != nullptr ? buffer_view(grad_zonal + e * n_rows, zonal_bytes)
                                                : buffer_view(radial, 0);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float dot = 0.0f;
      fvec<V> out;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        pre[j].v[i] = pre[j].v[i] + z[j] * x[j].v[i];
        const float h = g[j].v[i] * sc;
        dot = dot + h * x[j].v[i];
        out.v[i] = h * z[j];
      }
      dot = group_sum<RC>(dot);
      buffer_store_vec_stream<V>(ov, out_at[j], out);
      buffer_store_f32(gv, gz_at[j], dot);
    }
  }
  if (grad_inv != nullptr) {
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < V; ++i) total = total + g[j].v[i] * pre[j].v[i];
    total = group_sum<64>(total);
    if (lane == 0) grad_inv[node] = total;
  }
}

// Shared radial slots, backward.  LPE = S * RC lanes serve one edge (RC =
// C / 8 lanes per slot, 8 channels each) and EPI = 64 / LPE edges are
// handled side by side: lane (u, s, c) takes edge slot base + u, radial slot
// s and channels [8 c, 8 c + 8) for every row r that reads s (at most MAXR),
// with that node's upstream rows g[r + 1, :] held in registers:
//   grad_zonal[e, r]      = inv * sum_c g[r, c] radial[e, s, c]   (RC-lane butterfly)
//   grad_radial[e, s, c]  = sum_{r reads s} g[r, c] * (zonal[e, r] * inv)
//   grad_inv             += zonal[e, r] * sum_c g[r, c] radial[e, s, c]
// Each radial element is read and each gradient written once.  Every
// iteration loads UU wave steps' radial and zonal values before any of
// their arithmetic, which keeps enough bytes in flight per wave.  (Measured
// on the DeepMD map at C = 64: 8 channels per lane beat 4 (more butterfly
// steps) and 16 (register-bound occupancy), and the plain loop beat
// software-pipelined forms, whose loads waited for the previous step's
// stores: gfx9's vmcnt counts both.)  Fused multiply-adds in a fixed order:
// reproducible, within fp32 rounding of the oracle's (inv * g) . radial
// association.  Needs C % 8 == 0 with RC a power of two and S * RC <= 64.
template <int RC, int MAXR, bool kOrdered>
__global__ __launch_bounds__(kBlock) void gie_backward_shared_kernel(
    const float* __restrict__ grad_output, const float* __restrict__ zonal,
    const float* __restrict__ radial, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ order, const int64_t* __restrict__ radial_slot,
    const float* __restrict__ inv, float* __restrict__ grad_zonal, float* __restrict__ grad_radial,
    float* __restrict__ grad_inv, int64_t n_edges, int64_t n_nodes, int64_t n_rows,
    int64_t n_radial, int64_t channels) {
  constexpr int V = 8;
  constexpr int UU = 4;
  const int64_t node = block_index() * kWaves + (threadIdx.x >> 6);
  if (node >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  const int lpe = static_cast<int>(n_radial) * RC;
  const int epi = 64 / lpe;
  const int u = lane / lpe;
  const int w = lane - u * lpe;
  const bool active = u < epi;
  const int64_t s = active ? w / RC : -1;
  const int c = w % RC;
  const int64_t edge_stride = n_radial * channels;
  const int64_t radial_col = (active ? s : 0) * channels + c * V;
  const float scale = inv[node];

  // the rows of this lane's slot, ascending; unused entries point at row 0
  int row_of[MAXR];
  int count = 0;
#pragma unroll
  for (int k = 0; k < MAXR; ++k) row_of[k] = 0;
  bool stray_rows = false;  // rows whose slot is out of range: their zonal gradient is zero
  for (int64_t r = 0; r < n_rows; ++r) {
    const int64_t slot = radial_slot[r];
    stray_rows = stray_rows || static_cast<uint64_t>(slot) >= static_cast<uint64_t>(n_radial);
    const bool reads = active && slot == s;
#pragma unroll
    for (int k = 0; k < MAXR; ++k)
      if (reads && count == k) row_of[k] = static_cast<int>(r);
    count += reads ? 1 : 0;
  }

  float g[MAXR][V];
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const float* row = grad_output + (node * (n_rows + 1) + row_of[k] + 1) * channels + c * V;
#pragma unroll
    for (int q = 0; q < V / 4; ++q) {
      fvec<4> part;
#pragma unroll
      for (int i = 0; i < 4; ++i) part.v[i] = 0.0f;
      if (k < count) part = load_vec<4>(row + 4 * q);
#pragma unroll
      for (int i = 0; i < 4; ++i) g[k][4 * q + i] = part.v[i];
    }
  }

  float inv_partial = 0.0f;
  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  for (int64_t base = begin; base < end; base += UU * epi) {
    int64_t e[UU];
    float x[UU][V], z[UU][MAXR];
#pragma unroll
    for (int uu = 0; uu < UU; ++uu) {
      const int64_t at = base + uu * epi + u;
      e[uu] = active && at < end ? edge_of<kOrdered>(order, at, n_edges) : -1;
      const int64_t edge = e[uu] >= 0 ? e[uu] : begin;  // a valid edge to load from
#pragma unroll
      for (int q = 0; q < V / 4; ++q) {
        const fvec<4> part = load_vec<4>(radial + edge * edge_stride + radial_col + 4 * q);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[uu][4 * q + i] = part.v[i];
      }
#pragma unroll
      for (int k = 0; k < MAXR; ++k) z[uu][k] = zonal[edge * n_rows + row_of[k]];
    }
#pragma unroll
    for (int uu = 0; uu < UU; ++uu) {
      const bool use = e[uu] >= 0;
      float out[V];
#pragma unroll
      for (int i = 0; i < V; ++i) out[i] = 0.0f;
#pragma unroll
      for (int k = 0; k < MAXR; ++k) {
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) dot = __builtin_fmaf(g[k][i], x[uu][i], dot);
        dot = group_sum<RC>(dot);
        if (use && k < count && c == 0) {
          if (grad_zonal != nullptr) grad_zonal[e[uu] * n_rows + row_of[k]] = dot * scale;
          inv_partial = __builtin_fmaf(z[uu][k], dot, inv_partial);
        }
        const float weight = k < count ? z[uu][k] * scale : 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) out[i] = __builtin_fmaf(g[k][i], weight, out[i]);
      }
      if (use && grad_radial != nullptr)
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          fvec<4> part;
#pragma unroll
          for (int i = 0; i < 4; ++i) part.v[i] = out[4 * q + i];
          store_vec_stream<4>(grad_radial + e[uu] * edge_stride + radial_col + 4 * q, part);
        }
    }
  }
  if (stray_rows && grad_zonal != nullptr)
    for (int64_t r = 0; r < n_rows; ++r)
      if (static_cast<uint64_t>(radial_slot[r]) >= static_cast<uint64_t>(n_radial))
        for (int64_t at = begin + lane; at < end; at += 64) {
          const int64_t e = edge_of<kOrdered>(order, at, n_edges);
          if (e >= 0) grad_zonal[e * n_rows + r] = 0.0f;
        }
  if (grad_inv != nullptr) {
    const float total = group_sum<64>(inv_partial);
    if (lane == 0) grad_inv[node] = total;
  }
}

// Shared radial slots, backward, with S slots known at compile time: RC =
// C / 8 lanes serve one edge (lane c of the group owns channels [8 c, 8 c +
// 8) of every slot: S * 8 radial values) and EW = 64 / RC edges are handled
// side by side, every lane busy.  The node's upstream rows g[r + 1, :] sit in
// LDS (each wave its own node's), and the wave walks the rows slot by slot,
// in ascending order within a slot, with no masked iterations:
//   dot                   = sum_c g[r, c] radial[e, s(r), c]   (8 FMAs, RC-lane butterfly)
//   grad_zonal[e, r]      = inv * dot                          (kept by lane r mod RC)
//   grad_radial[e, s, c] += g[r, c] * (zonal[e, r] * inv)
//   grad_inv             += zonal[e, r] * dot                  (lane r mod RC)
// zonal[e, r] is loaded by lane r mod RC of the edge's group and reaches
// the others through ds_bpermute.  Each radial element is read and each
// gradient written once.  The dot products and grad_radial are
// gie_backward_shared_kernel's to the bit (same channel split, butterfly and
// row order); grad_inv adds the same terms over another lane partition.
// Needs C = 8 RC, n_rows <= ZR * RC and n_rows * C <= kEdgeLaneRowFloats.
constexpr int kEdgeLaneRowFloats = 4096;  // upstream floats staged per wave (16 KB)

template <int RC, int S, int ZR, bool kOrdered>
__global__ __launch_bounds__(kBlock) void gie_backward_edge_lanes_kernel(
    const float* __restrict__ grad_output, const float* __restrict__ zonal,
    const float* __restrict__ radial, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ order, const int64_t* __restrict__ radial_slot,
    const float* __restrict__ inv, float* __restrict__ grad_zonal, float* __restrict__ grad_radial,
    float* __restrict__ grad_inv, int64_t n_edges, int64_t n_nodes, int64_t n_rows,
    int64_t channels) {
  constexpr int V = 8;
  constexpr int EW = 64 / RC;        // edges per wave step
  constexpr int UU = 2;              // wave steps whose loads go out together
  extern __shared__ float staged[];  // [kWaves][rows * C]
  const int wave = threadIdx.x >> 6;
  const int64_t node = block_index() * kWaves + wave;
  const bool live = node < n_nodes;
  const int lane = threadIdx.x & 63;
  const int u = lane / RC, c = lane % RC;
  const int rows = static_cast<int>(n_rows);
  const int64_t edge_stride = S * channels;
  float* g_rows = staged + wave * rows * channels;
  const float scale = live ? inv[node] : 0.0f;

  // the node's upstream rows 1..R into this wave's LDS
  if (live) {
    const float* src = grad_output + (node * (n_rows + 1) + 1) * channels;
    for (int64_t q = lane; q < rows * channels / 4; q += 64) store_vec<4>(g_rows + 4 * q, load_vec<4>(src + 4 * q));
  }
  __syncthreads();
  if (!live) return;

  // the rows in slot order: lane k holds the k-th row of the slot-major list; first[s] bounds slot s
  int slot_of_row = lane < rows ? static_cast<int>(radial_slot[lane]) : -1;
  slot_of_row = static_cast<uint64_t>(slot_of_row) < static_cast<uint64_t>(S) ? slot_of_row : -1;
  int listed = 0, first[S + 1];
  first[0] = 0;
#pragma unroll
  for (int t = 0; t < S; ++t) {
    const uint64_t mine = __ballot(slot_of_row == t);
    const int before = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mine >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mine), 0u));
    // lane r (a row of slot t) becomes entry first[t] + before of the list
    if (slot_of_row == t) listed = first[t] + before;
    first[t + 1] = first[t] + __builtin_popcountll(mine);
  }
  int row_list = 0;  // lane k: the row at list position k
  {
    // scatter: row r goes to lane listed(r); a ds_permute writes each lane's value to the lane it names
    const int target = slot_of_row >= 0 ? listed : 63;
    row_list = __builtin_amdgcn_ds_permute(target << 2, lane);
  }

  float inv_partial = 0.0f;
  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  for (int64_t base = begin; base < end; base += UU * EW) {
    int64_t e[UU];
    float x[UU][S][V], zq[UU][ZR];
#pragma unroll
    for (int uu = 0; uu < UU; ++uu) {
      const int64_t at = base + uu * EW + u;
      e[uu] = at < end ? edge_of<kOrdered>(order, at, n_edges) : -1;
      const int64_t edge = e[uu] >= 0 ? e[uu] : begin;  // a valid edge to load from
#pragma unroll
      for (int t = 0; t < S; ++t)
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          const fvec<4> part = load_vec<4>(radial + edge * edge_stride + t * channels + c * V + 4 * q);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[uu][t][4 * q + i] = part.v[i];
        }
#pragma unroll
      for (int j = 0; j < ZR; ++j) {
        const int r = j * RC + c;
        zq[uu][j] = r < rows ? zonal[edge * n_rows + r] : 0.0f;
      }
    }
    float out[UU][S][V], dz[UU][ZR];
#pragma unroll
    for (int uu = 0; uu < UU; ++uu) {
#pragma unroll
      for (int t = 0; t < S; ++t)
#pragma unroll
        for (int i = 0; i < V; ++i) out[uu][t][i] = 0.0f;
#pragma unroll
      for (int j = 0; j < ZR; ++j) dz[uu][j] = 0.0f;
    }
#pragma unroll
    for (int t = 0; t < S; ++t) {
      for (int k = first[t]; k < first[t + 1]; ++k) {  // uniform: the rows of slot t, ascending
        const int r = __builtin_amdgcn_readlane(row_list, k);
        const int holder = r % RC, j = r / RC;
        const bool mine = c == holder;
        const fvec<4> g0 = load_vec<4>(g_rows + r * channels + c * V);
        const fvec<4> g1 = load_vec<4>(g_rows + r * channels + c * V + 4);
        const float g[V] = {g0.v[0], g0.v[1], g0.v[2], g0.v[3], g1.v[0], g1.v[1], g1.v[2], g1.v[3]};
#pragma unroll
        for (int uu = 0; uu < UU; ++uu) {  // the row's upstream values serve every edge step in flight
          float zr = zq[uu][0];
#pragma unroll
          for (int jj = 1; jj < ZR; ++jj) zr = j == jj ? zq[uu][jj] : zr;
          const float z = __int_as_float(
              __builtin_amdgcn_ds_bpermute((u * RC + holder) << 2, __float_as_int(zr)));
          float dot = 0.0f;
#pragma unroll
          for (int i = 0; i < V; ++i) dot = __builtin_fmaf(g[i], x[uu][t][i], dot);
          dot = group_sum<RC>(dot);
#pragma unroll
          for (int jj = 0; jj < ZR; ++jj) dz[uu][jj] = mine && j == jj ? dot * scale : dz[uu][jj];
          inv_partial = mine && e[uu] >= 0 ? __builtin_fmaf(z, dot, inv_partial) : inv_partial;
          const float weight = z * scale;
#pragma unroll
          for (int i = 0; i < V; ++i) out[uu][t][i] = __builtin_fmaf(g[i], weight, out[uu][t][i]);
        }
      }
    }
#pragma unroll
    for (int uu = 0; uu < UU; ++uu) {
      if (e[uu] >= 0) {
        if (grad_radial != nullptr)
#pragma unroll
          for (int t = 0; t < S; ++t)
#pragma unroll
            for (int q = 0; q < V / 4; ++q) {
              fvec<4> part;
#pragma unroll
              for (int i = 0; i < 4; ++i) part.v[i] = out[uu][t][4 * q + i];
              store_vec_stream<4>(grad_radial + e[uu] * edge_stride + t * channels + c * V + 4 * q, part);
            }
        if (grad_zonal != nullptr)
#pragma unroll
          for (int j = 0; j < ZR; ++j) {
            const int r = j * RC + c;
            if (r < rows) grad_zonal[e[uu] * n_rows + r] = dz[uu][j];  // 0 for a row whose slot is out of range
          }
      }
    }
  }
  if (grad_inv != nullptr) {
    const float total = group_sum<64>(inv_partial);
    if (lane == 0) grad_inv[node] = total;
  }
}

// General slot map: one wave per block.  Read chunks q = r * wc + c over
// rows x window chunks, write chunks t = s * wc + c over slots x window
// chunks.  LDS holds, per edge, the dot partials and the products
// h[r, c] * zonal[e, r]; the per-slot row lists are built once per block.
template <int V, int CPL>
__global__ __launch_bounds__(64) void gie_backward_general_kernel(
    const float* __restrict__ grad_output, const float* __restrict__ zonal,
    const float* __restrict__ radial, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ order, const int64_t* __restrict__ radial_slot,
    const float* __restrict__ inv, float* __restrict__ grad_zonal, float* __restrict__ grad_radial,
    float* __restrict__ grad_inv, int64_t n_edges, int64_t n_nodes, int64_t n_rows,
    int64_t n_radial, int64_t channels, int64_t window_base, int64_t window_chunks) {
  extern __shared__ float lds[];
  // Layout: dot[64*CPL] | product[64*CPL*V] | slot_begin[n_radial+1] | slot_rows[n_rows]
  float* dot_part = lds;
  float* product = lds + 64 * CPL;
  int* slot_begin = reinterpret_cast<int*>(product + 64 * CPL * V);
  int* slot_rows = slot_begin + n_radial + 1;

  const int64_t node = block_index();
  if (node >= n_nodes) return;
  const int lane = threadIdx.x;
  const int64_t wc = window_chunks;
  const bool ordered = order != nullptr;
  const int64_t edge_stride = n_radial * channels;
  const bool first_window = window_base == 0;

  if (lane == 0) {
    int cursor = 0;
    for (int64_t s = 0; s < n_radial; ++s) {
      slot_begin[s] = cursor;
      for (int64_t r = 0; r < n_rows; ++r)
        if (radial_slot[r] == s) slot_rows[cursor++] = static_cast<int>(r);
    }
    slot_begin[n_radial] = cursor;
  }
  __syncthreads();

  const float scale = inv[node];
  const int64_t read_chunks = n_rows * wc;
  const int64_t write_chunks = n_radial * wc;
  int64_t rrow[CPL], rcol[CPL], slotcol[CPL];
  bool rlive[CPL];
  fvec<V> g[CPL], h[CPL], pre[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t q = lane + 64 * j;
    const int64_t r = q / wc;
    const int64_t c = q - r * wc;
    rlive[j] = q < read_chunks;
    const int64_t s = rlive[j] ? radial_slot[r] : 0;
    rlive[j] = rlive[j] && static_cast<uint64_t>(s) < static_cast<uint64_t>(n_radial);
    rrow[j] = r;
    rcol[j] = window_base + c * V;
    slotcol[j] = s * channels + window_base + c * V;
    if (rlive[j]) {
      g[j] = load_vec<V>(grad_output + (node * (n_rows + 1) + r + 1) * channels + rcol[j]);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) g[j].v[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
      h[j].v[i] = g[j].v[i] * scale;
      pre[j].v[i] = 0.0f;
    }
  }

  int64_t begin, end;
  segment_bounds(offsets, node, n_edges, begin, end);
  for (int64_t slot = begin; slot < end; ++slot) {
    const int64_t e = ordered ? edge_of<true>(order, slot, n_edges) : slot;
    if (e < 0) continue;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float dot = 0.0f;
      fvec<V> u;
      if (rlive[j]) {
        const fvec<V> x = load_vec<V>(radial + e * edge_stride + slotcol[j]);
        const float z = zonal[e * n_rows + rrow[j]];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          pre[j].v[i] = pre[j].v[i] + z * x.v[i];
          dot = dot + h[j].v[i] * x.v[i];
          u.v[i] = h[j].v[i] * z;
        }
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) u.v[i] = 0.0f;
      }
      dot_part[lane + 64 * j] = dot;
#pragma unroll
      for (int i = 0; i < V; ++i) product[(lane + 64 * j) * V + i] = u.v[i];
    }
    __syncthreads();
    if (grad_zonal != nullptr)
      for (int64_t r = lane; r < n_rows; r += 64) {
        float sum = first_window ? 0.0f : grad_zonal[e * n_rows + r];
        for (int64_t c = 0; c < wc; ++c) sum = sum + dot_part[r * wc + c];
        grad_zonal[e * n_rows + r] = sum;
      }
    if (grad_radial != nullptr)
      for (int64_t t = lane; t < write_chunks; t += 64) {
        const int64_t s = t / wc;
        const int64_t c = t - s * wc;
        fvec<V> sum;
#pragma unroll
        for (int i = 0; i < V; ++i) sum.v[i] = 0.0f;
        for (int k = slot_begin[s]; k < slot_begin[s + 1]; ++k) {
          const int64_t q = static_cast<int64_t>(slot_rows[k]) * wc + c;
#pragma unroll
          for (int i = 0; i < V; ++i) sum.v[i] = sum.v[i] + product[q * V + i];
        }
        store_vec<V>(grad_radial + e * edge_stride + s * channels + window_base + c * V, sum);
      }
    __syncthreads();
  }
  if (grad_inv != nullptr) {
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < V; ++i) total = total + g[j].v[i] * pre[j].v[i];
    total = group_sum<64>(total);
    if (lane == 0) grad_inv[node] = first_window ? total : grad_inv[node] + total;
  }
}

int per_lane_for(int64_t chunks) {
  int cpl = 1;
  while (cpl < 8 && 64 * cpl < chunks) cpl <<= 1;
  return cpl;
}

template <int V, bool kOrdered>
int launch_forward(int cpl, const float* zonal, const float* radial, const int64_t* offsets,
                   const int64_t* order, const int64_t* radial_slot, const float* inv, float* out,
                   int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
                   int64_t channels, int64_t base, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
#define DPA4K_GIE_FWD(C)                                                                      \
  gie_forward_kernel<V, C, kOrdered><<<grid, kBlock, 0, stream>>>(                           \
      zonal, radial, offsets, order, radial_slot, inv, out, n_edges, n_nodes, n_rows, n_radial, \
      channels, base)
  switch (cpl) {
    case 1: DPA4K_GIE_FWD(1); break;
    case 2: DPA4K_GIE_FWD(2); break;
    case 4: DPA4K_GIE_FWD(4); break;
    default: DPA4K_GIE_FWD(8); break;
  }
#undef DPA4K_GIE_FWD
  return launched("gie_forward_kernel");
}

template <int V, int RC, bool kOrdered>
int launch_distinct(int cpl, const float* grad_output, const float* zonal, const float* radial,
                    const int64_t* offsets, const int64_t* order, const int64_t* radial_slot,
                    const float* inv, float* grad_zonal, float* grad_radial, float* grad_inv,
                    int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
                    int64_t channels, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
#define DPA4K_GIE_DIST(C)                                                                     \
  gie_backward_distinct_kernel<V, C, RC, kOrdered><<<grid, kBlock, 0, stream>>>(             \
      grad_output, zonal, radial, offsets, order, radial_slot, inv, grad_zonal, grad_radial,  \
      grad_inv, n_edges, n_nodes, n_rows, n_radial, channels)
  switch (cpl) {
    case 1: DPA4K_GIE_DIST(1); break;
    case 2: DPA4K_GIE_DIST(2); break;
    case 4: DPA4K_GIE_DIST(4); break;
    default: DPA4K_GIE_DIST(8); break;
  }
#undef DPA4K_GIE_DIST
  return launched("gie_backward_distinct_kernel");
}

template <int V, bool kOrdered>
int dispatch_distinct(int64_t row_chunks, int cpl, const float* grad_output, const float* zonal,
                      const float* radial, const int64_t* offsets, const int64_t* order,
                      const int64_t* radial_slot, const float* inv, float* grad_zonal,
                      float* grad_radial, float* grad_inv, int64_t n_edges, int64_t n_nodes,
                      int64_t n_rows, int64_t n_radial, int64_t channels, hipStream_t stream) {
#define DPA4K_GIE_RC(RCV)                                                                    \
  return launch_distinct<V, RCV, kOrdered>(cpl, grad_output, zonal, radial, offsets, order,  \
                                           radial_slot, inv, grad_zonal, grad_radial,        \
                                           grad_inv, n_edges, n_nodes, n_rows, n_radial,     \
                                           channels, stream)
  switch (row_chunks) {
    case 1: DPA4K_GIE_RC(1);
    case 2: DPA4K_GIE_RC(2);
    case 4: DPA4K_GIE_RC(4);
    case 8: DPA4K_GIE_RC(8);
    case 16: DPA4K_GIE_RC(16);
    case 32: DPA4K_GIE_RC(32);
    default: DPA4K_GIE_RC(64);
  }
#undef DPA4K_GIE_RC
}

template <int V>
int launch_general(int cpl, size_t lds_bytes, const float* grad_output, const float* zonal,
                   const float* radial, const int64_t* offsets, const int64_t* order,
                   const int64_t* radial_slot, const float* inv, float* grad_zonal,
                   float* grad_radial, float* grad_inv, int64_t n_edges, int64_t n_nodes,
                   int64_t n_rows, int64_t n_radial, int64_t channels, int64_t base, int64_t wc,
                   hipStream_t stream) {
#define DPA4K_GIE_GEN(C)                                                                      \
  gie_backward_general_kernel<V, C><<<launch_grid(n_nodes, 64), 64, lds_bytes,                \
                                      stream>>>(grad_output, zonal, radial, offsets, order,   \
                                                radial_slot, inv, grad_zonal, grad_radial,    \
                                                grad_inv, n_edges, n_nodes, n_rows, n_radial, \
                                                channels, base, wc)
  switch (cpl) {
    case 1: DPA4K_GIE_GEN(1); break;
    case 2: DPA4K_GIE_GEN(2); break;
    case 4: DPA4K_GIE_GEN(4); break;
    default: DPA4K_GIE_GEN(8); break;
  }
#undef DPA4K_GIE_GEN
  return launched("gie_backward_general_kernel");
}

// Bits of dpa4k_gie_group's host_info that pick a kernel: bit 2 = every slot
// feeds at most one row, bits 16..23 = the most rows that read one slot.
constexpr int32_t kSlotsDistinct = 2;
int slot_rows(int32_t slot_info) { return (slot_info >> 16) & 0xff; }
int rows_template(int rows) { return rows <= 4 ? 4 : 8; }

template <bool kOrdered>
int launch_forward_shared(int ppl, int maxr, const float* zonal, const float* radial, const int64_t* offsets,
                          const int64_t* order, const int64_t* radial_slot, const float* inv, float* out,
                          int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
                          int64_t channels, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
#define DPA4K_GIE_FWD_SHARED(P, M, B)                                                               \
  gie_forward_shared_kernel<P, M, B, kOrdered><<<grid, kBlock, 0, stream>>>(                        \
      zonal, radial, offsets, order, radial_slot, inv, out, n_edges, n_nodes, n_rows, n_radial, channels)
  const bool bcast = (channels / 4) % 16 == 0;  // groups of whole 16-lane rows
  if (ppl == 1) {
    if (bcast) {
      if (maxr == 4) DPA4K_GIE_FWD_SHARED(1, 4, true); else DPA4K_GIE_FWD_SHARED(1, 8, true);
    } else {
      if (maxr == 4) DPA4K_GIE_FWD_SHARED(1, 4, false); else DPA4K_GIE_FWD_SHARED(1, 8, false);
    }
  } else {
    if (bcast) {
      if (maxr == 4) DPA4K_GIE_FWD_SHARED(2, 4, true); else DPA4K_GIE_FWD_SHARED(2, 8, true);
    } else {
      if (maxr == 4) DPA4K_GIE_FWD_SHARED(2, 4, false); else DPA4K_GIE_FWD_SHARED(2, 8, false);
    }
  }
#undef DPA4K_GIE_FWD_SHARED
  return launched("gie_forward_shared_kernel");
}

template <int RC, bool kOrdered>
int launch_backward_shared(int maxr, const float* grad_output, const float* zonal, const float* radial,
                           const int64_t* offsets, const int64_t* order, const int64_t* radial_slot,
                           const float* inv, float* grad_zonal, float* grad_radial, float* grad_inv,
                           int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
                           int64_t channels, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
#define DPA4K_GIE_BWD_SHARED(M)                                                                       \
  gie_backward_shared_kernel<RC, M, kOrdered><<<grid, kBlock, 0, stream>>>(                          \
      grad_output, zonal, radial, offsets, order, radial_slot, inv, grad_zonal, grad_radial, grad_inv, \
      n_edges, n_nodes, n_rows, n_radial, channels)
  if (maxr == 4) DPA4K_GIE_BWD_SHARED(4); else DPA4K_GIE_BWD_SHARED(8);
#undef DPA4K_GIE_BWD_SHARED
  return launched("gie_backward_shared_kernel");
}

template <bool kOrdered>
int dispatch_backward_shared(int64_t rc, int maxr, const float* grad_output, const float* zonal,
                             const float* radial, const int64_t* offsets, const int64_t* order,
                             const int64_t* radial_slot, const float* inv, float* grad_zonal,
                             float* grad_radial, float* grad_inv, int64_t n_edges, int64_t n_nodes,
                             int64_t n_rows, int64_t n_radial, int64_t channels, hipStream_t stream) {
#define DPA4K_GIE_RC_SHARED(RCV)                                                                    \
  return launch_backward_shared<RCV, kOrdered>(maxr, grad_output, zonal, radial, offsets, order,    \
                                               radial_slot, inv, grad_zonal, grad_radial, grad_inv, \
                                               n_edges, n_nodes, n_rows, n_radial, channels, stream)
  switch (rc) {
    case 1: DPA4K_GIE_RC_SHARED(1);
    case 2: DPA4K_GIE_RC_SHARED(2);
    case 4: DPA4K_GIE_RC_SHARED(4);
    case 8: DPA4K_GIE_RC_SHARED(8);
    default: DPA4K_GIE_RC_SHARED(16);
  }
#undef DPA4K_GIE_RC_SHARED
}

template <bool kOrdered>
int dispatch_edge_lanes(const float* grad_output, const float* zonal, const float* radial, const int64_t* offsets,
                        const int64_t* order, const int64_t* radial_slot, const float* inv, float* grad_zonal,
                        float* grad_radial, float* grad_inv, int64_t n_edges, int64_t n_nodes, int64_t n_rows,
                        int64_t n_radial, int64_t channels, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
  const size_t lds = sizeof(float) * kWaves * static_cast<size_t>(n_rows * channels);
  const int rc = static_cast<int>(channels / 8);
  const int zr = n_rows <= 2 * rc ? 2 : 4;
#define DPA4K_GIE_EDGE_LANES(RC, S, ZR)                                                                 \
  gie_backward_edge_lanes_kernel<RC, S, ZR, kOrdered><<<grid, kBlock, lds, stream>>>(                  \
      grad_output, zonal, radial, offsets, order, radial_slot, inv, grad_zonal, grad_radial, grad_inv, \
      n_edges, n_nodes, n_rows, channels)
#define DPA4K_GIE_EDGE_LANES_S(RC, ZR)            \
  switch (n_radial) {                             \
    case 2: DPA4K_GIE_EDGE_LANES(RC, 2, ZR); break; \
    case 3: DPA4K_GIE_EDGE_LANES(RC, 3, ZR); break; \
    default: DPA4K_GIE_EDGE_LANES(RC, 4, ZR); break; \
  }
  if (rc == 8) {
    if (zr == 2) { DPA4K_GIE_EDGE_LANES_S(8, 2) } else { DPA4K_GIE_EDGE_LANES_S(8, 4) }
  } else {
    if (zr == 2) { DPA4K_GIE_EDGE_LANES_S(16, 2) } else { DPA4K_GIE_EDGE_LANES_S(16, 4) }
  }
#undef DPA4K_GIE_EDGE_LANES_S
#undef DPA4K_GIE_EDGE_LANES
  return launched("gie_backward_edge_lanes_kernel");
}

int check_shapes(int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
                 int64_t channels, const char* what) {
  if (n_edges < 0 || n_nodes < 0 || n_rows < 0 || n_radial < 0 || channels < 0)
    return fail(DPA4K_EINVAL, "%s: negative sizes", what);
  if (n_rows > 0 && n_radial == 0)
    return fail(DPA4K_EINVAL, "GIE radial slots are required for non-scalar rows");
  if (n_edges > 0 && n_nodes == 0) return fail(DPA4K_EINVAL, "GIE edges require destination nodes");
  if (!grid_fits(n_nodes, 64)) return fail(DPA4K_EINVAL, "GIE node count exceeds the launch limit");
  return DPA4K_OK;
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" int dpa4k_gie_zonal_scatter_forward_csr(
    const float* zonal, const float* radial, const int64_t* offsets, const int64_t* order,
    const int64_t* radial_slot, const float* inv_sqrt_deg, float* out, int64_t n_edges,
    int64_t n_nodes, int64_t n_rows, int64_t n_radial, int64_t channels, int32_t slot_info,
    dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_shapes(n_edges, n_nodes, n_rows, n_radial, channels, "GIE forward")) return s;
  if (n_nodes == 0 || channels == 0) return DPA4K_OK;
  if (offsets == nullptr || inv_sqrt_deg == nullptr || out == nullptr ||
      (n_rows > 0 && radial_slot == nullptr) ||
      (n_edges > 0 && n_rows > 0 && (zonal == nullptr || radial == nullptr)))
    return fail(DPA4K_EINVAL, "GIE forward: null pointer");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(radial) && aligned16(out);
  const int64_t row_chunks = vec4 ? channels / 4 : channels;
  // Shared slots: one pass over each edge's radial block, rows served per slot.
  const int most = slot_rows(slot_info);
  if (vec4 && !(slot_info & kSlotsDistinct) && most >= 2 && most <= 8 && n_rows >= 1 && n_rows <= 64 &&
      n_radial <= 64 && n_radial * row_chunks <= 128) {
    const int ppl = n_radial * row_chunks <= 64 ? 1 : 2;
    return order != nullptr
               ? launch_forward_shared<true>(ppl, rows_template(most), zonal, radial, offsets, order, radial_slot,
                                             inv_sqrt_deg, out, n_edges, n_nodes, n_rows, n_radial, channels,
                                             stream)
               : launch_forward_shared<false>(ppl, rows_template(most), zonal, radial, offsets, order,
                                              radial_slot, inv_sqrt_deg, out, n_edges, n_nodes, n_rows, n_radial,
                                              channels, stream);
  }
  const int64_t chunks = n_rows * row_chunks;
  const int cpl = per_lane_for(chunks);
  const int64_t window = 64 * static_cast<int64_t>(cpl);
  int64_t base = 0;
  do {
    int status;
    if (vec4)
      status = order != nullptr
                   ? launch_forward<4, true>(cpl, zonal, radial, offsets, order, radial_slot,
                                             inv_sqrt_deg, out, n_edges, n_nodes, n_rows, n_radial,
                                             channels, base, stream)
                   : launch_forward<4, false>(cpl, zonal, radial, offsets, order, radial_slot,
                                              inv_sqrt_deg, out, n_edges, n_nodes, n_rows,
                                              n_radial, channels, base, stream);
    else
      status = order != nullptr
                   ? launch_forward<1, true>(cpl, zonal, radial, offsets, order, radial_slot,
                                             inv_sqrt_deg, out, n_edges, n_nodes, n_rows, n_radial,
                                             channels, base, stream)
                   : launch_forward<1, false>(cpl, zonal, radial, offsets, order, radial_slot,
                                              inv_sqrt_deg, out, n_edges, n_nodes, n_rows,
                                              n_radial, channels, base, stream);
    if (status) return status;
    base += window;
  } while (base < chunks);
  return DPA4K_OK;
}

extern "C" int dpa4k_gie_zonal_scatter_backward_csr(
    const float* grad_output, const float* zonal, const float* radial, const int64_t* offsets,
    const int64_t* order, const int64_t* radial_slot, const float* inv_sqrt_deg,
    float* grad_zonal, float* grad_radial, float* grad_inv_sqrt_deg, int64_t n_edges,
    int64_t n_nodes, int64_t n_rows, int64_t n_radial, int64_t channels, int32_t slot_info,
    dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_shapes(n_edges, n_nodes, n_rows, n_radial, channels, "GIE backward")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr || inv_sqrt_deg == nullptr || grad_output == nullptr ||
      (n_rows > 0 && radial_slot == nullptr) ||
      (n_edges > 0 && (zonal == nullptr || radial == nullptr)))
    return fail(DPA4K_EINVAL, "GIE backward: null pointer");
  hipStream_t stream = as_stream(stream_handle);
  if (n_rows == 0 || channels == 0 || n_radial == 0) {
    // Nothing flows back: zero every requested output.
    if (grad_zonal != nullptr && n_edges * n_rows > 0)
      if (int s = zero_fill(grad_zonal, n_edges * n_rows * 4, stream)) return s;
    if (grad_radial != nullptr && n_edges * n_radial * channels > 0)
      if (int s = zero_fill(grad_radial, n_edges * n_radial * channels * 4, stream)) return s;
    if (grad_inv_sqrt_deg != nullptr)
      if (int s = zero_fill(grad_inv_sqrt_deg, n_nodes * 4, stream)) return s;
    return DPA4K_OK;
  }
  const bool vec4 = channels % 4 == 0 && aligned16(radial) && aligned16(grad_output) &&
                    (grad_radial == nullptr || aligned16(grad_radial));
  const int64_t row_chunks = vec4 ? channels / 4 : channels;
  // Register-only path: distinct slots, a power-of-two chunk count per row
  // and the whole radial block of an edge within 8 chunks per lane.
  const bool pow2 = row_chunks <= 64 && (row_chunks & (row_chunks - 1)) == 0;
  if ((slot_info & kSlotsDistinct) && pow2 && n_radial * row_chunks <= 512) {
    const int cpl = per_lane_for(n_radial * row_chunks);
    if (vec4)
      return order != nullptr
                 ? dispatch_distinct<4, true>(row_chunks, cpl, grad_output, zonal, radial, offsets,
                                              order, radial_slot, inv_sqrt_deg, grad_zonal,
                                              grad_radial, grad_inv_sqrt_deg, n_edges, n_nodes,
                                              n_rows, n_radial, channels, stream)
                 : dispatch_distinct<4, false>(row_chunks, cpl, grad_output, zonal, radial,
                                               offsets, order, radial_slot, inv_sqrt_deg,
                                               grad_zonal, grad_radial, grad_inv_sqrt_deg, n_edges,
                                               n_nodes, n_rows, n_radial, channels, stream);
    return order != nullptr
               ? dispatch_distinct<1, true>(row_chunks, cpl, grad_output, zonal, radial, offsets,
                                            order, radial_slot, inv_sqrt_deg, grad_zonal,
                                            grad_radial, grad_inv_sqrt_deg, n_edges, n_nodes,
                                            n_rows, n_radial, channels, stream)
               : dispatch_distinct<1, false>(row_chunks, cpl, grad_output, zonal, radial, offsets,
                                             order, radial_slot, inv_sqrt_deg, grad_zonal,
                                             grad_radial, grad_inv_sqrt_deg, n_edges, n_nodes,
                                             n_rows, n_radial, channels, stream);
  }
  // Shared slots, a few of them: one lane group per edge, every lane busy.
  if (vec4 && !(slot_info & kSlotsDistinct) && (channels == 64 || channels == 128) && n_radial >= 2 &&
      n_radial <= 4 && n_rows <= 4 * (channels / 8) && n_rows * channels <= kEdgeLaneRowFloats)
    return order != nullptr
               ? dispatch_edge_lanes<true>(grad_output, zonal, radial, offsets, order, radial_slot, inv_sqrt_deg,
                                           grad_zonal, grad_radial, grad_inv_sqrt_deg, n_edges, n_nodes, n_rows,
                                           n_radial, channels, stream)
               : dispatch_edge_lanes<false>(grad_output, zonal, radial, offsets, order, radial_slot, inv_sqrt_deg,
                                            grad_zonal, grad_radial, grad_inv_sqrt_deg, n_edges, n_nodes, n_rows,
                                            n_radial, channels, stream);
  // Shared slots with at most 8 rows per slot: registers only, 8 channels per lane.
  const int most = slot_rows(slot_info);
  const int64_t rc = channels / 8;
  if (vec4 && !(slot_info & kSlotsDistinct) && most >= 2 && most <= 8 && channels % 8 == 0 && rc <= 16 &&
      (rc & (rc - 1)) == 0 && n_radial * rc <= 64)
    return order != nullptr
               ? dispatch_backward_shared<true>(rc, rows_template(most), grad_output, zonal, radial, offsets, order,
                                                radial_slot, inv_sqrt_deg, grad_zonal, grad_radial,
                                                grad_inv_sqrt_deg, n_edges, n_nodes, n_rows, n_radial, channels,
                                                stream)
               : dispatch_backward_shared<false>(rc, rows_template(most), grad_output, zonal, radial, offsets,
                                                 order, radial_slot, inv_sqrt_deg, grad_zonal, grad_radial,
                                                 grad_inv_sqrt_deg, n_edges, n_nodes, n_rows, n_radial, channels,
                                                 stream);
  // General path: split the channels into windows of wc chunks so that both
  // rows x wc and slots x wc fit in 8 chunks per lane.
  const int64_t widest = n_rows > n_radial ? n_rows : n_radial;
  if (widest > 512)
    return fail(DPA4K_EINVAL, "GIE backward supports at most 512 rows and radial slots");
  int64_t wc = 512 / widest;
  if (wc > row_chunks) wc = row_chunks;
  const int cpl = per_lane_for((n_rows > n_radial ? n_rows : n_radial) * wc);
  const int vw = vec4 ? 4 : 1;
  const size_t lds_bytes = sizeof(float) * (64 * cpl + 64 * cpl * vw) +
                           sizeof(int) * static_cast<size_t>(n_radial + 1 + n_rows);
  if (lds_bytes > 64 * 1024) return fail(DPA4K_EINVAL, "GIE backward: slot map too large");
  for (int64_t c0 = 0; c0 < row_chunks; c0 += wc) {
    const int64_t this_wc = row_chunks - c0 < wc ? row_chunks - c0 : wc;
    const int status =
        vec4 ? launch_general<4>(cpl, lds_bytes, grad_output, zonal, radial, offsets, order,
                                 radial_slot, inv_sqrt_deg, grad_zonal, grad_radial,
                                 grad_inv_sqrt_deg, n_edges, n_nodes, n_rows, n_radial, channels,
                                 c0 * 4, this_wc, stream)
             : launch_general<1>(cpl, lds_bytes, grad_output, zonal, radial, offsets, order,
                                 radial_slot, inv_sqrt_deg, grad_zonal, grad_radial,
                                 grad_inv_sqrt_deg, n_edges, n_nodes, n_rows, n_radial, channels,
                                 c0, this_wc, stream);
    if (status) return status;
  }
  return DPA4K_OK;
}

extern "C" size_t dpa4k_gie_workspace_size(int64_t n_edges, int64_t n_nodes) {
  if (n_nodes <= 0) return 0;
  return round_up_256(static_cast<size_t>(n_nodes + 1) * 8) +
         round_up_256(static_cast<size_t>(n_edges > 0 ? n_edges : 1) * 8) +
         dpa4k_gie_group_workspace_size(n_edges, n_nodes);
}

namespace {
struct GroupedCsr {
  int64_t* offsets;
  int64_t* order;  // NULL when dst is already grouped
  int info;
};

int group_into(const int64_t* dst, const int64_t* radial_slot, int64_t n_edges, int64_t n_nodes,
               int64_t n_rows, int64_t n_radial, void* workspace, size_t workspace_bytes,
               dpa4k_stream_t stream, GroupedCsr& out) {
  const size_t needed = dpa4k_gie_workspace_size(n_edges, n_nodes);
  if (workspace == nullptr || workspace_bytes < needed)
    return fail(DPA4K_EWORKSPACE, "GIE: workspace of %zu bytes is smaller than %zu", workspace_bytes,
                needed);
  Carver carver{static_cast<char*>(workspace), workspace_bytes};
  out.offsets = carver.take<int64_t>(static_cast<size_t>(n_nodes + 1));
  int64_t* order = carver.take<int64_t>(static_cast<size_t>(n_edges > 0 ? n_edges : 1));
  void* rest = static_cast<char*>(workspace) + carver.used;
  int32_t info = 0;
  if (int s = dpa4k_gie_group(dst, radial_slot, n_edges, n_nodes, n_rows, n_radial, out.offsets,
                              order, &info, rest, workspace_bytes - carver.used, stream))
    return s;
  out.order = (info & 1) ? nullptr : order;
  out.info = info;
  return DPA4K_OK;
}
}  // namespace

extern "C" int dpa4k_gie_zonal_scatter_forward(const float* zonal, const float* radial,
                                               const int64_t* dst, const int64_t* radial_slot,
                                               const float* inv_sqrt_deg, float* out,
                                               int64_t n_edges, int64_t n_nodes, int64_t n_rows,
                                               int64_t n_radial, int64_t channels, void* workspace,
                                               size_t workspace_bytes, dpa4k_stream_t stream) {
  clear_error();
  if (int s = check_shapes(n_edges, n_nodes, n_rows, n_radial, channels, "GIE forward")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  GroupedCsr csr{};
  if (int s = group_into(dst, radial_slot, n_edges, n_nodes, n_rows, n_radial, workspace,
                         workspace_bytes, stream, csr))
    return s;
  return dpa4k_gie_zonal_scatter_forward_csr(zonal, radial, csr.offsets, csr.order, radial_slot,
                                             inv_sqrt_deg, out, n_edges, n_nodes, n_rows, n_radial,
                                             channels, csr.info, stream);
}

extern "C" int dpa4k_gie_zonal_scatter_backward(
    const float* grad_output, const float* zonal, const float* radial, const int64_t* dst,
    const int64_t* radial_slot, const float* inv_sqrt_deg, float* grad_zonal, float* grad_radial,
    float* grad_inv_sqrt_deg, int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
    int64_t channels, void* workspace, size_t workspace_bytes, dpa4k_stream_t stream) {
  clear_error();
  if (int s = check_shapes(n_edges, n_nodes, n_rows, n_radial, channels, "GIE backward")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  GroupedCsr csr{};
  if (int s = group_into(dst, radial_slot, n_edges, n_nodes, n_rows, n_radial, workspace,
                         workspace_bytes, stream, csr))
    return s;
  return dpa4k_gie_zonal_scatter_backward_csr(
      grad_output, zonal, radial, csr.offsets, csr.order, radial_slot, inv_sqrt_deg, grad_zonal,
      grad_radial, grad_inv_sqrt_deg, n_edges, n_nodes, n_rows, n_radial, channels, csr.info,
      stream);
}

namespace dpa4k {
namespace {

template <bool kOrdered>
int launch_gie_rmsnorm(int cpl, const float* zonal, const float* radial, const int64_t* offsets,
                       const int64_t* order, const int64_t* radial_slot, const float* inv, const float* scale,
                       float eps, float* y, float* x_out, float* inverse_rms, int64_t n_edges, int64_t n_nodes,
                       int64_t n_rows, int64_t n_radial, int64_t channels, hipStream_t stream) {
  const dim3 grid = launch_grid((n_nodes + kWaves - 1) / kWaves, kBlock);
#define DPA4K_GIE_RMS(C)                                                                              \
  gie_rmsnorm_forward_kernel<C, kOrdered><<<grid, kBlock, 0, stream>>>(                              \
      zonal, radial, offsets, order, radial_slot, inv, scale, eps, y, x_out, inverse_rms, n_edges, n_nodes, \
      n_rows, n_radial, channels)
  switch (cpl) {
    case 1: DPA4K_GIE_RMS(1); break;
    case 2: DPA4K_GIE_RMS(2); break;
    case 4: DPA4K_GIE_RMS(4); break;
    default: DPA4K_GIE_RMS(8); break;
  }
#undef DPA4K_GIE_RMS
  return launched("gie_rmsnorm_forward_kernel");
}

}  // namespace
}  // namespace dpa4k

extern "C" int dpa4k_gie_rmsnorm_supported(int64_t n_rows, int64_t channels) {
  return channels > 0 && channels % 4 == 0 && n_rows >= 0 && (n_rows + 1) * (channels / 4) <= 512 ? 1 : 0;
}

extern "C" int dpa4k_gie_rmsnorm_forward_csr(const float* zonal, const float* radial, const int64_t* offsets,
                                             const int64_t* order, const int64_t* radial_slot,
                                             const float* inv_sqrt_deg, const float* scale, float eps, float* y,
                                             float* x_out, float* inverse_rms, int64_t n_edges, int64_t n_nodes,
                                             int64_t n_rows, int64_t n_radial, int64_t channels,
                                             dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_shapes(n_edges, n_nodes, n_rows, n_radial, channels, "GIE RMSNorm")) return s;
  if (!dpa4k_gie_rmsnorm_supported(n_rows, channels))
    return fail(DPA4K_EINVAL, "GIE RMSNorm: rows of (n_rows + 1) * channels floats need channels %% 4 == 0 and "
                              "at most 2048 floats");
  if (!(eps > 0.0f) || eps == INFINITY) return fail(DPA4K_EINVAL, "GIE RMSNorm: eps must be finite and positive");
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr || inv_sqrt_deg == nullptr || y == nullptr || inverse_rms == nullptr ||
      (n_rows > 0 && radial_slot == nullptr) ||
      (n_edges > 0 && n_rows > 0 && (zonal == nullptr || radial == nullptr)))
    return fail(DPA4K_EINVAL, "GIE RMSNorm: null pointer");
  if (!aligned16(y) || (x_out != nullptr && !aligned16(x_out)) || (radial != nullptr && !aligned16(radial)) ||
      (scale != nullptr && !aligned16(scale)))
    return fail(DPA4K_EINVAL, "GIE RMSNorm: radial, scale and outputs must be 16-byte aligned");
  hipStream_t stream = as_stream(stream_handle);
  const int cpl = per_lane_for((n_rows + 1) * (channels / 4));
  return order != nullptr
             ? launch_gie_rmsnorm<true>(cpl, zonal, radial, offsets, order, radial_slot, inv_sqrt_deg, scale, eps, y,
                                        x_out, inverse_rms, n_edges, n_nodes, n_rows, n_radial, channels, stream)
             : launch_gie_rmsnorm<false>(cpl, zonal, radial, offsets, order, radial_slot, inv_sqrt_deg, scale, eps,
                                         y, x_out, inverse_rms, n_edges, n_nodes, n_rows, n_radial, channels, stream);
}

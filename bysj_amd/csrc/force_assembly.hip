// force_assembly (python/kernels/segment.py:314-332, csrc/force_assembly.cpp:106
// of the reference):
//   F_k = sum_{dst(e)=k} g_e - sum_{src(e)=k} g_e
//   W_k = sum_{src(e)=k} -(g_e outer v_e)           (row-major 3x3)
// as a gather over two CSR views: the natural (dst-grouped) edge order and
// the src_order permutation.  No atomics, no materialised (E, 9) product.
//
// Layout: a group of G = 32 lanes owns one atom (8 atoms per 256-thread
// workgroup).  Every load of the atom is issued before any arithmetic, and
// none sits in a branch:
//   * the source side reads its src_order ids (kSrcRounds per lane), then
//     gathers whole 12- or 24-byte rows g_e, v_e for them;
//   * the destination side streams the contiguous span grad_edge[3*begin,
//     3*end) in 16-byte chunks (kDstBytes per lane), the component of the
//     segment's scalar q being q mod 3.
// Both go through buffer views (32-bit offsets, one register per address,
// zeros past the end); the gathered rows too while the arrays are under
// 2 GiB.  Longer segments continue in loops.  Every lane accumulates all twelve
// outputs in double precision, a fixed DPP/swizzle butterfly over the 32
// lanes produces the totals and lanes 0..11 store one component each.  The
// summation order depends only on the CSR, so results are reproducible;
// fp32 inputs round once on output (products of two floats are exact in
// double), fp64 inputs keep double outputs.
//
// The source side is a random gather when atom numbering has no spatial
// locality: each 12-byte row then costs a whole cache line, which bounds the
// kernel well below the HBM roofline of its algorithmic bytes.
//
// The planned path (dpa4k_force_assembly_plan, once per graph) removes that
// gather from HBM.  The plan partitions the atoms into <= 256 contiguous
// buckets and the edges into tiles of kPlanTile, and sorts the edges stably
// by (tile, source bucket) with the library's counting sort.  Each call then
//   pass 1  streams the rows (g_e, v_e) in edge order into a buffer in that
//           sorted order: the reads are one contiguous stream, and the
//           writes of a tile stay inside its own kPlanTile rows of the
//           buffer, which the tile's blocks (one XCD) complete in their L2;
//   pass 2  is the kernel above with its source rows read from that buffer
//           through 32-bit positions: one 24- or 48-byte row per edge.  The
//           rows one bucket's atoms need lie in one short run per tile, so
//           the blocks of a bucket (one XCD: blocks are dealt to XCDs in
//           contiguous atom ranges) gather from a few hundred KB that their
//           L2 holds instead of from the whole input.
// The accumulation order is the unplanned kernel's, so both give the same
// bits.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kLogGroup = 5;
constexpr int kGroup = 1 << kLogGroup;
constexpr int kAtoms = kBlock / kGroup;
constexpr int kSrcRounds = 3;  // source rows per lane held in registers (96 per atom)
constexpr int kDstBytes = 48;  // destination bytes per lane held in registers (384 floats or 192 doubles per atom)

template <typename T>
struct Row3 {
  T x, y, z;
};

template <typename T>
__device__ __forceinline__ Row3<T> load_row(const T* __restrict__ base, int64_t e) {
  return *reinterpret_cast<const Row3<T>*>(base + 3 * e);
}

// 16 bytes of T from a buffer view (zeros past its end).
template <typename T>
struct Chunk {
  T v[16 / sizeof(T)];
};

template <typename T>
__device__ __forceinline__ Chunk<T> view_chunk(BufferView view, uint32_t offset) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(offset), 0, 0);
  return __builtin_bit_cast(Chunk<T>, raw);
}

__device__ __forceinline__ int64_t view_i64(BufferView view, uint32_t offset) {
  return __builtin_bit_cast(int64_t, __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(offset), 0, 0));
}

// Row e of a [E, 3] array through a view of the whole array; offset kNoRow reads zeros.
template <typename T>
__device__ __forceinline__ Row3<T> view_row(BufferView view, uint32_t offset) {
  if constexpr (sizeof(T) == 4) {
    // three dword loads: this toolchain lowers the 96-bit buffer-load builtin
    // to a single-dword load, dropping y and z
    return Row3<T>{buffer_load_f32(view, offset), buffer_load_f32(view, offset + 4u),
                   buffer_load_f32(view, offset + 8u)};
  } else {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(offset), 0, 0);
    const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(offset + 8u), 0, 0);
    const u32x2 c = __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(offset + 16u), 0, 0);
    return Row3<T>{__builtin_bit_cast(double, a), __builtin_bit_cast(double, b), __builtin_bit_cast(double, c)};
  }
}

// Adds a destination-side scalar: element q of the segment's 3 * degree
// scalars is component q mod 3 of its edge's row.
__device__ __forceinline__ void add_component(double (&acc)[12], int q, double value) {
  const int component = q % 3;
  acc[0] += component == 0 ? value : 0.0;
  acc[1] += component == 1 ? value : 0.0;
  acc[2] += component == 2 ? value : 0.0;
}

template <typename T>
__device__ __forceinline__ void add_source(double (&acc)[12], const Row3<T>& g, const Row3<T>& v) {
  const double g0 = g.x, g1 = g.y, g2 = g.z, v0 = v.x, v1 = v.y, v2 = v.z;
  acc[0] -= g0;
  acc[1] -= g1;
  acc[2] -= g2;
  acc[3] -= g0 * v0;
  acc[4] -= g0 * v1;
  acc[5] -= g0 * v2;
  acc[6] -= g1 * v0;
  acc[7] -= g1 * v1;
  acc[8] -= g1 * v2;
  acc[9] -= g2 * v0;
  acc[10] -= g2 * v1;
  acc[11] -= g2 * v2;
}

// Row (g_e, v_e) of the planned path's bucketed buffer ([E, 6] of T); offset
// kNoRow reads zeros.  Three 8-byte loads (f32) or three 16-byte loads (f64).
// The f32 halves are split from a 64-bit integer: with per-element access to
// the builtin's two-dword vector this toolchain emits a single-dword load and
// the high halves read garbage.
template <typename T>
__device__ __forceinline__ void view_pair(BufferView view, uint32_t offset, Row3<T>& g, Row3<T>& v) {
  if constexpr (sizeof(T) == 4) {
    auto pair = [&](uint32_t at, float& low, float& high) {
      const uint64_t bits = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(view, static_cast<int>(at), 0, 0));
      low = __builtin_bit_cast(float, static_cast<uint32_t>(bits));
      high = __builtin_bit_cast(float, static_cast<uint32_t>(bits >> 32));
    };
    pair(offset, g.x, g.y);
    pair(offset == kNoRow ? kNoRow : offset + 8u, g.z, v.x);
    pair(offset == kNoRow ? kNoRow : offset + 16u, v.y, v.z);
  } else {
    typedef double f64x2 __attribute__((ext_vector_type(2)));
    const f64x2 a = __builtin_bit_cast(f64x2, __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(offset), 0, 0));
    const f64x2 b = __builtin_bit_cast(
        f64x2, __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(offset == kNoRow ? kNoRow : offset + 16u), 0, 0));
    const f64x2 c = __builtin_bit_cast(
        f64x2, __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(offset == kNoRow ? kNoRow : offset + 32u), 0, 0));
    g = Row3<T>{a.x, a.y, b.x};
    v = Row3<T>{b.y, c.x, c.y};
  }
}

// kRowViews: the gathered rows' array is under 2^31 bytes, so they are
// addressed through 32-bit offsets into a view of the whole array (one
// register per address, zeros for a lane without a row); otherwise through
// pointers at a clamped id, with the rows of invalid slots zeroed afterwards.
// kPlanned: the source slots hold int32 positions (src_pos) into the bucketed
// buffer `rows` ([E, 6]: g_e then v_e) instead of int64 edge ids (src_order)
// into grad_edge and edge_vec.
template <typename T, bool kRowViews, bool kPlanned>
__global__ __launch_bounds__(kBlock) void force_assembly_kernel(
    const T* __restrict__ grad_edge, const T* __restrict__ edge_vec,
    const int64_t* __restrict__ dst_offsets, const int64_t* __restrict__ src_offsets,
    const int64_t* __restrict__ src_order, const int32_t* __restrict__ src_pos, const T* __restrict__ rows,
    T* __restrict__ force, T* __restrict__ virial, int64_t n_edges, int64_t n_nodes) {
  constexpr int kPer = 16 / sizeof(T);          // T per 16-byte chunk
  constexpr int kDstChunks = kDstBytes / 16;     // chunks per lane
  // Neighbouring atoms gather rows from the same destination segments when
  // atom numbering follows space, so each XCD takes a contiguous atom range
  // (of each grid row, when the atoms need more than one row of blocks).
  const int64_t block = static_cast<int64_t>(blockIdx.y) * gridDim.x + xcd_block(blockIdx.x, gridDim.x);
  const int64_t atom = block * kAtoms + (threadIdx.x >> kLogGroup);
  if (atom >= n_nodes) return;
  const int lane = threadIdx.x & (kGroup - 1);
  if (n_edges == 0) {  // no edges: every sum is empty (and no index below is valid)
    if (lane < 3)
      force[atom * 3 + lane] = T(0);
    else if (lane < 12)
      virial[atom * 9 + (lane - 3)] = T(0);
    return;
  }
  int64_t dst_begin, dst_end, src_begin, src_end;
  segment_bounds(dst_offsets, atom, n_edges, dst_begin, dst_end);
  segment_bounds(src_offsets, atom, n_edges, src_begin, src_end);
  const int64_t src_count = src_end - src_begin;
  const int64_t dst_scalars = 3 * (dst_end - dst_begin);

  // ---- issue the loads ----
  // No load sits in a branch: a load inside a divergent branch is waited
  // for before the branch closes, and the round trips this section overlaps
  // would run one after another.  The two atoms of a wave are consecutive,
  // so their segments are adjacent in both CSRs: one view per CSR, based at
  // the wave's first segment, serves both, and each lane reads its own
  // window at a 32-bit offset (views read zeros past their ends).  A window
  // whose offset would not fit (a neighbouring segment of some 10^8 edges)
  // is left to the loops below.  The source ids go first, so that waiting
  // for them leaves the destination chunks in flight while the rows they
  // name are requested.
  constexpr int64_t kWindowBytes = 4096;  // covers both windows of a lane
  const int64_t wave_dst = uniform_i64(dst_begin), wave_src = uniform_i64(src_begin);
  constexpr int64_t kSlotBytes = kPlanned ? 4 : 8;
  const int64_t dst_base = (dst_begin - wave_dst) * 3 * static_cast<int64_t>(sizeof(T));
  const int64_t src_base = (src_begin - wave_src) * kSlotBytes;
  const bool dst_window = dst_base >= 0 && dst_base < int64_t(kNoRow) - kWindowBytes;
  const bool src_window = src_base >= 0 && src_base < int64_t(kNoRow) - kWindowBytes;

  const BufferView slots = kPlanned ? buffer_view(src_pos + wave_src, (n_edges - wave_src) * 4)
                                    : buffer_view(src_order + wave_src, (n_edges - wave_src) * 8);
  int64_t edge[kSrcRounds];  // edge ids, or positions in `rows` when planned
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) {
    const uint32_t offset =
        src_window ? static_cast<uint32_t>(src_base) + static_cast<uint32_t>(r * kGroup + lane) * kSlotBytes : kNoRow;
    if constexpr (kPlanned)
      edge[r] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(slots, static_cast<int>(offset), 0, 0));
    else
      edge[r] = view_i64(slots, offset);
  }
  const BufferView dst_view =
      buffer_view(grad_edge + 3 * wave_dst, 3 * (n_edges - wave_dst) * static_cast<int64_t>(sizeof(T)));
  // Chunk r of a lane holds scalars [q, q + kPer) of the segment, q = (r * kGroup + lane) * kPer.  A chunk
  // that straddles the end of the array reads its dwords inside the view and zeros past it: gfx950 checks
  // the range of a raw buffer load dword by dword.
  Chunk<T> d[kDstChunks];
#pragma unroll
  for (int r = 0; r < kDstChunks; ++r) {
    const uint32_t q = static_cast<uint32_t>(r * kGroup + lane) * kPer;
    d[r] = view_chunk<T>(dst_view, dst_window ? static_cast<uint32_t>(dst_base) + q * sizeof(T) : kNoRow);
  }
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) {
    const bool valid = src_window && r * kGroup + lane < src_count &&
                       static_cast<uint64_t>(edge[r]) < static_cast<uint64_t>(n_edges);
    edge[r] = valid ? edge[r] : -1;
  }
  Row3<T> g[kSrcRounds], v[kSrcRounds];
  if constexpr (kPlanned && kRowViews) {
    const BufferView row_view = buffer_view(rows, 6 * n_edges * static_cast<int64_t>(sizeof(T)));
#pragma unroll
    for (int r = 0; r < kSrcRounds; ++r) {
      const uint32_t offset = edge[r] >= 0 ? static_cast<uint32_t>(edge[r]) * (6u * sizeof(T)) : kNoRow;
      view_pair<T>(row_view, offset, g[r], v[r]);
    }
  } else if constexpr (kPlanned) {
#pragma unroll
    for (int r = 0; r < kSrcRounds; ++r) {
      const int64_t e = edge[r] >= 0 ? edge[r] : 0;
      g[r] = load_row(rows, 2 * e);
      v[r] = load_row(rows, 2 * e + 1);
    }
#pragma unroll
    for (int r = 0; r < kSrcRounds; ++r) {
      const bool valid = edge[r] >= 0;
      g[r] = Row3<T>{valid ? g[r].x : T(0), valid ? g[r].y : T(0), valid ? g[r].z : T(0)};
      v[r] = Row3<T>{valid ? v[r].x : T(0), valid ? v[r].y : T(0), valid ? v[r].z : T(0)};
    }
  } else if constexpr (kRowViews) {
    const int64_t bytes = 3 * n_edges * static_cast<int64_t>(sizeof(T));
    const BufferView g_view = buffer_view(grad_edge, bytes), v_view = buffer_view(edge_vec, bytes);
#pragma unroll
    for (int r = 0; r < kSrcRounds; ++r) {
      const uint32_t offset = edge[r] >= 0 ? static_cast<uint32_t>(edge[r]) * (3u * sizeof(T)) : kNoRow;
      g[r] = view_row<T>(g_view, offset);
      v[r] = view_row<T>(v_view, offset);
    }
  } else {
#pragma unroll
    for (int r = 0; r < kSrcRounds; ++r) {
      const int64_t e = edge[r] >= 0 ? edge[r] : 0;
      g[r] = load_row(grad_edge, e);
      v[r] = load_row(edge_vec, e);
    }
#pragma unroll
    for (int r = 0; r < kSrcRounds; ++r) {
      const bool valid = edge[r] >= 0;
      g[r] = Row3<T>{valid ? g[r].x : T(0), valid ? g[r].y : T(0), valid ? g[r].z : T(0)};
      v[r] = Row3<T>{valid ? v[r].x : T(0), valid ? v[r].y : T(0), valid ? v[r].z : T(0)};
    }
  }

  // ---- accumulate ----
  double acc[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) acc[i] = 0.0;
#pragma unroll
  for (int r = 0; r < kDstChunks; ++r)
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int q = (r * kGroup + lane) * kPer + i;  // the window ends well before 2^31 scalars
      add_component(acc, q, q < dst_scalars ? static_cast<double>(d[r].v[i]) : 0.0);
    }
  const T* dst_row = grad_edge + 3 * dst_begin;
  for (int64_t q = (dst_window ? kDstChunks * kGroup * kPer : 0) + lane; q < dst_scalars; q += kGroup)
    add_component(acc, static_cast<int>(q % 3), static_cast<double>(dst_row[q]));
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) add_source(acc, g[r], v[r]);
  for (int64_t slot = src_begin + (src_window ? kSrcRounds * kGroup : 0) + lane; slot < src_end; slot += kGroup) {
    if constexpr (kPlanned) {
      const int64_t at = src_pos[slot];
      if (static_cast<uint64_t>(at) >= static_cast<uint64_t>(n_edges)) continue;
      add_source(acc, load_row(rows, 2 * at), load_row(rows, 2 * at + 1));
    } else {
      const int64_t e = edge_of<true>(src_order, slot, n_edges);
      if (e < 0) continue;
      add_source(acc, load_row(grad_edge, e), load_row(edge_vec, e));
    }
  }

#pragma unroll
  for (int i = 0; i < 12; ++i) acc[i] = group_sum<kGroup>(acc[i]);

  double mine = acc[0];
#pragma unroll
  for (int i = 1; i < 12; ++i) mine = lane == i ? acc[i] : mine;
  if (lane < 3)
    force[atom * 3 + lane] = static_cast<T>(mine);
  else if (lane < 12)
    virial[atom * 9 + (lane - 3)] = static_cast<T>(mine);
}

template <typename T>
int run(const T* grad_edge, const T* edge_vec, const int64_t* dst_offsets,
        const int64_t* src_offsets, const int64_t* src_order, T* force, T* virial,
        int64_t n_edges, int64_t n_nodes, dpa4k_stream_t stream_handle) {
  clear_error();
  if (n_edges < 0) return fail(DPA4K_EINVAL, "force assembly: negative edge count");
  if (n_nodes <= 0) return fail(DPA4K_EINVAL, "force assembly requires at least one atom");
  if (!grid_fits((n_nodes + kAtoms - 1) / kAtoms, kBlock))
    return fail(DPA4K_EINVAL, "force assembly atom count exceeds the launch limit");
  if (dst_offsets == nullptr || src_offsets == nullptr || force == nullptr || virial == nullptr ||
      (n_edges > 0 && (grad_edge == nullptr || edge_vec == nullptr || src_order == nullptr)))
    return fail(DPA4K_EINVAL, "force assembly: null pointer");
  hipStream_t stream = as_stream(stream_handle);
  const dim3 grid = launch_grid((n_nodes + kAtoms - 1) / kAtoms, kBlock);
  if (3 * n_edges * static_cast<int64_t>(sizeof(T)) < (int64_t(1) << 31))
    force_assembly_kernel<T, true, false><<<grid, kBlock, 0, stream>>>(
        grad_edge, edge_vec, dst_offsets, src_offsets, src_order, nullptr, nullptr, force, virial, n_edges, n_nodes);
  else
    force_assembly_kernel<T, false, false><<<grid, kBlock, 0, stream>>>(
        grad_edge, edge_vec, dst_offsets, src_offsets, src_order, nullptr, nullptr, force, virial, n_edges, n_nodes);
  return launched("force_assembly_kernel");
}

// ---------------------------------------------------------------------------
// planned path
// ---------------------------------------------------------------------------

unsigned int grid_stride_blocks(int64_t items) {
  const int64_t wanted = (items + 255) / 256;
  return static_cast<unsigned int>(wanted < 1 ? 1 : (wanted > 8192 ? 8192 : wanted));
}

constexpr int64_t kPlanTile = 8192;   // edges per pass-1 tile
constexpr int64_t kPlanBuckets = 256;  // most source-atom buckets

// Tiles and buckets of a graph: `bucket_atoms` consecutive atoms per bucket.
struct PlanShape {
  int64_t tiles, buckets, bucket_atoms;
};

PlanShape plan_shape(int64_t n_edges, int64_t n_nodes) {
  PlanShape shape;
  shape.tiles = (n_edges + kPlanTile - 1) / kPlanTile;
  const int64_t wanted = n_nodes < kPlanBuckets ? n_nodes : kPlanBuckets;
  shape.bucket_atoms = (n_nodes + wanted - 1) / wanted;
  shape.buckets = (n_nodes + shape.bucket_atoms - 1) / shape.bucket_atoms;
  return shape;
}

// The plan's arrays, carved in this order from the caller's buffer.
struct PlanArrays {
  int32_t* edge_row;   // [E] row of each edge in the (tile, bucket)-sorted buffer
  int32_t* src_pos;    // [E] row of each source-CSR slot (-1: invalid src_order entry)
  void* rows;          // [E, 6] of the value type
};

bool carve_plan(void* plan, size_t plan_bytes, int64_t n_edges, int64_t value_bytes, PlanArrays& out) {
  Carver carver{static_cast<char*>(plan), plan_bytes};
  const size_t count = static_cast<size_t>(n_edges > 0 ? n_edges : 1);
  out.edge_row = carver.take<int32_t>(count);
  out.src_pos = carver.take<int32_t>(count);
  out.rows = value_bytes == 8 ? static_cast<void*>(carver.take<double>(6 * count))
                              : static_cast<void*>(carver.take<float>(6 * count));
  return out.edge_row && out.src_pos && out.rows;
}

struct PlanScratch {
  int64_t *key, *order, *tile_offsets;
  int32_t* status;
  void* sort;
  size_t sort_bytes;
};

size_t plan_sort_bytes(int64_t n_edges, const PlanShape& shape) {
  return dpa4k_group_by_key_workspace_size(n_edges, shape.tiles * shape.buckets);
}

bool carve_scratch(void* workspace, size_t bytes, int64_t n_edges, const PlanShape& shape, PlanScratch& out) {
  Carver carver{static_cast<char*>(workspace), bytes};
  const size_t count = static_cast<size_t>(n_edges > 0 ? n_edges : 1);
  const size_t cells = static_cast<size_t>(shape.tiles * shape.buckets);
  out.key = carver.take<int64_t>(count);
  out.order = carver.take<int64_t>(count);
  out.tile_offsets = carver.take<int64_t>(cells + 1);
  out.status = carver.take<int32_t>(1);
  out.sort_bytes = plan_sort_bytes(n_edges, shape);
  out.sort = carver.take<char>(out.sort_bytes);
  return out.key && out.order && out.tile_offsets && out.status && out.sort;
}

// key[q] = tile(e) * buckets + bucket(src of e) for the edge e = src_order[q]
// of every source slot q; the atom of slot q is found by a binary search of
// src_offsets.  Edges no valid slot names keep key tile(e) * buckets.
__global__ __launch_bounds__(256) void plan_default_keys_kernel(int64_t* __restrict__ key, int64_t n_edges,
                                                                int64_t buckets) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n_edges; e += stride)
    key[e] = (e / kPlanTile) * buckets;
}

__global__ __launch_bounds__(256) void plan_source_keys_kernel(const int64_t* __restrict__ src_offsets,
                                                               const int64_t* __restrict__ src_order,
                                                               int64_t* __restrict__ key, int64_t n_edges,
                                                               int64_t n_nodes, int64_t buckets,
                                                               int64_t bucket_atoms) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < n_edges; q += stride) {
    int64_t low = 0, high = n_nodes;  // the last atom k with src_offsets[k] <= q
    while (high - low > 1) {
      const int64_t mid = (low + high) / 2;
      if (src_offsets[mid] <= q) low = mid; else high = mid;
    }
    const int64_t e = src_order[q];
    if (static_cast<uint64_t>(e) < static_cast<uint64_t>(n_edges))
      key[e] = (e / kPlanTile) * buckets + low / bucket_atoms;
  }
}

// Sorted slot p (tile-major, then bucket, then edge) is row p of the
// buffer: record that row for its edge.
__global__ __launch_bounds__(256) void plan_rows_kernel(const int64_t* __restrict__ order,
                                                        int32_t* __restrict__ edge_row, int64_t n_edges) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n_edges; p += stride)
    edge_row[order[p]] = static_cast<int32_t>(p);
}

__global__ __launch_bounds__(256) void plan_source_positions_kernel(const int64_t* __restrict__ src_order,
                                                                    const int32_t* __restrict__ position,
                                                                    int32_t* __restrict__ src_pos, int64_t n_edges) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < n_edges; q += stride) {
    const int64_t e = src_order[q];
    src_pos[q] = static_cast<uint64_t>(e) < static_cast<uint64_t>(n_edges) ? position[e] : -1;
  }
}

// Pass 1: edge e's row (g_e, v_e) to row edge_row[e] of the buffer, one
// edge per thread.  The reads are one contiguous stream; the writes of a
// tile stay inside the tile's own kPlanTile rows, and the blocks of a tile
// (consecutive logical blocks) run on one XCD, so its L2 assembles whole
// lines before they are written back.  (Measured against the transposed
// form, contiguous writes of rows gathered inside the tile: slightly
// slower.)
template <typename T>
__global__ __launch_bounds__(256) void force_place_rows_kernel(const T* __restrict__ grad_edge,
                                                               const T* __restrict__ edge_vec,
                                                               const int32_t* __restrict__ edge_row,
                                                               T* __restrict__ rows, int64_t n_edges) {
  const int64_t block = static_cast<int64_t>(blockIdx.y) * gridDim.x + xcd_block(blockIdx.x, gridDim.x);
  const int64_t e = block * 256 + threadIdx.x;
  if (e >= n_edges) return;
  const int64_t to = edge_row[e];
  const Row3<T> g = load_row(grad_edge, e);
  const Row3<T> v = load_row(edge_vec, e);
  *reinterpret_cast<Row3<T>*>(rows + 6 * to) = g;
  *reinterpret_cast<Row3<T>*>(rows + 6 * to + 3) = v;
}

size_t plan_bytes_for(int64_t n_edges, int64_t value_bytes) {
  const size_t count = static_cast<size_t>(n_edges > 0 ? n_edges : 1);
  return 2 * round_up_256(count * 4) + round_up_256(count * 6 * static_cast<size_t>(value_bytes));
}

int check_plan_shapes(int64_t n_edges, int64_t n_nodes, const char* what) {
  if (n_edges < 0) return fail(DPA4K_EINVAL, "%s: negative edge count", what);
  if (n_nodes <= 0) return fail(DPA4K_EINVAL, "%s requires at least one atom", what);
  if (n_edges > int64_t(0x7fffffff)) return fail(DPA4K_EINVAL, "%s: more than 2^31 - 1 edges", what);
  return DPA4K_OK;
}

template <typename T>
int run_planned(const T* grad_edge, const T* edge_vec, const int64_t* dst_offsets, const int64_t* src_offsets,
                T* force, T* virial, int64_t n_edges, int64_t n_nodes, void* plan, size_t plan_bytes,
                dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_plan_shapes(n_edges, n_nodes, "planned force assembly")) return s;
  if (!grid_fits((n_nodes + kAtoms - 1) / kAtoms, kBlock))
    return fail(DPA4K_EINVAL, "force assembly atom count exceeds the launch limit");
  if (dst_offsets == nullptr || src_offsets == nullptr || force == nullptr || virial == nullptr || plan == nullptr ||
      (n_edges > 0 && (grad_edge == nullptr || edge_vec == nullptr)))
    return fail(DPA4K_EINVAL, "planned force assembly: null pointer");
  if (plan_bytes < plan_bytes_for(n_edges, sizeof(T)))
    return fail(DPA4K_EINVAL, "planned force assembly: plan of %zu bytes is smaller than %zu", plan_bytes,
                plan_bytes_for(n_edges, sizeof(T)));
  PlanArrays arrays;
  if (!carve_plan(plan, plan_bytes, n_edges, sizeof(T), arrays))
    return fail(DPA4K_EINVAL, "planned force assembly: plan too small");
  hipStream_t stream = as_stream(stream_handle);
  T* rows = static_cast<T*>(arrays.rows);
  if (n_edges > 0) {
    force_place_rows_kernel<T><<<launch_grid((n_edges + 255) / 256, 256), 256, 0, stream>>>(
        grad_edge, edge_vec, arrays.edge_row, rows, n_edges);
    if (int s = launched("force_place_rows_kernel")) return s;
  }
  const dim3 grid = launch_grid((n_nodes + kAtoms - 1) / kAtoms, kBlock);
  if (6 * n_edges * static_cast<int64_t>(sizeof(T)) < (int64_t(1) << 31))
    force_assembly_kernel<T, true, true><<<grid, kBlock, 0, stream>>>(
        grad_edge, edge_vec, dst_offsets, src_offsets, nullptr, arrays.src_pos, rows, force, virial, n_edges, n_nodes);
  else
    force_assembly_kernel<T, false, true><<<grid, kBlock, 0, stream>>>(
        grad_edge, edge_vec, dst_offsets, src_offsets, nullptr, arrays.src_pos, rows, force, virial, n_edges, n_nodes);
  return launched("force_assembly_kernel");
}

}  // namespace
}  // namespace dpa4k

extern "C" int dpa4k_force_assembly_f32(const float* grad_edge, const float* edge_vec,
                                        const int64_t* dst_offsets, const int64_t* src_offsets,
                                        const int64_t* src_order, float* force, float* virial,
                                        int64_t n_edges, int64_t n_nodes,
                                        dpa4k_stream_t stream) {
  return dpa4k::run<float>(grad_edge, edge_vec, dst_offsets, src_offsets, src_order, force, virial,
                           n_edges, n_nodes, stream);
}

extern "C" int dpa4k_force_assembly_f64(const double* grad_edge, const double* edge_vec,
                                        const int64_t* dst_offsets, const int64_t* src_offsets,
                                        const int64_t* src_order, double* force, double* virial,
                                        int64_t n_edges, int64_t n_nodes,
                                        dpa4k_stream_t stream) {
  return dpa4k::run<double>(grad_edge, edge_vec, dst_offsets, src_offsets, src_order, force,
                            virial, n_edges, n_nodes, stream);
}

extern "C" size_t dpa4k_force_assembly_plan_size(int64_t n_edges, int64_t n_nodes, int64_t value_bytes) {
  (void)n_nodes;
  if (n_edges < 0 || (value_bytes != 4 && value_bytes != 8)) return 0;
  return dpa4k::plan_bytes_for(n_edges, value_bytes);
}

extern "C" size_t dpa4k_force_assembly_plan_workspace_size(int64_t n_edges, int64_t n_nodes) {
  using namespace dpa4k;
  if (n_edges < 0 || n_nodes <= 0) return 0;
  const PlanShape shape = plan_shape(n_edges, n_nodes);
  const size_t count = static_cast<size_t>(n_edges > 0 ? n_edges : 1);
  const size_t cells = static_cast<size_t>(shape.tiles * shape.buckets);
  return 2 * round_up_256(count * 8) + round_up_256((cells + 1) * 8) + round_up_256(4) +
         round_up_256(plan_sort_bytes(n_edges, shape));
}

extern "C" int dpa4k_force_assembly_plan(const int64_t* src_offsets, const int64_t* src_order, int64_t n_edges,
                                         int64_t n_nodes, int64_t value_bytes, void* plan, size_t plan_bytes,
                                         void* workspace, size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  using namespace dpa4k;
  clear_error();
  if (int s = check_plan_shapes(n_edges, n_nodes, "force assembly plan")) return s;
  if (value_bytes != 4 && value_bytes != 8) return fail(DPA4K_EINVAL, "force assembly plan: values of 4 or 8 bytes");
  if (src_offsets == nullptr || plan == nullptr || (n_edges > 0 && src_order == nullptr))
    return fail(DPA4K_EINVAL, "force assembly plan: null pointer");
  const size_t needed = dpa4k_force_assembly_plan_size(n_edges, n_nodes, value_bytes);
  if (plan_bytes < needed)
    return fail(DPA4K_EINVAL, "force assembly plan: buffer of %zu bytes is smaller than %zu", plan_bytes, needed);
  const size_t scratch_needed = dpa4k_force_assembly_plan_workspace_size(n_edges, n_nodes);
  if (workspace == nullptr || workspace_bytes < scratch_needed)
    return fail(DPA4K_EWORKSPACE, "force assembly plan: workspace of %zu bytes is smaller than %zu", workspace_bytes,
                scratch_needed);
  if (n_edges == 0) return DPA4K_OK;
  const PlanShape shape = plan_shape(n_edges, n_nodes);
  PlanArrays arrays;
  PlanScratch scratch;
  if (!carve_plan(plan, plan_bytes, n_edges, value_bytes, arrays) ||
      !carve_scratch(workspace, workspace_bytes, n_edges, shape, scratch))
    return fail(DPA4K_EINVAL, "force assembly plan: buffers too small");
  hipStream_t stream = as_stream(stream_handle);
  const unsigned int blocks = grid_stride_blocks(n_edges);
  plan_default_keys_kernel<<<blocks, 256, 0, stream>>>(scratch.key, n_edges, shape.buckets);
  if (int s = launched("plan_default_keys_kernel")) return s;
  plan_source_keys_kernel<<<blocks, 256, 0, stream>>>(src_offsets, src_order, scratch.key, n_edges, n_nodes,
                                                      shape.buckets, shape.bucket_atoms);
  if (int s = launched("plan_source_keys_kernel")) return s;
  // keys lie in [0, tiles * buckets) by construction: the status word is not read
  if (int s = dpa4k_group_by_key_async(scratch.key, n_edges, shape.tiles * shape.buckets, scratch.order,
                                       scratch.tile_offsets, scratch.status, scratch.sort, scratch.sort_bytes,
                                       stream_handle))
    return s;
  plan_rows_kernel<<<blocks, 256, 0, stream>>>(scratch.order, arrays.edge_row, n_edges);
  if (int s = launched("plan_rows_kernel")) return s;
  plan_source_positions_kernel<<<blocks, 256, 0, stream>>>(src_order, arrays.edge_row, arrays.src_pos, n_edges);
  return launched("plan_source_positions_kernel");
}

extern "C" int dpa4k_force_assembly_f32_planned(const float* grad_edge, const float* edge_vec,
                                                const int64_t* dst_offsets, const int64_t* src_offsets,
                                                float* force, float* virial, int64_t n_edges, int64_t n_nodes,
                                                void* plan, size_t plan_bytes, dpa4k_stream_t stream) {
  return dpa4k::run_planned<float>(grad_edge, edge_vec, dst_offsets, src_offsets, force, virial, n_edges, n_nodes,
                                   plan, plan_bytes, stream);
}

extern "C" int dpa4k_force_assembly_f64_planned(const double* grad_edge, const double* edge_vec,
                                                const int64_t* dst_offsets, const int64_t* src_offsets,
                                                double* force, double* virial, int64_t n_edges, int64_t n_nodes,
                                                void* plan, size_t plan_bytes, dpa4k_stream_t stream) {
  return dpa4k::run_planned<double>(grad_edge, edge_vec, dst_offsets, src_offsets, force, virial, n_edges, n_nodes,
                                    plan, plan_bytes, stream);
}

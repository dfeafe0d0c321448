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
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
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

// kRowViews: 3 * E * sizeof(T) < 2^31, so the gathered rows are addressed
// through 32-bit offsets into views of the whole arrays (one register per
// address, zeros for a lane without a row); otherwise through pointers at a
// clamped edge id, with the rows of invalid slots zeroed afterwards.
template <typename T, bool kRowViews>
__global__ __launch_bounds__(kBlock) void force_assembly_kernel(
    const T* __restrict__ grad_edge, const T* __restrict__ edge_vec,
    const int64_t* __restrict__ dst_offsets, const int64_t* __restrict__ src_offsets,
    const int64_t* __restrict__ src_order, T* __restrict__ force, T* __restrict__ virial,
    int64_t n_edges, int64_t n_nodes) {
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
  const int64_t dst_base = (dst_begin - wave_dst) * 3 * static_cast<int64_t>(sizeof(T));
  const int64_t src_base = (src_begin - wave_src) * 8;
  const bool dst_window = dst_base >= 0 && dst_base < int64_t(kNoRow) - kWindowBytes;
  const bool src_window = src_base >= 0 && src_base < int64_t(kNoRow) - kWindowBytes;

  const BufferView slots = buffer_view(src_order + wave_src, (n_edges - wave_src) * 8);
  int64_t edge[kSrcRounds];
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) {
    const uint32_t offset = src_window ? static_cast<uint32_t>(src_base) + static_cast<uint32_t>(r * kGroup + lane) * 8u
                                       : kNoRow;
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
  if constexpr (kRowViews) {
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
    const int64_t e = edge_of<true>(src_order, slot, n_edges);
    if (e < 0) continue;
    add_source(acc, load_row(grad_edge, e), load_row(edge_vec, e));
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
    force_assembly_kernel<T, true><<<grid, kBlock, 0, stream>>>(grad_edge, edge_vec, dst_offsets, src_offsets,
                                                                src_order, force, virial, n_edges, n_nodes);
  else
    force_assembly_kernel<T, false><<<grid, kBlock, 0, stream>>>(grad_edge, edge_vec, dst_offsets, src_offsets,
                                                                 src_order, force, virial, n_edges, n_nodes);
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

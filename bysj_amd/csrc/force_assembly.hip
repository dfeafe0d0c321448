// force_assembly (python/kernels/segment.py:314-332, csrc/force_assembly.cpp:106
// of the reference):
//   F_k = sum_{dst(e)=k} g_e - sum_{src(e)=k} g_e
//   W_k = sum_{src(e)=k} -(g_e outer v_e)           (row-major 3x3)
// as a gather over two CSR views: the natural (dst-grouped) edge order and
// the src_order permutation.  No atomics, no materialised (E, 9) product.
//
// Layout: a group of G = 32 lanes owns one atom (8 atoms per 256-thread
// workgroup).  Every load of the atom is issued before any arithmetic:
//   * the source side gathers whole 12- or 24-byte rows g_e, v_e through
//     src_order (one row pair per lane, SRC_R rounds held in registers);
//   * the destination side streams the contiguous span grad_edge[3*begin,
//     3*end) as scalars (DST_R rounds in registers), the component of
//     scalar f being f mod 3.
// Longer segments continue in loops.  Every lane accumulates all twelve
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
constexpr int kSrcRounds = 3;   // source rows per lane held in registers
constexpr int kDstRounds = 9;   // destination scalars per lane held in registers

template <typename T>
struct Row3 {
  T x, y, z;
};

template <typename T>
__device__ __forceinline__ Row3<T> load_row(const T* __restrict__ base, int64_t e) {
  return *reinterpret_cast<const Row3<T>*>(base + 3 * e);
}

__device__ __forceinline__ void add_component(double (&acc)[12], int64_t f, double value) {
  const int component = static_cast<int>(f % 3);
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

template <typename T>
__global__ __launch_bounds__(kBlock) void force_assembly_kernel(
    const T* __restrict__ grad_edge, const T* __restrict__ edge_vec,
    const int64_t* __restrict__ dst_offsets, const int64_t* __restrict__ src_offsets,
    const int64_t* __restrict__ src_order, T* __restrict__ force, T* __restrict__ virial,
    int64_t n_edges, int64_t n_nodes) {
  // Neighbouring atoms gather rows from the same destination segments when
  // atom numbering follows space, so each XCD takes a contiguous atom range
  // (of each grid row, when the atoms need more than one row of blocks).
  const int64_t block = static_cast<int64_t>(blockIdx.y) * gridDim.x + xcd_block(blockIdx.x, gridDim.x);
  const int64_t atom = block * kAtoms + (threadIdx.x >> kLogGroup);
  if (atom >= n_nodes) return;
  const int lane = threadIdx.x & (kGroup - 1);
  int64_t dst_begin, dst_end, src_begin, src_end;
  segment_bounds(dst_offsets, atom, n_edges, dst_begin, dst_end);
  segment_bounds(src_offsets, atom, n_edges, src_begin, src_end);

  // ---- issue the loads ----
  int64_t edge[kSrcRounds];
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) {
    const int64_t slot = src_begin + r * kGroup + lane;
    edge[r] = slot < src_end ? edge_of<true>(src_order, slot, n_edges) : -1;
  }
  Row3<T> g[kSrcRounds], v[kSrcRounds];
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) {
    if (edge[r] >= 0) {
      g[r] = load_row(grad_edge, edge[r]);
      v[r] = load_row(edge_vec, edge[r]);
    } else {
      g[r] = v[r] = Row3<T>{T(0), T(0), T(0)};
    }
  }
  const int64_t dst_stop = 3 * dst_end;
  T d[kDstRounds];
#pragma unroll
  for (int r = 0; r < kDstRounds; ++r) {
    const int64_t f = 3 * dst_begin + r * kGroup + lane;
    d[r] = f < dst_stop ? grad_edge[f] : T(0);
  }

  // ---- accumulate ----
  double acc[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) acc[i] = 0.0;
#pragma unroll
  for (int r = 0; r < kDstRounds; ++r)
    add_component(acc, 3 * dst_begin + r * kGroup + lane, static_cast<double>(d[r]));
  for (int64_t f = 3 * dst_begin + kDstRounds * kGroup + lane; f < dst_stop; f += kGroup)
    add_component(acc, f, static_cast<double>(grad_edge[f]));
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) add_source(acc, g[r], v[r]);
  for (int64_t slot = src_begin + kSrcRounds * kGroup + lane; slot < src_end; slot += kGroup) {
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
  force_assembly_kernel<T><<<launch_grid((n_nodes + kAtoms - 1) / kAtoms, kBlock), kBlock, 0, stream>>>(
      grad_edge, edge_vec, dst_offsets, src_offsets, src_order, force, virial, n_edges, n_nodes);
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

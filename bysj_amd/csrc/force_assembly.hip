// force_assembly (python/kernels/segment.py:314-332, csrc/force_assembly.cpp:106
// of the reference):
//   F_k = sum_{dst(e)=k} g_e - sum_{src(e)=k} g_e
//   W_k = sum_{src(e)=k} -(g_e outer v_e)           (row-major 3x3)
// as a gather over two CSR views: the natural (dst-grouped) edge order and
// the src_order permutation.  No atomics, no materialised (E, 9) product.
//
// Layout: a group of G = 16 lanes owns one atom (16 atoms per 256-thread
// block).  On the destination side the group streams the contiguous span
// grad_edge[3*begin, 3*end) as scalars (fully coalesced, the component of
// scalar f is f mod 3, advanced incrementally); on the source side each lane
// gathers whole edges through src_order.  Every lane accumulates all twelve
// outputs in double precision, then a fixed DPP/swizzle butterfly over the
// 16 lanes produces the totals, and lanes 0..11 store one component each.
// The summation order depends only on the CSR, so results are reproducible;
// fp32 inputs round once on output (double products of two floats are
// exact), fp64 inputs keep double outputs.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kGroup = 16;
constexpr int kAtoms = kBlock / kGroup;

template <typename T>
__global__ __launch_bounds__(kBlock) void force_assembly_kernel(
    const T* __restrict__ grad_edge, const T* __restrict__ edge_vec,
    const int64_t* __restrict__ dst_offsets, const int64_t* __restrict__ src_offsets,
    const int64_t* __restrict__ src_order, T* __restrict__ force, T* __restrict__ virial,
    int64_t n_edges, int64_t n_nodes) {
  const int64_t atom = static_cast<int64_t>(blockIdx.x) * kAtoms + threadIdx.x / kGroup;
  if (atom >= n_nodes) return;
  const int lane = threadIdx.x % kGroup;

  double acc[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) acc[i] = 0.0;

  int64_t begin, end;
  segment_bounds(dst_offsets, atom, n_edges, begin, end);
  {
    constexpr int kStep = kGroup % 3;
    const int64_t stop = 3 * end;
    int64_t f = 3 * begin + lane;
    int component = static_cast<int>(f % 3);
    for (; f < stop; f += kGroup) {
      const double value = static_cast<double>(grad_edge[f]);
      acc[0] += component == 0 ? value : 0.0;
      acc[1] += component == 1 ? value : 0.0;
      acc[2] += component == 2 ? value : 0.0;
      component += kStep;
      if (component >= 3) component -= 3;
    }
  }

  segment_bounds(src_offsets, atom, n_edges, begin, end);
  for (int64_t slot = begin + lane; slot < end; slot += kGroup) {
    const int64_t e = edge_of<true>(src_order, slot, n_edges);
    if (e < 0) continue;
    const double g0 = grad_edge[3 * e], g1 = grad_edge[3 * e + 1], g2 = grad_edge[3 * e + 2];
    const double v0 = edge_vec[3 * e], v1 = edge_vec[3 * e + 1], v2 = edge_vec[3 * e + 2];
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
  if ((n_nodes + kAtoms - 1) / kAtoms > kMaxGrid)
    return fail(DPA4K_EINVAL, "force assembly atom count exceeds the HIP grid limit");
  if (dst_offsets == nullptr || src_offsets == nullptr || force == nullptr || virial == nullptr ||
      (n_edges > 0 && (grad_edge == nullptr || edge_vec == nullptr || src_order == nullptr)))
    return fail(DPA4K_EINVAL, "force assembly: null pointer");
  hipStream_t stream = as_stream(stream_handle);
  force_assembly_kernel<T><<<blocks_for(n_nodes, kAtoms), kBlock, 0, stream>>>(
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

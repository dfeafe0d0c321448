// Row-wise RMSNorm, forward and backward (python/kernels/rmsnorm.py:46-85,
// csrc/rmsnorm.cpp:99-157 of the reference; oracle python/reference/rmsnorm.py:40-52):
//   inv = 1 / sqrt(mean(x^2) + eps),  y = (x * inv) * scale
//   u = grad * scale,  grad_x = inv * u - (x * inv^3) * mean(x * u)
//   grad_scale[w] = sum_rows grad * (x * inv)
//
// One wave per row.  Rows of up to 64 * 16 float4 chunks (W <= 4096) stay in
// registers between the sum of squares and the scaled store, so x is read
// once; the row sum is a DPP / swizzle / bpermute butterfly.  Wider rows take
// a two-pass streaming kernel.  The reference accumulates grad_scale with one
// float atomic per (row, column); here each wave keeps per-column partials
// for its fixed set of rows, the partials go to the workspace and a two-level
// column reduction sums them in a fixed order.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kPartialWaves = 2048;   // waves of the grad_scale backward
constexpr int kLevel = 32;            // partial rows summed per thread per level

__device__ __forceinline__ float inverse_rms_of(float sum_squares, int64_t width, float eps) {
  return 1.0f / sqrtf(sum_squares / static_cast<float>(width) + eps);
}

template <int V, int CPL>
__global__ __launch_bounds__(kBlock) void rmsnorm_forward_kernel(
    const float* __restrict__ x, const float* __restrict__ scale, float* __restrict__ y,
    float* __restrict__ inverse_rms, int64_t rows, int64_t width, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t chunks = width / V;
  const float* xr = x + row * width;
  float* yr = y + row * width;
  if constexpr (CPL > 0) {
    fvec<V> value[CPL];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t q = lane + 64 * j;
      if (q < chunks) {
        value[j] = load_vec<V>(xr + q * V);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) value[j].v[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < V; ++i) sum = sum + value[j].v[i] * value[j].v[i];
    }
    sum = group_sum<64>(sum);
    const float inv = inverse_rms_of(sum, width, eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t q = lane + 64 * j;
      if (q >= chunks) continue;
      fvec<V> out;
      fvec<V> s;
      if (scale != nullptr) s = load_vec<V>(scale + q * V);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        out.v[i] = value[j].v[i] * inv;
        if (scale != nullptr) out.v[i] = out.v[i] * s.v[i];
      }
      store_vec<V>(yr + q * V, out);
    }
    if (lane == 0) inverse_rms[row] = inv;
  } else {
    float sum = 0.0f;
    for (int64_t q = lane; q < chunks; q += 64) {
      const fvec<V> value = load_vec<V>(xr + q * V);
#pragma unroll
      for (int i = 0; i < V; ++i) sum = sum + value.v[i] * value.v[i];
    }
    sum = group_sum<64>(sum);
    const float inv = inverse_rms_of(sum, width, eps);
    for (int64_t q = lane; q < chunks; q += 64) {
      const fvec<V> value = load_vec<V>(xr + q * V);
      fvec<V> out;
      fvec<V> s;
      if (scale != nullptr) s = load_vec<V>(scale + q * V);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        out.v[i] = value.v[i] * inv;
        if (scale != nullptr) out.v[i] = out.v[i] * s.v[i];
      }
      store_vec<V>(yr + q * V, out);
    }
    if (lane == 0) inverse_rms[row] = inv;
  }
}

// Register path (CPL > 0): wave w handles rows w, w + waves, ...; with
// `partial` non-null it also stores its per-column sum of grad * (x * inv)
// as row w of the [waves, W] partial matrix.
template <int V, int CPL>
__global__ __launch_bounds__(kBlock) void rmsnorm_backward_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ scale,
    const float* __restrict__ inverse_rms, float* __restrict__ grad_x, float* __restrict__ partial,
    int64_t rows, int64_t width) {
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWaves;
  const int lane = threadIdx.x & 63;
  const int64_t chunks = width / V;

  fvec<V> s[CPL], column[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t q = lane + 64 * j;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      s[j].v[i] = 1.0f;
      column[j].v[i] = 0.0f;
    }
    if (scale != nullptr && q < chunks) s[j] = load_vec<V>(scale + q * V);
  }

  for (int64_t row = wave_id; row < rows; row += waves) {
    const float* gr = grad + row * width;
    const float* xr = x + row * width;
    fvec<V> g[CPL], xv[CPL], u[CPL];
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t q = lane + 64 * j;
      if (q < chunks) {
        g[j] = load_vec<V>(gr + q * V);
        xv[j] = load_vec<V>(xr + q * V);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) g[j].v[i] = xv[j].v[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < V; ++i) {
        u[j].v[i] = scale != nullptr ? g[j].v[i] * s[j].v[i] : g[j].v[i];
        dot = dot + xv[j].v[i] * u[j].v[i];
      }
    }
    dot = group_sum<64>(dot);
    const float mean_dot = dot / static_cast<float>(width);
    const float inv = inverse_rms[row];
    const float inv3 = inv * inv * inv;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t q = lane + 64 * j;
      if (q >= chunks) continue;
      fvec<V> out;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        out.v[i] = inv * u[j].v[i] - xv[j].v[i] * inv3 * mean_dot;
        if (partial != nullptr) column[j].v[i] = column[j].v[i] + g[j].v[i] * (xv[j].v[i] * inv);
      }
      store_vec<V>(grad_x + row * width + q * V, out);
    }
  }
  if (partial != nullptr) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t q = lane + 64 * j;
      if (q < chunks) store_vec<V>(partial + wave_id * width + q * V, column[j]);
    }
  }
}

// Streaming grad_x for wide rows: two passes over the row.
template <int V>
__global__ __launch_bounds__(kBlock) void rmsnorm_backward_wide_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ scale,
    const float* __restrict__ inverse_rms, float* __restrict__ grad_x, int64_t rows,
    int64_t width) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t chunks = width / V;
  const float* gr = grad + row * width;
  const float* xr = x + row * width;
  float dot = 0.0f;
  for (int64_t q = lane; q < chunks; q += 64) {
    const fvec<V> g = load_vec<V>(gr + q * V);
    const fvec<V> xv = load_vec<V>(xr + q * V);
    fvec<V> s;
    if (scale != nullptr) s = load_vec<V>(scale + q * V);
#pragma unroll
    for (int i = 0; i < V; ++i) dot = dot + xv.v[i] * (scale != nullptr ? g.v[i] * s.v[i] : g.v[i]);
  }
  dot = group_sum<64>(dot);
  const float mean_dot = dot / static_cast<float>(width);
  const float inv = inverse_rms[row];
  const float inv3 = inv * inv * inv;
  for (int64_t q = lane; q < chunks; q += 64) {
    const fvec<V> g = load_vec<V>(gr + q * V);
    const fvec<V> xv = load_vec<V>(xr + q * V);
    fvec<V> s;
    if (scale != nullptr) s = load_vec<V>(scale + q * V);
    fvec<V> out;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float u = scale != nullptr ? g.v[i] * s.v[i] : g.v[i];
      out.v[i] = inv * u - xv.v[i] * inv3 * mean_dot;
    }
    store_vec<V>(grad_x + row * width + q * V, out);
  }
}

// grad_scale for wide rows: thread per column, rows summed in order.
__global__ __launch_bounds__(kBlock) void rmsnorm_scale_columns_kernel(
    const float* __restrict__ grad, const float* __restrict__ x,
    const float* __restrict__ inverse_rms, float* __restrict__ grad_scale, int64_t rows,
    int64_t width) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (col >= width) return;
  float sum = 0.0f;
  for (int64_t row = 0; row < rows; ++row)
    sum = sum + grad[row * width + col] * (x[row * width + col] * inverse_rms[row]);
  grad_scale[col] = sum;
}

// out[b, w] = sum_{i < group, b*group + i < n} in[b*group + i, w]
__global__ __launch_bounds__(kBlock) void reduce_rows_kernel(const float* __restrict__ in,
                                                             int64_t n, int64_t width,
                                                             int64_t group,
                                                             float* __restrict__ out) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (col >= width) return;
  const int64_t first = b * group;
  const int64_t last = first + group < n ? first + group : n;
  float sum = 0.0f;
  for (int64_t r = first; r < last; ++r) sum = sum + in[r * width + col];
  out[b * width + col] = sum;
}

int per_lane_for(int64_t chunks) {
  int cpl = 1;
  while (cpl < 16 && 64 * cpl < chunks) cpl <<= 1;
  return 64 * cpl >= chunks ? cpl : 0;
}

template <int V>
int launch_forward(int cpl, const float* x, const float* scale, float* y, float* inverse_rms,
                   int64_t rows, int64_t width, float eps, hipStream_t stream) {
  const unsigned int grid = blocks_for(rows, kWaves);
#define DPA4K_RMS_FWD(C)                                                                  \
  rmsnorm_forward_kernel<V, C><<<grid, kBlock, 0, stream>>>(x, scale, y, inverse_rms, rows, \
                                                            width, eps)
  switch (cpl) {
    case 1: DPA4K_RMS_FWD(1); break;
    case 2: DPA4K_RMS_FWD(2); break;
    case 4: DPA4K_RMS_FWD(4); break;
    case 8: DPA4K_RMS_FWD(8); break;
    case 16: DPA4K_RMS_FWD(16); break;
    default: DPA4K_RMS_FWD(0); break;
  }
#undef DPA4K_RMS_FWD
  return launched("rmsnorm_forward_kernel");
}

template <int V>
int launch_backward(int cpl, unsigned int grid, const float* grad, const float* x,
                    const float* scale, const float* inverse_rms, float* grad_x, float* partial,
                    int64_t rows, int64_t width, hipStream_t stream) {
#define DPA4K_RMS_BWD(C)                                                                      \
  rmsnorm_backward_kernel<V, C><<<grid, kBlock, 0, stream>>>(grad, x, scale, inverse_rms,      \
                                                             grad_x, partial, rows, width)
  switch (cpl) {
    case 1: DPA4K_RMS_BWD(1); break;
    case 2: DPA4K_RMS_BWD(2); break;
    case 4: DPA4K_RMS_BWD(4); break;
    case 8: DPA4K_RMS_BWD(8); break;
    default: DPA4K_RMS_BWD(16); break;
  }
#undef DPA4K_RMS_BWD
  return launched("rmsnorm_backward_kernel");
}

unsigned int partial_blocks(int64_t rows) {
  const int64_t wanted = (rows + kWaves - 1) / kWaves;
  const int64_t cap = kPartialWaves / kWaves;
  return static_cast<unsigned int>(wanted < 1 ? 1 : (wanted > cap ? cap : wanted));
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" int dpa4k_rmsnorm_forward(const float* x, const float* scale, float* y,
                                     float* inverse_rms, int64_t rows, int64_t width, float eps,
                                     dpa4k_stream_t stream_handle) {
  clear_error();
  if (rows < 0) return fail(DPA4K_EINVAL, "RMSNorm: negative row count");
  if (width <= 0) return fail(DPA4K_EINVAL, "RMSNorm feature dimension must be positive");
  if (!(eps > 0.0f) || !(eps < INFINITY))
    return fail(DPA4K_EINVAL, "RMSNorm eps must be a finite positive number");
  if ((rows + kWaves - 1) / kWaves > kMaxGrid)
    return fail(DPA4K_EINVAL, "RMSNorm row count exceeds the HIP grid limit");
  if (rows == 0) return DPA4K_OK;
  if (x == nullptr || y == nullptr || inverse_rms == nullptr)
    return fail(DPA4K_EINVAL, "RMSNorm: null pointer");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = width % 4 == 0 && aligned16(x) && aligned16(y) &&
                    (scale == nullptr || aligned16(scale));
  const int64_t chunks = vec4 ? width / 4 : width;
  const int cpl = per_lane_for(chunks);
  return vec4 ? launch_forward<4>(cpl, x, scale, y, inverse_rms, rows, width, eps, stream)
              : launch_forward<1>(cpl, x, scale, y, inverse_rms, rows, width, eps, stream);
}

extern "C" size_t dpa4k_rmsnorm_backward_workspace_size(int64_t rows, int64_t width) {
  if (rows <= 0 || width <= 0) return 0;
  const int64_t waves = static_cast<int64_t>(partial_blocks(rows)) * kWaves;
  const int64_t level = (waves + kLevel - 1) / kLevel;
  return round_up_256(static_cast<size_t>(waves * width) * 4) +
         round_up_256(static_cast<size_t>(level * width) * 4);
}

extern "C" int dpa4k_rmsnorm_backward(const float* grad, const float* x, const float* scale,
                                      const float* inverse_rms, float* grad_x, float* grad_scale,
                                      int64_t rows, int64_t width, void* workspace,
                                      size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  clear_error();
  if (rows < 0) return fail(DPA4K_EINVAL, "RMSNorm: negative row count");
  if (width <= 0) return fail(DPA4K_EINVAL, "RMSNorm feature dimension must be positive");
  if (grad_scale != nullptr && scale == nullptr)
    return fail(DPA4K_EINVAL, "cannot compute a scale gradient when scale is omitted");
  hipStream_t stream = as_stream(stream_handle);
  if (rows == 0) {
    if (grad_scale != nullptr) return zero_fill(grad_scale, width * sizeof(float), stream);
    return DPA4K_OK;
  }
  if (grad == nullptr || x == nullptr || inverse_rms == nullptr || grad_x == nullptr)
    return fail(DPA4K_EINVAL, "RMSNorm backward: null pointer");
  const bool vec4 = width % 4 == 0 && aligned16(grad) && aligned16(x) && aligned16(grad_x) &&
                    (scale == nullptr || aligned16(scale));
  const int64_t chunks = vec4 ? width / 4 : width;
  const int cpl = per_lane_for(chunks);
  if (cpl == 0) {
    const unsigned int grid = blocks_for(rows, kWaves);
    if (vec4)
      rmsnorm_backward_wide_kernel<4><<<grid, kBlock, 0, stream>>>(grad, x, scale, inverse_rms,
                                                                    grad_x, rows, width);
    else
      rmsnorm_backward_wide_kernel<1><<<grid, kBlock, 0, stream>>>(grad, x, scale, inverse_rms,
                                                                    grad_x, rows, width);
    if (int s = launched("rmsnorm_backward_wide_kernel")) return s;
    if (grad_scale != nullptr) {
      rmsnorm_scale_columns_kernel<<<blocks_for(width, kBlock), kBlock, 0, stream>>>(
          grad, x, inverse_rms, grad_scale, rows, width);
      return launched("rmsnorm_scale_columns_kernel");
    }
    return DPA4K_OK;
  }
  if (grad_scale == nullptr) {
    const unsigned int grid = blocks_for(rows, kWaves);
    return vec4 ? launch_backward<4>(cpl, grid, grad, x, scale, inverse_rms, grad_x, nullptr, rows,
                                     width, stream)
                : launch_backward<1>(cpl, grid, grad, x, scale, inverse_rms, grad_x, nullptr, rows,
                                     width, stream);
  }
  const size_t needed = dpa4k_rmsnorm_backward_workspace_size(rows, width);
  if (workspace == nullptr || workspace_bytes < needed)
    return fail(DPA4K_EWORKSPACE, "RMSNorm backward: workspace of %zu bytes is smaller than %zu",
                workspace_bytes, needed);
  const unsigned int grid = partial_blocks(rows);
  const int64_t waves = static_cast<int64_t>(grid) * kWaves;
  const int64_t level = (waves + kLevel - 1) / kLevel;
  Carver carver{static_cast<char*>(workspace), workspace_bytes};
  float* partial = carver.take<float>(static_cast<size_t>(waves * width));
  float* partial2 = carver.take<float>(static_cast<size_t>(level * width));
  int s = vec4 ? launch_backward<4>(cpl, grid, grad, x, scale, inverse_rms, grad_x, partial, rows,
                                    width, stream)
               : launch_backward<1>(cpl, grid, grad, x, scale, inverse_rms, grad_x, partial, rows,
                                    width, stream);
  if (s) return s;
  reduce_rows_kernel<<<dim3(blocks_for(width, kBlock), static_cast<unsigned int>(level)), kBlock, 0,
                       stream>>>(partial, waves, width, kLevel, partial2);
  if (int t = launched("reduce_rows_kernel")) return t;
  reduce_rows_kernel<<<dim3(blocks_for(width, kBlock), 1), kBlock, 0, stream>>>(
      partial2, level, width, level, grad_scale);
  return launched("reduce_rows_kernel");
}

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
// for its fixed set of rows (two rows loaded per round), the four waves of a
// workgroup add theirs in LDS, the workgroup partials go to the workspace and
// a workgroup per 64 columns sums them (its waves split the rows, each load
// reading 256 contiguous bytes) -- every order fixed.
#include <mutex>
#include <vector>

#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kPartialWaves = 3072;   // waves of the grad_scale backward (resident at 3 per SIMD)
constexpr int64_t kRegisterMaxWidth = 64 * 16 * 4;  // widest row the register kernels hold

// Column partials of dpa4k_rmsnorm_backward_noalloc: one row per workgroup of
// the grad_scale backward (at most kPartialWaves / kWaves of them) of at most
// kRegisterMaxWidth floats, the most the register kernels ever write
// (DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES).  Every device the library runs on
// holds its own copy until the process ends.  Host code never uses this name
// as an address: it reaches the array through the per-device pointer that
// scratch_for_stream() obtains from hipGetSymbolAddress.
static_assert(int64_t(kPartialWaves / kWaves) * kRegisterMaxWidth * 4 == DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES,
              "the header's scratch size must match the partial matrix bound");
__device__ __align__(256) float scratch[DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES / 4];

__device__ __forceinline__ float inverse_rms_of(float sum_squares, int64_t width, float eps) {
  return 1.0f / sqrtf(sum_squares / static_cast<float>(width) + eps);
}

template <int V, int CPL>
__global__ __launch_bounds__(kBlock) void rmsnorm_forward_kernel(
    const float* __restrict__ x, const float* __restrict__ scale, float* __restrict__ y,
    float* __restrict__ inverse_rms, int64_t rows, int64_t width, float eps) {
  const int64_t row = block_index() * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t chunks = width / V;
  const float* xr = x + row * width;
  float* yr = y + row * width;
  if constexpr (CPL > 0) {
    // The row and the scale chunks are loaded before the reduction, through
    // views (zeros past the row), so that no load sits in a branch: a load in
    // a divergent branch is waited for before the branch closes, and the
    // chunk loads would follow one another instead of overlapping.
    const BufferView row_x = buffer_view(x + uniform_i64(row) * width, width * 4);
    const BufferView row_s = buffer_view(scale, scale != nullptr ? width * 4 : 0);
    fvec<V> value[CPL], s[CPL];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t offset = static_cast<uint32_t>(lane + 64 * j) * (V * 4u);
      value[j] = buffer_load_vec<V>(row_x, offset);
      s[j] = buffer_load_vec<V>(row_s, offset);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < V; ++i) sum = sum + value[j].v[i] * value[j].v[i];
    sum = group_sum<64>(sum);
    const float inv = inverse_rms_of(sum, width, eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t q = lane + 64 * j;
      if (q >= chunks) continue;
      fvec<V> out;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        out.v[i] = value[j].v[i] * inv;
        if (scale != nullptr) out.v[i] = out.v[i] * s[j].v[i];
      }
      store_vec_stream<V>(yr + q * V, out);
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

// Register path (CPL > 0): wave w handles rows w, w + waves, ... (two per round); with
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

  // Rows wave_id, wave_id + waves, ... two per round: both rows' loads are
  // issued before either is reduced.  The rows are read once and loaded
  // non-temporally (config 3R: 261 -> 247 us).
  for (int64_t first = wave_id; first < rows; first += 2 * waves) {
    fvec<V> g[2][CPL], xv[2][CPL];
    float inv[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t row = first + r * waves;
      const bool ok = row < rows;
      inv[r] = ok ? inverse_rms[row] : 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int64_t q = lane + 64 * j;
        if (ok && q < chunks) {
          g[r][j] = load_vec_stream<V>(grad + row * width + q * V);
          xv[r][j] = load_vec_stream<V>(x + row * width + q * V);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) g[r][j].v[i] = xv[r][j].v[i] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t row = first + r * waves;
      fvec<V> u[CPL];
      float dot = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < V; ++i) {
          u[j].v[i] = scale != nullptr ? g[r][j].v[i] * s[j].v[i] : g[r][j].v[i];
          dot = dot + xv[r][j].v[i] * u[j].v[i];
        }
      dot = group_sum<64>(dot);
      if (row >= rows) continue;
      const float mean_dot = dot / static_cast<float>(width);
      const float inv3 = inv[r] * inv[r] * inv[r];
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int64_t q = lane + 64 * j;
        if (q >= chunks) continue;
        fvec<V> out;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          out.v[i] = inv[r] * u[j].v[i] - xv[r][j].v[i] * inv3 * mean_dot;
          if (partial != nullptr) column[j].v[i] = column[j].v[i] + g[r][j].v[i] * (xv[r][j].v[i] * inv[r]);
        }
        store_vec_stream<V>(grad_x + row * width + q * V, out);
      }
    }
  }
  if (partial != nullptr) {
    // the four waves' column sums meet in LDS and are added in wave order;
    // the workgroup writes one row of the [workgroups, W] partial matrix
    extern __shared__ float columns[];  // [kWaves][CPL * 64 * V]
    constexpr int kSpan = CPL * 64 * V;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < V; ++i) columns[wave * kSpan + (lane + 64 * j) * V + i] = column[j].v[i];
    __syncthreads();
    for (int64_t c = threadIdx.x; c < width; c += kBlock) {
      float sum = columns[c];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) sum = sum + columns[w * kSpan + c];
      partial[static_cast<int64_t>(blockIdx.x) * width + c] = sum;
    }
  }
}

// grad_scale[w] = sum over the workgroup partial rows [n, W]: one workgroup
// of kColumnWaves waves per 64 columns, lane l on column 64 b + l.  Wave k
// adds, in order, the rows of its share [k p, (k + 1) p) (p = n / kColumnWaves
// rounded up), so each of its loads reads 256 consecutive bytes of one row;
// the waves' sums are then added in wave order.
constexpr int kColumnWaves = 16;

__global__ __launch_bounds__(kColumnWaves * 64) void partial_columns_kernel(const float* __restrict__ partial,
                                                                            int64_t n, int64_t width,
                                                                            float* __restrict__ grad_scale) {
  __shared__ float wave_sum[kColumnWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t column = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const int64_t per = (n + kColumnWaves - 1) / kColumnWaves;
  const int64_t first = wave * per;
  const int64_t last = first + per < n ? first + per : n;
  float sum = 0.0f;
  if (column < width) {
    const float* source = partial + column;
    int64_t r = first;
    // eight loads in flight, added in row order
    for (; r + 8 <= last; r += 8) {
      float value[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) value[i] = source[(r + i) * width];
#pragma unroll
      for (int i = 0; i < 8; ++i) sum = sum + value[i];
    }
    for (; r < last; ++r) sum = sum + source[r * width];
  }
  wave_sum[wave][lane] = sum;
  __syncthreads();
  if (wave == 0 && column < width) {
    float total = 0.0f;
#pragma unroll
    for (int k = 0; k < kColumnWaves; ++k) total = total + wave_sum[k][lane];
    grad_scale[column] = total;
  }
}

// Streaming grad_x for wide rows: two passes over the row.
template <int V>
__global__ __launch_bounds__(kBlock) void rmsnorm_backward_wide_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ scale,
    const float* __restrict__ inverse_rms, float* __restrict__ grad_x, int64_t rows,
    int64_t width) {
  const int64_t row = block_index() * kWaves + (threadIdx.x >> 6);
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

int per_lane_for(int64_t chunks) {
  int cpl = 1;
  while (cpl < 16 && 64 * cpl < chunks) cpl <<= 1;
  return 64 * cpl >= chunks ? cpl : 0;
}

template <int V>
int launch_forward(int cpl, const float* x, const float* scale, float* y, float* inverse_rms,
                   int64_t rows, int64_t width, float eps, hipStream_t stream) {
  const dim3 grid = launch_grid((rows + kWaves - 1) / kWaves, kBlock);
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
#define DPA4K_RMS_BWD(C)                                                                              \
  rmsnorm_backward_kernel<V, C><<<grid, kBlock, partial != nullptr ? kWaves * C * 64 * V * sizeof(float) : 0, \
                                  stream>>>(grad, x, scale, inverse_rms, grad_x, partial, rows, width)
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

// Device address of `scratch` on the device that runs `stream`, looked up once
// per device with that device current (the null stream runs on the current
// device).  Sets `out` or returns an error status.
int scratch_for_stream(hipStream_t stream, float*& out) {
  static std::mutex lock;
  static std::vector<float*> per_device;
  int current = 0;
  if (int s = hip_status(hipGetDevice(&current), "hipGetDevice")) return s;
  int device = current;
  if (stream != nullptr) {
    if (int s = hip_status(hipStreamGetDevice(stream, &device), "hipStreamGetDevice")) return s;
  }
  std::lock_guard<std::mutex> guard(lock);
  if (per_device.empty()) {
    int count = 0;
    if (int s = hip_status(hipGetDeviceCount(&count), "hipGetDeviceCount")) return s;
    per_device.assign(static_cast<size_t>(count > 0 ? count : 1), nullptr);
  }
  if (device < 0 || static_cast<size_t>(device) >= per_device.size())
    return fail(DPA4K_EHIP, "RMSNorm backward: stream on unknown device %d", device);
  if (per_device[device] == nullptr) {
    if (device != current) {
      if (int s = hip_status(hipSetDevice(device), "hipSetDevice")) return s;
    }
    void* address = nullptr;
    const hipError_t found = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (device != current) {
      if (int s = hip_status(hipSetDevice(current), "hipSetDevice")) return s;
    }
    if (int s = hip_status(found, "hipGetSymbolAddress(scratch)")) return s;
    if (address == nullptr) return fail(DPA4K_EHIP, "hipGetSymbolAddress(scratch) returned a null address");
    per_device[device] = static_cast<float*>(address);
  }
  out = per_device[device];
  return DPA4K_OK;
}

size_t backward_workspace_bytes(int64_t rows, int64_t width) {
  if (rows <= 0 || width <= 0) return 0;
  return round_up_256(static_cast<size_t>(partial_blocks(rows)) * static_cast<size_t>(width) * 4);
}

// The backward with its column partials in `workspace` (checked against the size the
// shape needs; only the register kernels with a scale gradient use it), or, with
// `static_scratch`, in this device's `scratch` array.
int rmsnorm_backward(const float* grad, const float* x, const float* scale, const float* inverse_rms,
                     float* grad_x, float* grad_scale, int64_t rows, int64_t width, void* workspace,
                     size_t workspace_bytes, bool static_scratch, hipStream_t stream) {
  if (rows < 0) return fail(DPA4K_EINVAL, "RMSNorm: negative row count");
  if (width <= 0) return fail(DPA4K_EINVAL, "RMSNorm feature dimension must be positive");
  if (grad_scale != nullptr && scale == nullptr)
    return fail(DPA4K_EINVAL, "cannot compute a scale gradient when scale is omitted");
  // the scale gradient takes one thread per column along one grid row
  if (grad_scale != nullptr && width > 4294967295LL / kBlock * kBlock)
    return fail(DPA4K_EINVAL, "RMSNorm scale gradient: feature dimension exceeds the launch limit");
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
    const dim3 grid = launch_grid((rows + kWaves - 1) / kWaves, kBlock);
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
    // the register kernel strides over rows: one row of blocks covers any count
    const int64_t wanted = (rows + kWaves - 1) / kWaves;
    const int64_t limit = row_block_limit(kBlock);
    const unsigned int grid = static_cast<unsigned int>(wanted < limit ? wanted : limit);
    return vec4 ? launch_backward<4>(cpl, grid, grad, x, scale, inverse_rms, grad_x, nullptr, rows,
                                     width, stream)
                : launch_backward<1>(cpl, grid, grad, x, scale, inverse_rms, grad_x, nullptr, rows,
                                     width, stream);
  }
  const size_t needed = backward_workspace_bytes(rows, width);
  if (static_scratch) {
    // every row of partials the register kernels write fits (width <= kRegisterMaxWidth here)
    if (needed > static_cast<size_t>(DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES))
      return fail(DPA4K_EINVAL,
                  "RMSNorm backward (no allocation): %zu bytes of column partials exceed the %d-byte scratch",
                  needed, DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES);
    float* address = nullptr;
    if (int s = scratch_for_stream(stream, address)) return s;
    workspace = address;
    workspace_bytes = DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES;
  }
  if (workspace == nullptr || workspace_bytes < needed)
    return fail(DPA4K_EWORKSPACE, "RMSNorm backward: workspace of %zu bytes is smaller than %zu",
                workspace_bytes, needed);
  const unsigned int grid = partial_blocks(rows);
  float* partial = static_cast<float*>(workspace);
  int s = vec4 ? launch_backward<4>(cpl, grid, grad, x, scale, inverse_rms, grad_x, partial, rows,
                                    width, stream)
               : launch_backward<1>(cpl, grid, grad, x, scale, inverse_rms, grad_x, partial, rows,
                                    width, stream);
  if (s) return s;
  partial_columns_kernel<<<static_cast<unsigned int>((width + 63) / 64), kColumnWaves * 64, 0, stream>>>(
      partial, grid, width, grad_scale);
  return launched("partial_columns_kernel");
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
  if (!grid_fits((rows + kWaves - 1) / kWaves, kBlock))
    return fail(DPA4K_EINVAL, "RMSNorm row count exceeds the launch limit");
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
  return backward_workspace_bytes(rows, width);
}

extern "C" int dpa4k_rmsnorm_backward(const float* grad, const float* x, const float* scale,
                                      const float* inverse_rms, float* grad_x, float* grad_scale,
                                      int64_t rows, int64_t width, void* workspace,
                                      size_t workspace_bytes, dpa4k_stream_t stream_handle) {
  clear_error();
  return rmsnorm_backward(grad, x, scale, inverse_rms, grad_x, grad_scale, rows, width, workspace,
                          workspace_bytes, false, as_stream(stream_handle));
}

extern "C" int dpa4k_rmsnorm_backward_noalloc(const float* grad, const float* x, const float* scale,
                                              const float* inverse_rms, float* grad_x, float* grad_scale,
                                              int64_t rows, int64_t width, dpa4k_stream_t stream_handle) {
  clear_error();
  return rmsnorm_backward(grad, x, scale, inverse_rms, grad_x, grad_scale, rows, width, nullptr, 0, true,
                          as_stream(stream_handle));
}

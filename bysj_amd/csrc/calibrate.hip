// Stream calibration for the measurement harness (no reference counterpart).
//
// The roofline of every operator here is HBM bandwidth.  Besides MI355X's
// nominal 8 TB/s, bench.py reports what plain streams reach on the same
// part in the same run: a read-only pass, a copy, and a copy of exactly a
// given operator's byte counts.  Grid-stride kernels, four 16-byte chunks
// per thread per round with every load of a round issued first,
// non-temporal loads and stores (non-temporal loads raise a 1 GiB read pass
// from about 6.1 to 7.0 TB/s and a 1 GiB copy from 5.6 to 5.9 TB/s, so the
// streams priced here are the faster ones).
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kRound = 4;

// Sums every float4 chunk of src; one word per workgroup is written only for
// an impossible sum, which keeps the loads alive without extra traffic.
__global__ __launch_bounds__(kBlock) void stream_read_kernel(const float* __restrict__ src, int64_t chunks,
                                                             float* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kRound;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kBlock * kRound + threadIdx.x; base < chunks;
       base += stride) {
    f32x4 x[kRound];
#pragma unroll
    for (int r = 0; r < kRound; ++r) {
      const int64_t i = base + static_cast<int64_t>(r) * kBlock;
      x[r] = i < chunks ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + 4 * i)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int r = 0; r < kRound; ++r) acc += x[r];
  }
  const float total = acc.x + acc.y + acc.z + acc.w;
  if (total == -1.0e38f) sink[blockIdx.x] = total;
}

// dst[i] = src[i] over `write_chunks` float4 chunks, reading `read_chunks`
// (>= write_chunks) so that reads and writes can match an operator's counts.
__global__ __launch_bounds__(kBlock) void stream_copy_kernel(const float* __restrict__ src, int64_t read_chunks,
                                                             float* __restrict__ dst, int64_t write_chunks) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kRound;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kBlock * kRound + threadIdx.x; base < read_chunks;
       base += stride) {
    f32x4 x[kRound];
#pragma unroll
    for (int r = 0; r < kRound; ++r) {
      const int64_t i = base + static_cast<int64_t>(r) * kBlock;
      x[r] = i < read_chunks ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + 4 * i)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int r = 0; r < kRound; ++r) {
      const int64_t i = base + static_cast<int64_t>(r) * kBlock;
      if (i < write_chunks) __builtin_nontemporal_store(x[r], reinterpret_cast<f32x4*>(dst + 4 * i));
    }
  }
}

}  // namespace
}  // namespace dpa4k

extern "C" int dpa4k_stream_calibrate(const float* src, int64_t read_floats, float* dst, int64_t write_floats,
                                      dpa4k_stream_t stream_handle) {
  using namespace dpa4k;
  clear_error();
  if (read_floats < 0 || write_floats < 0 || write_floats > read_floats || read_floats % 4 || write_floats % 4)
    return fail(DPA4K_EINVAL, "stream calibration: counts must be multiples of 4 with writes <= reads");
  if (read_floats == 0) return DPA4K_OK;
  if (src == nullptr || dst == nullptr || !aligned16(src) || !aligned16(dst))
    return fail(DPA4K_EINVAL, "stream calibration: null or unaligned buffer");
  hipStream_t stream = as_stream(stream_handle);
  const int64_t chunks = read_floats / 4;
  const int64_t wanted = (chunks + kBlock * kRound - 1) / (kBlock * kRound);
  const unsigned int grid = static_cast<unsigned int>(wanted < 8192 ? wanted : 8192);
  if (write_floats == 0) {
    if (grid > 0) stream_read_kernel<<<grid, kBlock, 0, stream>>>(src, chunks, dst);
    return launched("stream_read_kernel");
  }
  stream_copy_kernel<<<grid, kBlock, 0, stream>>>(src, chunks, dst, write_floats / 4);
  return launched("stream_copy_kernel");
}

// Shared host/device helpers of libdpa4k (gfx950 / CDNA4, wave64).
//
// Host side: error plumbing for the C ABI (status codes + a thread-local
// message) and workspace carving.  Device side: clamped CSR bounds and
// cross-lane butterflies built from DPP (xor 1, 2), ds_swizzle bit mode
// (xor 4, 8, 16) and ds_bpermute (xor 32).  The butterflies must be executed
// with every lane of the group active; all callers keep them in code that is
// uniform over the lane group.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/dpa4k.h"

namespace dpa4k {

// ---------------------------------------------------------------------------
// Host: status plumbing
// ---------------------------------------------------------------------------

// Stores a printf-style message as the thread's last error and returns `code`.
int fail(int code, const char* format, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; DPA4K_EHIP with the kernel name on
// failure, DPA4K_OK otherwise.
int launched(const char* kernel);

// Wraps a HIP runtime call result.
int hip_status(hipError_t status, const char* what);

// Clears the thread's last error (called on entry by every ABI function).
void clear_error();

// Enqueues a kernel that writes `bytes` zero bytes at `pointer` (4-byte
// aligned, `bytes` a multiple of 4).  Used instead of hipMemsetAsync so that
// callers may capture the library's launches into a HIP graph.
int zero_fill(void* pointer, size_t bytes, hipStream_t stream);

inline hipStream_t as_stream(dpa4k_stream_t stream) {
  return reinterpret_cast<hipStream_t>(stream);
}

inline bool aligned16(const void* pointer) {
  return (reinterpret_cast<uintptr_t>(pointer) & 15u) == 0;
}

// Rounds a byte count up to the 256-byte granularity used for every carve.
constexpr size_t round_up_256(size_t bytes) { return (bytes + 255u) & ~size_t(255u); }

// Sequential bump allocator over a caller-provided workspace.
struct Carver {
  char* base;
  size_t size;
  size_t used = 0;
  template <typename T>
  T* take(size_t count) {
    const size_t bytes = round_up_256(count * sizeof(T));
    if (used + bytes > size) return nullptr;
    T* out = reinterpret_cast<T*>(base + used);
    used += bytes;
    return out;
  }
};

inline unsigned int blocks_for(int64_t items, int64_t per_block) {
  return static_cast<unsigned int>((items + per_block - 1) / per_block);
}

// ---------------------------------------------------------------------------
// Host/device: grids of more blocks than one row holds
// ---------------------------------------------------------------------------
//
// HIP launches fewer than 2^32 work-items along each grid dimension
// (gridDim.x * blockDim.x < 2^32): at most 16,777,215 blocks of 256 threads
// along x.  Kernels that take one unit of work per block (a segment, a group
// of rows) are launched on launch_grid(blocks, threads): a 1-D grid up to that
// limit, and beyond it rows of equal length along y.  The kernel numbers its
// blocks with block_index(), which is blockIdx.x in a 1-D grid, and returns
// from the few blocks of the last row that lie past its work.

// Most blocks of `threads` threads along x (the hardware limit, or the lower
// limit set with dpa4k_set_launch_row_limit).
int64_t row_block_limit(int threads);

// Grid of at least `blocks` blocks (blocks >= 1); rows.x * rows.y < blocks +
// rows.y, so at most rows.y - 1 blocks find no work.
inline dim3 launch_grid(int64_t blocks, int threads) {
  const int64_t limit = row_block_limit(threads);
  if (blocks <= limit) return dim3(static_cast<unsigned int>(blocks), 1u, 1u);
  const int64_t rows = (blocks + limit - 1) / limit;
  const int64_t per_row = (blocks + rows - 1) / rows;
  return dim3(static_cast<unsigned int>(per_row), static_cast<unsigned int>(rows), 1u);
}

// Whether launch_grid() can express `blocks` (its rows are bounded like its
// columns).
inline bool grid_fits(int64_t blocks, int threads) {
  return blocks / row_block_limit(threads) < 4294967295LL;
}

__device__ __forceinline__ int64_t block_index() {
  return static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
}

// ---------------------------------------------------------------------------
// Device: XCD-aware block order
// ---------------------------------------------------------------------------

// gfx950 deals the workgroups of a launch to its 8 XCDs round-robin
// (workgroup b runs on XCD b mod 8), and each XCD has its own L2.  This
// bijection on [0, blocks) renumbers them so that every XCD runs one
// contiguous range of logical blocks: XCD x gets blocks/8 logical blocks
// (plus one for the first blocks mod 8 XCDs) starting at
// x * (blocks/8) + min(x, blocks mod 8).  Kernels whose neighbouring blocks
// share data then find it in their own L2.
constexpr unsigned int kXcds = 8;

__device__ __forceinline__ unsigned int xcd_block(unsigned int block, unsigned int blocks) {
  const unsigned int xcd = block % kXcds;
  const unsigned int index = block / kXcds;
  const unsigned int whole = blocks / kXcds;
  const unsigned int extra = blocks % kXcds;
  return xcd * whole + (xcd < extra ? xcd : extra) + index;
}

// ---------------------------------------------------------------------------
// Device: CSR bounds
// ---------------------------------------------------------------------------

// Segment [begin, end) of `segment`, clamped to [0, n_edges] so that a
// malformed offsets array cannot send a kernel out of bounds.
__device__ __forceinline__ void segment_bounds(const int64_t* __restrict__ offsets,
                                               int64_t segment, int64_t n_edges,
                                               int64_t& begin, int64_t& end) {
  int64_t b = offsets[segment];
  int64_t e = offsets[segment + 1];
  b = b < 0 ? 0 : (b > n_edges ? n_edges : b);
  e = e < b ? b : (e > n_edges ? n_edges : e);
  begin = b;
  end = e;
}

// Edge addressed by CSR slot `slot`; -1 when `order` holds an out-of-range
// entry (the caller skips it).
template <bool kOrdered>
__device__ __forceinline__ int64_t edge_of(const int64_t* __restrict__ order,
                                           int64_t slot, int64_t n_edges) {
  if constexpr (!kOrdered) {
    return slot;
  } else {
    const int64_t edge = order[slot];
    return static_cast<uint64_t>(edge) < static_cast<uint64_t>(n_edges) ? edge : -1;
  }
}

// ---------------------------------------------------------------------------
// Device: cross-lane butterflies (lane ^ MASK within the wave)
// ---------------------------------------------------------------------------

template <int MASK>
__device__ __forceinline__ int xor_lane(int value) {
  static_assert(MASK >= 1 && MASK <= 32 && (MASK & (MASK - 1)) == 0, "power-of-two mask");
  if constexpr (MASK == 1) {
    // DPP quad_perm [1,0,3,2]
    return __builtin_amdgcn_update_dpp(0, value, 0xB1, 0xF, 0xF, false);
  } else if constexpr (MASK == 2) {
    // DPP quad_perm [2,3,0,1]
    return __builtin_amdgcn_update_dpp(0, value, 0x4E, 0xF, 0xF, false);
  } else if constexpr (MASK < 32) {
    // ds_swizzle bit mode inside each 32-lane half: and 0x1F, or 0, xor MASK
    return __builtin_amdgcn_ds_swizzle(value, 0x1F | (MASK << 10));
  } else {
    // crosses the 32-lane halves: ds_bpermute
    const int lane = __lane_id();
    return __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, value);
  }
}

template <int MASK>
__device__ __forceinline__ float xor_lane(float value) {
  return __int_as_float(xor_lane<MASK>(__float_as_int(value)));
}

template <int MASK>
__device__ __forceinline__ double xor_lane(double value) {
  const int64_t bits = __double_as_longlong(value);
  const int lo = xor_lane<MASK>(static_cast<int>(bits & 0xffffffffll));
  const int hi = xor_lane<MASK>(static_cast<int>(bits >> 32));
  return __longlong_as_double((static_cast<int64_t>(hi) << 32) |
                              (static_cast<int64_t>(lo) & 0xffffffffll));
}

// Sum over the aligned group of GROUP lanes containing this lane (GROUP a
// power of two <= 64); every lane of the group receives the total.  The
// butterfly order is fixed, so the result is reproducible.
template <int GROUP, typename T>
__device__ __forceinline__ T group_sum(T value) {
  if constexpr (GROUP >= 2) value += xor_lane<1>(value);
  if constexpr (GROUP >= 4) value += xor_lane<2>(value);
  if constexpr (GROUP >= 8) value += xor_lane<4>(value);
  if constexpr (GROUP >= 16) value += xor_lane<8>(value);
  if constexpr (GROUP >= 32) value += xor_lane<16>(value);
  if constexpr (GROUP >= 64) value += xor_lane<32>(value);
  return value;
}

template <int GROUP>
__device__ __forceinline__ float group_max(float value) {
  if constexpr (GROUP >= 2) value = fmaxf(value, xor_lane<1>(value));
  if constexpr (GROUP >= 4) value = fmaxf(value, xor_lane<2>(value));
  if constexpr (GROUP >= 8) value = fmaxf(value, xor_lane<4>(value));
  if constexpr (GROUP >= 16) value = fmaxf(value, xor_lane<8>(value));
  if constexpr (GROUP >= 32) value = fmaxf(value, xor_lane<16>(value));
  if constexpr (GROUP >= 64) value = fmaxf(value, xor_lane<32>(value));
  return value;
}

// Sum across lanes that differ only in the bits [FROM, 64) of the lane id
// (i.e. across the 64/FROM sub-groups of FROM lanes); lanes keep their
// position inside the sub-group.
template <int FROM, typename T>
__device__ __forceinline__ T across_sum(T value) {
  if constexpr (FROM <= 1) value += xor_lane<1>(value);
  if constexpr (FROM <= 2) value += xor_lane<2>(value);
  if constexpr (FROM <= 4) value += xor_lane<4>(value);
  if constexpr (FROM <= 8) value += xor_lane<8>(value);
  if constexpr (FROM <= 16) value += xor_lane<16>(value);
  if constexpr (FROM <= 32) value += xor_lane<32>(value);
  return value;
}

template <int FROM>
__device__ __forceinline__ float across_max(float value) {
  if constexpr (FROM <= 1) value = fmaxf(value, xor_lane<1>(value));
  if constexpr (FROM <= 2) value = fmaxf(value, xor_lane<2>(value));
  if constexpr (FROM <= 4) value = fmaxf(value, xor_lane<4>(value));
  if constexpr (FROM <= 8) value = fmaxf(value, xor_lane<8>(value));
  if constexpr (FROM <= 16) value = fmaxf(value, xor_lane<16>(value));
  if constexpr (FROM <= 32) value = fmaxf(value, xor_lane<32>(value));
  return value;
}

// Plain vector of N floats with 16-byte (N == 4) or natural alignment.
template <int N>
struct alignas(N == 4 ? 16 : 4) fvec {
  float v[N];
};

template <int N>
__device__ __forceinline__ fvec<N> load_vec(const float* __restrict__ p) {
  if constexpr (N == 4) {
    const float4 raw = *reinterpret_cast<const float4*>(p);
    return fvec<4>{{raw.x, raw.y, raw.z, raw.w}};
  } else {
    fvec<N> out;
#pragma unroll
    for (int i = 0; i < N; ++i) out.v[i] = p[i];
    return out;
  }
}

template <int N>
__device__ __forceinline__ void store_vec(float* __restrict__ p, const fvec<N>& value) {
  if constexpr (N == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(value.v[0], value.v[1], value.v[2], value.v[3]);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = value.v[i];
  }
}

// Non-temporal variants for streams that are written once and not re-read by
// the same kernel (outputs of [E, C] size).
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Non-temporal load of rows read once, so that they do not displace lines
// the kernel reads again (per-edge scales gathered through an order, the
// order itself, offsets).
template <int N>
__device__ __forceinline__ fvec<N> load_vec_stream(const float* __restrict__ p) {
  if constexpr (N == 4) {
    const f32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return fvec<4>{{raw.x, raw.y, raw.z, raw.w}};
  } else {
    fvec<N> out;
#pragma unroll
    for (int i = 0; i < N; ++i) out.v[i] = __builtin_nontemporal_load(p + i);
    return out;
  }
}

template <int N>
__device__ __forceinline__ void store_vec_stream(float* __restrict__ p, const fvec<N>& value) {
  if constexpr (N == 4) {
    f32x4 raw = {value.v[0], value.v[1], value.v[2], value.v[3]};
    __builtin_nontemporal_store(raw, reinterpret_cast<f32x4*>(p));
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) __builtin_nontemporal_store(value.v[i], p + i);
  }
}

// ---------------------------------------------------------------------------
// Device: buffer views
// ---------------------------------------------------------------------------
//
// A buffer view is a buffer resource over a byte range starting at a
// wave-uniform address.  A load at an offset at or past the end of the range
// returns zeros and a store there is dropped, both without a memory access.
// A lane that has no row therefore issues the same instruction as its
// neighbours with the offset kNoRow instead of branching around it.  This
// matters for latency: arithmetic on a value loaded inside a branch is
// placed in that branch by the compiler, which must then wait for the load
// before the branch ends, and the loads of consecutive tiles stop
// overlapping.  Offsets are 32-bit, and callers rebase views so that the
// offsets they use stay below 2^31.
constexpr uint32_t kNoRow = 0x80000000u;

// Word 3 of a gfx9-family buffer resource: 32-bit data format, no swizzle.
constexpr int kBufferFlags = 0x00020000;

typedef __amdgpu_buffer_rsrc_t BufferView;

__device__ __forceinline__ BufferView buffer_view(const void* base, int64_t bytes) {
  const int64_t records = bytes < 0 ? 0 : (bytes > int64_t(kNoRow) ? int64_t(kNoRow) : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(static_cast<uint32_t>(records)), kBufferFlags);
}

// The rows [base, n_rows) of a row-major float array with `width` floats per
// row; `base` must be wave-uniform.
__device__ __forceinline__ BufferView row_view(const float* p, int64_t base, int64_t n_rows, int64_t width) {
  return buffer_view(p + base * width, (n_rows - base) * width * 4);
}

// `value` of the lowest active lane, as a wave-uniform (scalar) value.
__device__ __forceinline__ int64_t uniform_i64(int64_t value) {
  const uint64_t bits = static_cast<uint64_t>(value);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bits));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bits >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Cache policy of buffer loads and stores: 0 the default, kNonTemporal for
// data read or written once.
constexpr int kNonTemporal = 2;

template <int kPolicy = 0>
__device__ __forceinline__ float buffer_load_f32(BufferView view, uint32_t offset) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_raw_buffer_load_b32(view, static_cast<int>(offset), 0, kPolicy));
}

template <int N, int kPolicy = 0>
__device__ __forceinline__ fvec<N> buffer_load_vec(BufferView view, uint32_t offset) {
  fvec<N> out;
  if constexpr (N == 4) {
    const f32x4 raw = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(offset),
                                                                                        0, kPolicy));
    out.v[0] = raw.x;
    out.v[1] = raw.y;
    out.v[2] = raw.z;
    out.v[3] = raw.w;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      out.v[i] = buffer_load_f32<kPolicy>(view, offset == kNoRow ? kNoRow : offset + 4u * i);
  }
  return out;
}

// Non-temporal (cache policy nt) store of N floats; dropped at kNoRow.
template <int N>
__device__ __forceinline__ void buffer_store_vec_stream(BufferView view, uint32_t offset, const fvec<N>& value) {
  if constexpr (N == 4) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const f32x4 raw = {value.v[0], value.v[1], value.v[2], value.v[3]};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, raw), view, static_cast<int>(offset), 0,
                                           kNonTemporal);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value.v[i]), view,
                                            static_cast<int>(offset == kNoRow ? kNoRow : offset + 4u * i), 0,
                                            kNonTemporal);
  }
}

__device__ __forceinline__ void buffer_store_f32(BufferView view, uint32_t offset, float value) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), view, static_cast<int>(offset), 0, 0);
}

}  // namespace dpa4k

// segment_softmax forward and backward (python/kernels/segment.py:233-280,
// csrc/segment_softmax.cpp:235-343 of the reference; the arithmetic follows
// the oracle chain python/reference/segment.py:63-118).
//
// Edge-major layout for rows of up to 64 vector chunks (C <= 256): LC lanes
// cover one edge row (a power of two >= C/4), so one wave reads P = 64/LC
// edges per load instruction (C = 8: 2 lanes per 32-byte row, 32 edges per
// wave-load).  A 256-thread block owns four consecutive segments:
//   * degree-binned schedule: a segment of at most RMAX*P edges is handled by
//     one wave, its effective logits held in registers between the max, sum
//     and write passes (one HBM read of logit/env, one write of alpha);
//   * a longer segment (hub) is handled afterwards by all four waves of the
//     block: each wave takes every fourth tile of P slots, per-wave partial
//     maxima and sums are combined in LDS in a fixed order.
// Reductions across the P edge slots of a wave are DPP / ds_swizzle /
// ds_bpermute butterflies, so every result is reproducible bit for bit.
// Rows wider than 64 chunks use a channel-major kernel (one lane per chunk,
// sequential passes over the segment).
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

// l_e = logit + 2 ln(max(env, 1e-30)) for env > 0, else -inf (no mass).
__device__ __forceinline__ float effective_logit(float logit, float env) {
  return env > 0.0f ? logit + 2.0f * logf(fmaxf(env, 1e-30f)) : -INFINITY;
}

// d l_e / d env = 2 / env where the clamp is inactive, 0 elsewhere.
__device__ __forceinline__ float env_gradient(float row_sum, float env) {
  return env >= 1e-30f ? row_sum * 2.0f / env : 0.0f;
}

template <int LOG_LC>
struct Shape {
  static constexpr int LC = 1 << LOG_LC;   // lanes per edge row
  static constexpr int P = 64 / LC;        // edges per wave-load
  static constexpr int RMAX = LOG_LC <= 2 ? 4 : (LOG_LC == 3 ? 8 : 16);  // register tiles
};

template <int V, int LOG_LC, bool kNull, bool kOrdered>
__global__ __launch_bounds__(kBlock) void softmax_forward_kernel(
    const float* __restrict__ logit, const float* __restrict__ env,
    const int64_t* __restrict__ offsets, const float* __restrict__ null_logit,
    const int64_t* __restrict__ order, float* __restrict__ alpha, float* __restrict__ null_alpha,
    int64_t n_edges, int64_t n_nodes, int64_t channels) {
  using S = Shape<LOG_LC>;
  constexpr int LC = S::LC, P = S::P, RMAX = S::RMAX;
  __shared__ float partial[kWaves][LC * V];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int k = lane & (LC - 1);
  const int p = lane >> LOG_LC;
  const bool live = k < channels / V;
  const int64_t column = static_cast<int64_t>(k) * V;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kWaves;

  // ---- short segments: one wave each, logits staged in registers --------
  {
    const int64_t segment = first + wave;
    int64_t begin = 0, end = 0;
    if (segment < n_nodes) segment_bounds(offsets, segment, n_edges, begin, end);
    if (segment < n_nodes && end - begin <= RMAX * P) {
      const int64_t degree = end - begin;
      float value[RMAX][V];
      int64_t edge[RMAX];
      float peak[V];
#pragma unroll
      for (int v = 0; v < V; ++v) peak[v] = -INFINITY;
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        edge[i] = -1;
#pragma unroll
        for (int v = 0; v < V; ++v) value[i][v] = -INFINITY;
        if (static_cast<int64_t>(i) * P < degree) {
          const int64_t slot = begin + static_cast<int64_t>(i) * P + p;
          if (slot < end && live) {
            const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
            if (e >= 0) {
              edge[i] = e;
              const float envelope = env[e];
              const fvec<V> x = load_vec<V>(logit + e * channels + column);
#pragma unroll
              for (int v = 0; v < V; ++v) value[i][v] = effective_logit(x.v[v], envelope);
            }
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) peak[v] = fmaxf(peak[v], value[i][v]);
      }
      float null_value[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        peak[v] = across_max<LC>(peak[v]);
        null_value[v] = -INFINITY;
      }
      if (kNull && live) {
        const fvec<V> n0 = load_vec<V>(null_logit + segment * channels + column);
#pragma unroll
        for (int v = 0; v < V; ++v) null_value[v] = n0.v[v];
      }
      float total[V], null_weight[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (kNull) peak[v] = fmaxf(peak[v], null_value[v]);
        total[v] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        if (static_cast<int64_t>(i) * P < degree) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const float w = peak[v] > -INFINITY ? expf(value[i][v] - peak[v]) : 0.0f;
            value[i][v] = w;
            total[v] += w;
          }
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        total[v] = across_sum<LC>(total[v]);
        null_weight[v] = kNull && peak[v] > -INFINITY ? expf(null_value[v] - peak[v]) : 0.0f;
        total[v] = total[v] + null_weight[v];
        if (!(total[v] > 0.0f)) total[v] = 1.0f;
      }
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        if (static_cast<int64_t>(i) * P < degree && edge[i] >= 0) {
          fvec<V> out;
#pragma unroll
          for (int v = 0; v < V; ++v) out.v[v] = value[i][v] / total[v];
          store_vec_stream<V>(alpha + edge[i] * channels + column, out);
        }
      }
      if (kNull && p == 0 && live) {
        fvec<V> out;
#pragma unroll
        for (int v = 0; v < V; ++v) out.v[v] = null_weight[v] / total[v];
        store_vec<V>(null_alpha + segment * channels + column, out);
      }
    }
  }

  // ---- long segments: the whole block, three streaming passes -----------
  for (int w = 0; w < kWaves; ++w) {
    const int64_t segment = first + w;
    if (segment >= n_nodes) break;
    int64_t begin, end;
    segment_bounds(offsets, segment, n_edges, begin, end);
    if (end - begin <= RMAX * P) continue;
    const int64_t tiles = (end - begin + P - 1) / P;

    float peak[V];
#pragma unroll
    for (int v = 0; v < V; ++v) peak[v] = -INFINITY;
    for (int64_t t = wave; t < tiles; t += kWaves) {
      const int64_t slot = begin + t * P + p;
      if (slot < end && live) {
        const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) {
          const float envelope = env[e];
          const fvec<V> x = load_vec<V>(logit + e * channels + column);
#pragma unroll
          for (int v = 0; v < V; ++v) peak[v] = fmaxf(peak[v], effective_logit(x.v[v], envelope));
        }
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) peak[v] = across_max<LC>(peak[v]);
    if (p == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[wave][k * V + v] = peak[v];
    __syncthreads();
    float null_value[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float m = partial[0][k * V + v];
      for (int q = 1; q < kWaves; ++q) m = fmaxf(m, partial[q][k * V + v]);
      peak[v] = m;
      null_value[v] = -INFINITY;
    }
    if (kNull && live) {
      const fvec<V> n0 = load_vec<V>(null_logit + segment * channels + column);
#pragma unroll
      for (int v = 0; v < V; ++v) null_value[v] = n0.v[v];
    }
    if (kNull)
#pragma unroll
      for (int v = 0; v < V; ++v) peak[v] = fmaxf(peak[v], null_value[v]);
    __syncthreads();

    float total[V];
#pragma unroll
    for (int v = 0; v < V; ++v) total[v] = 0.0f;
    for (int64_t t = wave; t < tiles; t += kWaves) {
      const int64_t slot = begin + t * P + p;
      if (slot < end && live) {
        const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) {
          const float envelope = env[e];
          const fvec<V> x = load_vec<V>(logit + e * channels + column);
#pragma unroll
          for (int v = 0; v < V; ++v)
            if (peak[v] > -INFINITY) total[v] += expf(effective_logit(x.v[v], envelope) - peak[v]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) total[v] = across_sum<LC>(total[v]);
    if (p == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[wave][k * V + v] = total[v];
    __syncthreads();
    float null_weight[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float sum = partial[0][k * V + v];
      for (int q = 1; q < kWaves; ++q) sum = sum + partial[q][k * V + v];
      null_weight[v] = kNull && peak[v] > -INFINITY ? expf(null_value[v] - peak[v]) : 0.0f;
      sum = sum + null_weight[v];
      total[v] = sum > 0.0f ? sum : 1.0f;
    }
    __syncthreads();

    for (int64_t t = wave; t < tiles; t += kWaves) {
      const int64_t slot = begin + t * P + p;
      if (slot < end && live) {
        const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) {
          const float envelope = env[e];
          const fvec<V> x = load_vec<V>(logit + e * channels + column);
          fvec<V> out;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const float w8 = peak[v] > -INFINITY
                                 ? expf(effective_logit(x.v[v], envelope) - peak[v])
                                 : 0.0f;
            out.v[v] = w8 / total[v];
          }
          store_vec_stream<V>(alpha + e * channels + column, out);
        }
      }
    }
    if (kNull && wave == 0 && p == 0 && live) {
      fvec<V> out;
#pragma unroll
      for (int v = 0; v < V; ++v) out.v[v] = null_weight[v] / total[v];
      store_vec<V>(null_alpha + segment * channels + column, out);
    }
  }
}

template <int V, int LOG_LC, bool kNull, bool kOrdered>
__global__ __launch_bounds__(kBlock) void softmax_backward_kernel(
    const float* __restrict__ alpha, const float* __restrict__ grad_alpha,
    const float* __restrict__ env, const int64_t* __restrict__ offsets,
    const float* __restrict__ null_alpha, const float* __restrict__ grad_null_alpha,
    const int64_t* __restrict__ order, float* __restrict__ grad_logit,
    float* __restrict__ grad_null_logit, float* __restrict__ grad_env, int64_t n_edges,
    int64_t n_nodes, int64_t channels) {
  using S = Shape<LOG_LC>;
  constexpr int LC = S::LC, P = S::P, RMAX = S::RMAX;
  __shared__ float partial[kWaves][LC * V];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int k = lane & (LC - 1);
  const int p = lane >> LOG_LC;
  const bool live = k < channels / V;
  const int64_t column = static_cast<int64_t>(k) * V;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kWaves;

  {
    const int64_t segment = first + wave;
    int64_t begin = 0, end = 0;
    if (segment < n_nodes) segment_bounds(offsets, segment, n_edges, begin, end);
    if (segment < n_nodes && end - begin <= RMAX * P) {
      const int64_t degree = end - begin;
      float a[RMAX][V], ga[RMAX][V];
      int64_t edge[RMAX];
      float expect[V];
#pragma unroll
      for (int v = 0; v < V; ++v) expect[v] = 0.0f;
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        edge[i] = -1;
#pragma unroll
        for (int v = 0; v < V; ++v) a[i][v] = ga[i][v] = 0.0f;
        if (static_cast<int64_t>(i) * P < degree) {
          const int64_t slot = begin + static_cast<int64_t>(i) * P + p;
          if (slot < end && live) {
            const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
            if (e >= 0) {
              edge[i] = e;
              const fvec<V> x = load_vec<V>(alpha + e * channels + column);
              const fvec<V> g = load_vec<V>(grad_alpha + e * channels + column);
#pragma unroll
              for (int v = 0; v < V; ++v) {
                a[i][v] = x.v[v];
                ga[i][v] = g.v[v];
              }
            }
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) expect[v] = expect[v] + a[i][v] * ga[i][v];
      }
      float a0[V], g0[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        expect[v] = across_sum<LC>(expect[v]);
        a0[v] = g0[v] = 0.0f;
      }
      if (kNull && live) {
        const fvec<V> x = load_vec<V>(null_alpha + segment * channels + column);
        const fvec<V> g = load_vec<V>(grad_null_alpha + segment * channels + column);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          a0[v] = x.v[v];
          g0[v] = g.v[v];
        }
      }
      if (kNull)
#pragma unroll
        for (int v = 0; v < V; ++v) expect[v] = expect[v] + a0[v] * g0[v];
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        if (static_cast<int64_t>(i) * P < degree) {
          fvec<V> out;
          float row = 0.0f;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            out.v[v] = a[i][v] * (ga[i][v] - expect[v]);
            row += out.v[v];
          }
          row = group_sum<LC>(edge[i] >= 0 ? row : 0.0f);
          if (edge[i] >= 0) {
            store_vec_stream<V>(grad_logit + edge[i] * channels + column, out);
            if (k == 0) grad_env[edge[i]] = env_gradient(row, env[edge[i]]);
          }
        }
      }
      if (kNull && p == 0 && live) {
        fvec<V> out;
#pragma unroll
        for (int v = 0; v < V; ++v) out.v[v] = a0[v] * (g0[v] - expect[v]);
        store_vec<V>(grad_null_logit + segment * channels + column, out);
      }
    }
  }

  for (int w = 0; w < kWaves; ++w) {
    const int64_t segment = first + w;
    if (segment >= n_nodes) break;
    int64_t begin, end;
    segment_bounds(offsets, segment, n_edges, begin, end);
    if (end - begin <= RMAX * P) continue;
    const int64_t tiles = (end - begin + P - 1) / P;

    float expect[V];
#pragma unroll
    for (int v = 0; v < V; ++v) expect[v] = 0.0f;
    for (int64_t t = wave; t < tiles; t += kWaves) {
      const int64_t slot = begin + t * P + p;
      if (slot < end && live) {
        const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) {
          const fvec<V> x = load_vec<V>(alpha + e * channels + column);
          const fvec<V> g = load_vec<V>(grad_alpha + e * channels + column);
#pragma unroll
          for (int v = 0; v < V; ++v) expect[v] = expect[v] + x.v[v] * g.v[v];
        }
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) expect[v] = across_sum<LC>(expect[v]);
    if (p == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) partial[wave][k * V + v] = expect[v];
    __syncthreads();
    float a0[V], g0[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float sum = partial[0][k * V + v];
      for (int q = 1; q < kWaves; ++q) sum = sum + partial[q][k * V + v];
      expect[v] = sum;
      a0[v] = g0[v] = 0.0f;
    }
    __syncthreads();
    if (kNull && live) {
      const fvec<V> x = load_vec<V>(null_alpha + segment * channels + column);
      const fvec<V> g = load_vec<V>(grad_null_alpha + segment * channels + column);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        a0[v] = x.v[v];
        g0[v] = g.v[v];
      }
    }
    if (kNull)
#pragma unroll
      for (int v = 0; v < V; ++v) expect[v] = expect[v] + a0[v] * g0[v];

    for (int64_t t = wave; t < tiles; t += kWaves) {
      const int64_t slot = begin + t * P + p;
      int64_t e = -1;
      fvec<V> out;
      float row = 0.0f;
      if (slot < end && live) {
        e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) {
          const fvec<V> x = load_vec<V>(alpha + e * channels + column);
          const fvec<V> g = load_vec<V>(grad_alpha + e * channels + column);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            out.v[v] = x.v[v] * (g.v[v] - expect[v]);
            row += out.v[v];
          }
        }
      }
      row = group_sum<LC>(row);
      if (e >= 0) {
        store_vec_stream<V>(grad_logit + e * channels + column, out);
        if (k == 0) grad_env[e] = env_gradient(row, env[e]);
      }
    }
    if (kNull && wave == 0 && p == 0 && live) {
      fvec<V> out;
#pragma unroll
      for (int v = 0; v < V; ++v) out.v[v] = a0[v] * (g0[v] - expect[v]);
      store_vec<V>(grad_null_logit + segment * channels + column, out);
    }
  }
}

// ---- rows wider than 64 chunks: one wave per segment, lane per chunk ----

template <bool kOrdered>
__global__ __launch_bounds__(kBlock) void softmax_forward_wide_kernel(
    const float* __restrict__ logit, const float* __restrict__ env,
    const int64_t* __restrict__ offsets, const float* __restrict__ null_logit,
    const int64_t* __restrict__ order, float* __restrict__ alpha, float* __restrict__ null_alpha,
    int64_t n_edges, int64_t n_nodes, int64_t channels) {
  const int64_t segment = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (segment >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  for (int64_t c = lane; c < channels; c += 64) {
    float peak = -INFINITY;
    for (int64_t slot = begin; slot < end; ++slot) {
      const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
      if (e >= 0) peak = fmaxf(peak, effective_logit(logit[e * channels + c], env[e]));
    }
    const float null_value = null_logit != nullptr ? null_logit[segment * channels + c] : -INFINITY;
    if (null_logit != nullptr) peak = fmaxf(peak, null_value);
    float total = 0.0f;
    if (peak > -INFINITY)
      for (int64_t slot = begin; slot < end; ++slot) {
        const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) total = total + expf(effective_logit(logit[e * channels + c], env[e]) - peak);
      }
    const float null_weight =
        null_logit != nullptr && peak > -INFINITY ? expf(null_value - peak) : 0.0f;
    total = total + null_weight;
    if (!(total > 0.0f)) total = 1.0f;
    for (int64_t slot = begin; slot < end; ++slot) {
      const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
      if (e < 0) continue;
      const float w = peak > -INFINITY
                          ? expf(effective_logit(logit[e * channels + c], env[e]) - peak)
                          : 0.0f;
      alpha[e * channels + c] = w / total;
    }
    if (null_logit != nullptr) null_alpha[segment * channels + c] = null_weight / total;
  }
}

template <bool kOrdered>
__global__ __launch_bounds__(kBlock) void softmax_backward_wide_kernel(
    const float* __restrict__ alpha, const float* __restrict__ grad_alpha,
    const float* __restrict__ env, const int64_t* __restrict__ offsets,
    const float* __restrict__ null_alpha, const float* __restrict__ grad_null_alpha,
    const int64_t* __restrict__ order, float* __restrict__ grad_logit,
    float* __restrict__ grad_null_logit, float* __restrict__ grad_env, int64_t n_edges,
    int64_t n_nodes, int64_t channels) {
  const int64_t segment = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (segment >= n_nodes) return;
  const int lane = threadIdx.x & 63;
  int64_t begin, end;
  segment_bounds(offsets, segment, n_edges, begin, end);
  const bool has_null = null_alpha != nullptr;
  // Channel windows of 64 lanes; grad_env keeps the raw channel sum until the
  // last window, which applies the 2 / env factor.
  for (int64_t base = 0; base < channels; base += 64) {
    const int64_t c = base + lane;
    const bool live = c < channels;
    const bool last = base + 64 >= channels;
    float expect = 0.0f;
    if (live)
      for (int64_t slot = begin; slot < end; ++slot) {
        const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
        if (e >= 0) expect = expect + alpha[e * channels + c] * grad_alpha[e * channels + c];
      }
    if (has_null && live)
      expect = expect + null_alpha[segment * channels + c] * grad_null_alpha[segment * channels + c];
    for (int64_t slot = begin; slot < end; ++slot) {
      const int64_t e = edge_of<kOrdered>(order, slot, n_edges);
      if (e < 0) continue;
      float out = 0.0f;
      if (live) {
        out = alpha[e * channels + c] * (grad_alpha[e * channels + c] - expect);
        grad_logit[e * channels + c] = out;
      }
      float row = group_sum<64>(out);
      if (lane == 0) {
        if (base > 0) row = grad_env[e] + row;
        grad_env[e] = last ? env_gradient(row, env[e]) : row;
      }
    }
    if (has_null && live)
      grad_null_logit[segment * channels + c] =
          null_alpha[segment * channels + c] * (grad_null_alpha[segment * channels + c] - expect);
  }
}

int lanes_log_for(int64_t chunks) {
  int log = 0;
  while ((int64_t(1) << log) < chunks) ++log;
  return log;
}

template <int V, int LOG_LC>
int launch_forward(const float* logit, const float* env, const int64_t* offsets,
                   const float* null_logit, const int64_t* order, float* alpha, float* null_alpha,
                   int64_t n_edges, int64_t n_nodes, int64_t channels, hipStream_t stream) {
  const unsigned int grid = blocks_for(n_nodes, kWaves);
#define DPA4K_SOFTMAX_FWD(NULLV, ORD)                                                        \
  softmax_forward_kernel<V, LOG_LC, NULLV, ORD><<<grid, kBlock, 0, stream>>>(               \
      logit, env, offsets, null_logit, order, alpha, null_alpha, n_edges, n_nodes, channels)
  if (null_logit != nullptr) {
    if (order != nullptr) DPA4K_SOFTMAX_FWD(true, true); else DPA4K_SOFTMAX_FWD(true, false);
  } else {
    if (order != nullptr) DPA4K_SOFTMAX_FWD(false, true); else DPA4K_SOFTMAX_FWD(false, false);
  }
#undef DPA4K_SOFTMAX_FWD
  return launched("softmax_forward_kernel");
}

template <int V, int LOG_LC>
int launch_backward(const float* alpha, const float* grad_alpha, const float* env,
                    const int64_t* offsets, const float* null_alpha, const float* grad_null_alpha,
                    const int64_t* order, float* grad_logit, float* grad_null_logit,
                    float* grad_env, int64_t n_edges, int64_t n_nodes, int64_t channels,
                    hipStream_t stream) {
  const unsigned int grid = blocks_for(n_nodes, kWaves);
#define DPA4K_SOFTMAX_BWD(NULLV, ORD)                                                        \
  softmax_backward_kernel<V, LOG_LC, NULLV, ORD><<<grid, kBlock, 0, stream>>>(              \
      alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order, grad_logit,       \
      grad_null_logit, grad_env, n_edges, n_nodes, channels)
  if (null_alpha != nullptr) {
    if (order != nullptr) DPA4K_SOFTMAX_BWD(true, true); else DPA4K_SOFTMAX_BWD(true, false);
  } else {
    if (order != nullptr) DPA4K_SOFTMAX_BWD(false, true); else DPA4K_SOFTMAX_BWD(false, false);
  }
#undef DPA4K_SOFTMAX_BWD
  return launched("softmax_backward_kernel");
}

template <int V, typename... Args>
int dispatch_forward(int log_lc, Args... args) {
  switch (log_lc) {
    case 0: return launch_forward<V, 0>(args...);
    case 1: return launch_forward<V, 1>(args...);
    case 2: return launch_forward<V, 2>(args...);
    case 3: return launch_forward<V, 3>(args...);
    case 4: return launch_forward<V, 4>(args...);
    case 5: return launch_forward<V, 5>(args...);
    default: return launch_forward<V, 6>(args...);
  }
}

template <int V, typename... Args>
int dispatch_backward(int log_lc, Args... args) {
  switch (log_lc) {
    case 0: return launch_backward<V, 0>(args...);
    case 1: return launch_backward<V, 1>(args...);
    case 2: return launch_backward<V, 2>(args...);
    case 3: return launch_backward<V, 3>(args...);
    case 4: return launch_backward<V, 4>(args...);
    case 5: return launch_backward<V, 5>(args...);
    default: return launch_backward<V, 6>(args...);
  }
}

int check_common(int64_t n_edges, int64_t n_nodes, int64_t channels, const char* what) {
  if (n_edges < 0 || n_nodes < 0) return fail(DPA4K_EINVAL, "%s: negative sizes", what);
  if (channels <= 0) return fail(DPA4K_EINVAL, "%s requires at least one channel", what);
  if ((n_nodes + kWaves - 1) / kWaves > kMaxGrid)
    return fail(DPA4K_EINVAL, "%s: segment count too large", what);
  return DPA4K_OK;
}

}  // namespace
}  // namespace dpa4k

using namespace dpa4k;

extern "C" int dpa4k_segment_softmax_forward(const float* logit, const float* env,
                                             const int64_t* offsets, const float* null_logit,
                                             const int64_t* order, float* alpha, float* null_alpha,
                                             int64_t n_edges, int64_t n_nodes, int64_t channels,
                                             dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_common(n_edges, n_nodes, channels, "segment softmax")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr || (n_edges > 0 && (logit == nullptr || env == nullptr || alpha == nullptr)))
    return fail(DPA4K_EINVAL, "segment softmax: null pointer");
  if ((null_logit == nullptr) != (null_alpha == nullptr))
    return fail(DPA4K_EINVAL, "segment softmax: null_logit and null_alpha go together");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(logit) && aligned16(alpha) &&
                    (null_logit == nullptr || (aligned16(null_logit) && aligned16(null_alpha)));
  const int64_t chunks = vec4 ? channels / 4 : channels;
  if (chunks > 64) {
    const unsigned int grid = blocks_for(n_nodes, kWaves);
    if (order != nullptr)
      softmax_forward_wide_kernel<true><<<grid, kBlock, 0, stream>>>(
          logit, env, offsets, null_logit, order, alpha, null_alpha, n_edges, n_nodes, channels);
    else
      softmax_forward_wide_kernel<false><<<grid, kBlock, 0, stream>>>(
          logit, env, offsets, null_logit, order, alpha, null_alpha, n_edges, n_nodes, channels);
    return launched("softmax_forward_wide_kernel");
  }
  const int log_lc = lanes_log_for(chunks);
  return vec4 ? dispatch_forward<4>(log_lc, logit, env, offsets, null_logit, order, alpha,
                                    null_alpha, n_edges, n_nodes, channels, stream)
              : dispatch_forward<1>(log_lc, logit, env, offsets, null_logit, order, alpha,
                                    null_alpha, n_edges, n_nodes, channels, stream);
}

extern "C" int dpa4k_segment_softmax_backward(const float* alpha, const float* grad_alpha,
                                              const float* env, const int64_t* offsets,
                                              const float* null_alpha, const float* grad_null_alpha,
                                              const int64_t* order, float* grad_logit,
                                              float* grad_null_logit, float* grad_env,
                                              int64_t n_edges, int64_t n_nodes, int64_t channels,
                                              dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_common(n_edges, n_nodes, channels, "segment softmax backward")) return s;
  if (n_nodes == 0) return DPA4K_OK;
  if (offsets == nullptr ||
      (n_edges > 0 && (alpha == nullptr || grad_alpha == nullptr || env == nullptr ||
                       grad_logit == nullptr || grad_env == nullptr)))
    return fail(DPA4K_EINVAL, "segment softmax backward: null pointer");
  const bool has_null = null_alpha != nullptr;
  if (has_null != (grad_null_alpha != nullptr) || has_null != (grad_null_logit != nullptr))
    return fail(DPA4K_EINVAL,
                "segment softmax requires null_alpha and grad_null_alpha together");
  hipStream_t stream = as_stream(stream_handle);
  const bool vec4 = channels % 4 == 0 && aligned16(alpha) && aligned16(grad_alpha) &&
                    aligned16(grad_logit) &&
                    (!has_null || (aligned16(null_alpha) && aligned16(grad_null_alpha) &&
                                   aligned16(grad_null_logit)));
  const int64_t chunks = vec4 ? channels / 4 : channels;
  if (chunks > 64) {
    const unsigned int grid = blocks_for(n_nodes, kWaves);
    if (order != nullptr)
      softmax_backward_wide_kernel<true><<<grid, kBlock, 0, stream>>>(
          alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order, grad_logit,
          grad_null_logit, grad_env, n_edges, n_nodes, channels);
    else
      softmax_backward_wide_kernel<false><<<grid, kBlock, 0, stream>>>(
          alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order, grad_logit,
          grad_null_logit, grad_env, n_edges, n_nodes, channels);
    return launched("softmax_backward_wide_kernel");
  }
  const int log_lc = lanes_log_for(chunks);
  return vec4 ? dispatch_backward<4>(log_lc, alpha, grad_alpha, env, offsets, null_alpha,
                                     grad_null_alpha, order, grad_logit, grad_null_logit,
                                     grad_env, n_edges, n_nodes, channels, stream)
              : dispatch_backward<1>(log_lc, alpha, grad_alpha, env, offsets, null_alpha,
                                     grad_null_alpha, order, grad_logit, grad_null_logit,
                                     grad_env, n_edges, n_nodes, channels, stream);
}

// Edge-stream elementwise chain, fused into one pass: the reference's
// candidate C4 (docs/task2-hip-fusion-plan.md:280-300; designed there, not
// implemented).  DeepMD's SeZM blocks spend most of their elementwise time in
// chains of add_/mul/copy_ over [E, R, C] edge tensors (residual, gate,
// accumulate), each a separate pass over HBM; this kernel reads every input
// of such a chain once and writes its result once.
//
//   acc[e, r, c] = sum over k < n_terms, left to right, of (a_k * b_k) * coef_k
//   out[e, r, c] = act(acc[e, r, c])
//
// Every operand is an fp32 view over (edge, row, channel) given by three
// element strides; a zero stride broadcasts the operand along that axis, so a
// per-edge scalar, a per-row gate or a per-channel weight is a term factor
// like a full tensor.  b_k may be absent (factor 1).  Each product is rounded
// before the next operation (the library is built with -ffp-contract=off), so
// without an activation the result equals the eager fp32 chain
//   t_k = a_k * b_k;  t_k = t_k * coef_k;  acc = t_0 + t_1 + ...
// bit for bit.  Activations:
//   silu   act(x) = x * sigmoid(x)
//   gate   SeZM's gated activation: rows r with gate_row[r] < 0 (the scalar
//          channels) take silu; the others x * sigmoid(gate[e, gate_row[r], c])
// with sigmoid(x) = 1 / (1 + 2^(-x log2 e)) through v_exp_f32 / v_rcp_f32.
//
// One thread per chunk of V consecutive channels of one (edge, row): V = 4
// (one 16-byte load per operand) when C % 4 == 0 and every operand that
// varies along the channels is contiguous along them and 16-byte aligned,
// else V = 1.  The
// output is written with non-temporal stores.  Any size that fits in memory:
// the grid continues in rows along y past one grid row.
#include "common.h"

namespace dpa4k {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxTerms = DPA4K_EDGE_STREAM_MAX_TERMS;
constexpr int kMaxGateRows = DPA4K_EDGE_STREAM_MAX_GATE_ROWS;
constexpr float kLog2e = 1.4426950408889634f;

struct Operand {
  const float* base;
  int64_t edge, row, channel;  // element strides
};

struct CombineArgs {
  Operand a[kMaxTerms];
  Operand b[kMaxTerms];
  float coef[kMaxTerms];
  int b_is_one;  // bit k: term k has no second factor (b[k] repeats a[k])
  int n_terms;
  int activation;
  Operand gate;
  int8_t gate_row[kMaxGateRows];
  float* out;
  int64_t rows, channels;  // R, C
  int64_t chunks;          // E * R * C / V
};

// Operand (e, r, c .. c + V - 1).  With V = 4 every operand takes one
// 16-byte load, so no load sits in a branch: a channel-contiguous operand
// (16-byte aligned, checked on the host) loads its four values; a
// channel-broadcast one loads the aligned 16-byte block that holds its
// element and splats the element.  That block lies in the element's own
// page, so the load cannot leave mapped memory; the other bytes are unused.
template <int V>
__device__ __forceinline__ fvec<V> operand_value(const Operand& op, int64_t e, int64_t r, int64_t c) {
  const float* p = op.base + e * op.edge + r * op.row + c * op.channel;
  fvec<V> value;
  if constexpr (V == 1) {
    value.v[0] = *p;
  } else {
    const uint32_t slot = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) >> 2) & 3u;
    const fvec<4> raw = load_vec<4>(p - slot);  // the aligned block (float data is 4-byte aligned)
    // two selects (no branch): bit 0 picks within a pair, bit 1 the pair
    const bool odd = (slot & 1u) != 0u;
    const float low = odd ? raw.v[1] : raw.v[0];
    const float high = odd ? raw.v[3] : raw.v[2];
    const float element = (slot & 2u) != 0u ? high : low;
    const bool broadcast = op.channel == 0;
#pragma unroll
    for (int i = 0; i < V; ++i) value.v[i] = broadcast ? element : raw.v[i];
  }
  return value;
}

__device__ __forceinline__ float sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// kTerms terms, activation kAct.  Every load is unconditional: an absent
// second factor is loaded from its term's first factor (the host passes that
// operand twice) and replaced by 1 after the loads, and a row without a gate
// loads gate index 0 and ignores it.
template <int V, int kTerms, int kAct>
__global__ __launch_bounds__(kBlock) void edge_stream_combine_kernel(const CombineArgs args) {
  const int64_t q = block_index() * kBlock + threadIdx.x;
  if (q >= args.chunks) return;
  const int64_t chunks_per_row = args.channels / V;
  int64_t row_index, c, e, r;
  if (args.chunks > int64_t(0xffffffff)) {
    row_index = q / chunks_per_row;
    c = (q - row_index * chunks_per_row) * V;
    e = row_index / args.rows;
    r = row_index - e * args.rows;
  } else {
    // every index below 2^32: 32-bit divisions
    const uint32_t q32 = static_cast<uint32_t>(q);
    const uint32_t per = static_cast<uint32_t>(chunks_per_row);
    const uint32_t row32 = q32 / per;
    const uint32_t rows32 = static_cast<uint32_t>(args.rows);
    const uint32_t e32 = row32 / rows32;
    row_index = row32;
    c = static_cast<int64_t>(q32 - row32 * per) * V;
    e = e32;
    r = row32 - e32 * rows32;
  }

  // the gate index first (its load overlaps the operands'), then every operand
  const int gate_index = kAct == DPA4K_ACT_GATE ? args.gate_row[r] : -1;
  fvec<V> av[kTerms], bv[kTerms];
#pragma unroll
  for (int k = 0; k < kTerms; ++k) {
    av[k] = operand_value<V>(args.a[k], e, r, c);
    bv[k] = operand_value<V>(args.b[k], e, r, c);
  }
  fvec<V> gv;
  if constexpr (kAct == DPA4K_ACT_GATE) gv = operand_value<V>(args.gate, e, gate_index < 0 ? 0 : gate_index, c);

  fvec<V> acc;
#pragma unroll
  for (int k = 0; k < kTerms; ++k) {
    const bool one = ((args.b_is_one >> k) & 1) != 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float t = (av[k].v[i] * (one ? 1.0f : bv[k].v[i])) * args.coef[k];
      acc.v[i] = k == 0 ? t : acc.v[i] + t;
    }
  }
  if constexpr (kAct == DPA4K_ACT_SILU) {
#pragma unroll
    for (int i = 0; i < V; ++i) acc.v[i] = acc.v[i] * sigmoid(acc.v[i]);
  } else if constexpr (kAct == DPA4K_ACT_GATE) {
#pragma unroll
    for (int i = 0; i < V; ++i) acc.v[i] = acc.v[i] * sigmoid(gate_index < 0 ? acc.v[i] : gv.v[i]);
  }
  store_vec_stream<V>(args.out + row_index * args.channels + c, acc);
}

template <int V, int kTerms>
void launch_terms(const CombineArgs& args, dim3 grid, hipStream_t stream) {
  switch (args.activation) {
    case DPA4K_ACT_SILU:
      edge_stream_combine_kernel<V, kTerms, DPA4K_ACT_SILU><<<grid, kBlock, 0, stream>>>(args);
      break;
    case DPA4K_ACT_GATE:
      edge_stream_combine_kernel<V, kTerms, DPA4K_ACT_GATE><<<grid, kBlock, 0, stream>>>(args);
      break;
    default:
      edge_stream_combine_kernel<V, kTerms, DPA4K_ACT_NONE><<<grid, kBlock, 0, stream>>>(args);
  }
}

template <int V>
void launch_vector(const CombineArgs& args, dim3 grid, hipStream_t stream) {
  switch (args.n_terms) {
    case 1: launch_terms<V, 1>(args, grid, stream); break;
    case 2: launch_terms<V, 2>(args, grid, stream); break;
    case 3: launch_terms<V, 3>(args, grid, stream); break;
    default: launch_terms<V, 4>(args, grid, stream);
  }
}

bool vector_operand(const dpa4k_edge_operand& op) {
  // broadcast along the channels, or contiguous along them with 16-byte rows
  if (op.stride[2] == 0) return true;
  return op.stride[2] == 1 && aligned16(op.data) && op.stride[0] % 4 == 0 && op.stride[1] % 4 == 0;
}

Operand operand_of(const dpa4k_edge_operand& op) {
  return Operand{op.data, op.stride[0], op.stride[1], op.stride[2]};
}

bool strides_ok(const dpa4k_edge_operand& op) {
  return op.stride[0] >= 0 && op.stride[1] >= 0 && op.stride[2] >= 0;
}

}  // namespace
}  // namespace dpa4k

extern "C" int dpa4k_edge_stream_combine(const dpa4k_edge_operand* a, const dpa4k_edge_operand* b,
                                         const float* coef, int n_terms, int activation,
                                         const dpa4k_edge_operand* gate, const int32_t* gate_row,
                                         float* out, int64_t n_edges, int64_t n_rows, int64_t channels,
                                         dpa4k_stream_t stream_handle) {
  using namespace dpa4k;
  clear_error();
  if (n_edges < 0 || n_rows < 0 || channels < 0)
    return fail(DPA4K_EINVAL, "edge_stream_combine: negative shape");
  if (n_terms < 1 || n_terms > kMaxTerms)
    return fail(DPA4K_EINVAL, "edge_stream_combine: 1 to %d terms, got %d", kMaxTerms, n_terms);
  if (activation != DPA4K_ACT_NONE && activation != DPA4K_ACT_SILU && activation != DPA4K_ACT_GATE)
    return fail(DPA4K_EINVAL, "edge_stream_combine: unknown activation %d", activation);
  int64_t row_elements = 0, elements = 0;
  if (__builtin_mul_overflow(n_rows, channels, &row_elements) ||
      __builtin_mul_overflow(n_edges, row_elements, &elements))
    return fail(DPA4K_EINVAL, "edge_stream_combine: shape overflows 64 bits");
  if (elements == 0) return DPA4K_OK;
  if (a == nullptr || coef == nullptr) return fail(DPA4K_EINVAL, "edge_stream_combine: null term array");
  if (out == nullptr) return fail(DPA4K_EINVAL, "edge_stream_combine: null output");

  CombineArgs args{};
  bool vec = channels % 4 == 0 && aligned16(out);
  for (int k = 0; k < n_terms; ++k) {
    if (a[k].data == nullptr) return fail(DPA4K_EINVAL, "edge_stream_combine: term %d has no first factor", k);
    if (!strides_ok(a[k]) || (b != nullptr && b[k].data != nullptr && !strides_ok(b[k])))
      return fail(DPA4K_EINVAL, "edge_stream_combine: term %d has a negative stride", k);
    args.a[k] = operand_of(a[k]);
    vec = vec && vector_operand(a[k]);
    if (b != nullptr && b[k].data != nullptr) {
      args.b[k] = operand_of(b[k]);
      vec = vec && vector_operand(b[k]);
    } else {
      args.b[k] = args.a[k];
      args.b_is_one |= 1 << k;
    }
    args.coef[k] = coef[k];
  }
  args.n_terms = n_terms;
  args.activation = activation;
  if (activation == DPA4K_ACT_GATE) {
    if (n_rows > kMaxGateRows)
      return fail(DPA4K_EINVAL, "edge_stream_combine: the gate activation takes at most %d rows", kMaxGateRows);
    if (gate_row == nullptr) return fail(DPA4K_EINVAL, "edge_stream_combine: gate activation without gate rows");
    int32_t gates = 0;
    for (int64_t r = 0; r < n_rows; ++r) {
      if (gate_row[r] >= kMaxGateRows)
        return fail(DPA4K_EINVAL, "edge_stream_combine: gate row %d of row %lld out of range", gate_row[r],
                    static_cast<long long>(r));
      args.gate_row[r] = static_cast<int8_t>(gate_row[r] < 0 ? -1 : gate_row[r]);
      gates = gate_row[r] >= gates ? gate_row[r] + 1 : gates;
    }
    if (gates > 0) {
      if (gate == nullptr || gate->data == nullptr)
        return fail(DPA4K_EINVAL, "edge_stream_combine: gated rows without a gate tensor");
      if (!strides_ok(*gate)) return fail(DPA4K_EINVAL, "edge_stream_combine: gate has a negative stride");
      args.gate = operand_of(*gate);
      vec = vec && vector_operand(*gate);
    } else {
      args.gate = args.a[0];  // loaded (in bounds) and ignored: no row is gated
    }
  }
  args.out = out;
  args.rows = n_rows;
  args.channels = channels;
  const int V = vec ? 4 : 1;
  args.chunks = elements / V;
  const int64_t blocks = (args.chunks + kBlock - 1) / kBlock;
  if (!grid_fits(blocks, kBlock)) return fail(DPA4K_EINVAL, "edge_stream_combine: exceeds the launch limit");
  const dim3 grid = launch_grid(blocks, kBlock);
  hipStream_t stream = as_stream(stream_handle);
  if (vec)
    launch_vector<4>(args, grid, stream);
  else
    launch_vector<1>(args, grid, stream);
  return launched("edge_stream_combine_kernel");
}

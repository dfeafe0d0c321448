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
// The planned path (dpa4k_force_assembly_plan, once per graph; below) replaces
// that gather with a blocked two-level reduction over spatial blobs of edges.
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

// kRowViews: the gathered rows' array is under 2^31 bytes, so they are
// addressed through 32-bit offsets into a view of the whole array (one
// register per address, zeros for a lane without a row); otherwise through
// pointers at a clamped id, with the rows of invalid slots zeroed afterwards.
template <typename T, bool kRowViews>
__global__ __launch_bounds__(kBlock) void force_assembly_kernel(
    const T* __restrict__ grad_edge, const T* __restrict__ edge_vec,
    const int64_t* __restrict__ dst_offsets, const int64_t* __restrict__ src_offsets,
    const int64_t* __restrict__ src_order, T* __restrict__ force, T* __restrict__ virial, int64_t n_edges, int64_t n_nodes) {
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
  constexpr int64_t kSlotBytes = 8;
  const int64_t dst_base = (dst_begin - wave_dst) * 3 * static_cast<int64_t>(sizeof(T));
  const int64_t src_base = (src_begin - wave_src) * kSlotBytes;
  const bool dst_window = dst_base >= 0 && dst_base < int64_t(kNoRow) - kWindowBytes;
  const bool src_window = src_base >= 0 && src_base < int64_t(kNoRow) - kWindowBytes;

  const BufferView slots = buffer_view(src_order + wave_src, (n_edges - wave_src) * 8);
  int64_t edge[kSrcRounds];
#pragma unroll
  for (int r = 0; r < kSrcRounds; ++r) {
    const uint32_t offset =
        src_window ? static_cast<uint32_t>(src_base) + static_cast<uint32_t>(r * kGroup + lane) * kSlotBytes : kNoRow;
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

// ---------------------------------------------------------------------------
// planned path: spatial blobs of edges, partial sums per (blob, source atom)
// ---------------------------------------------------------------------------
//
// Plan (once per graph).  The atoms are put in a spatial order: positions are
// recovered from the edge vectors along a breadth-first tree of the graph
// (r_k = r_s - v_e for the edge e = (dst k, src s) that first reaches k), and
// the atoms are sorted by the Morton code of those positions.  Concatenating
// the destination segments in that order and cutting the result into windows
// of kBlobRows rows gives the blobs: each holds the incoming edges of a few
// dozen atoms that lie close together, so the sources of its edges repeat
// (about 6.5 edges per source at the config-4 shape).  A segment that crosses
// a window boundary is split into pieces, one per window.  Within each blob
// the edges are grouped by source atom, the atoms in their spatial order
// (the source slots listed position by position, then sorted stably by
// blob): a run of equal sources is a record.
//
// Pass 1 (force_blob_kernel, one workgroup per blob) reads the blob's rows
// (g_e, v_e) into LDS (the rows of a piece are contiguous in the inputs), sums
// each piece's g_e (the destination side, in double), and sums each record's
// -g_e and -(g_e outer v_e) from LDS: 12 values per record, in the value
// type (float32 records with fused products, float64 records in double).
// Pass 2 (force_records_kernel) adds, per atom, its pieces and its records in
// double in a fixed order (blob order) and writes force and virial.  Every
// sum has a fixed order: results are reproducible run to run.  They differ
// from the direct kernel's in the last bits (other association; float32
// records round each of their few terms).
//
// HBM bytes per call (f32, config 4: E = 5.9M, 916k records): the rows once
// (24 B per edge), the plan's row and entry indices (6 B per edge), the
// records written and read (2 x 48 B each), against the direct kernel's 12-byte
// random gathers that cost a line each.

constexpr int kBlobThreads = 512;
constexpr int64_t kBlobBytes = 67584;  // LDS rows of one blob: two workgroups per CU
constexpr int kRecordLanes = 16;       // pass 2: lanes per atom
constexpr int kScanBlock = 1024;       // elements per block of the plan's scans
constexpr int32_t kUnreached = 0x7fffffff;
constexpr int kMaxLevels = 4096;       // breadth-first levels before the rest count as unreached
constexpr int kBoxBlocks = 256;

template <typename T>
constexpr int64_t blob_rows_of() { return kBlobBytes / (6 * static_cast<int64_t>(sizeof(T))); }

int64_t blob_rows(int64_t value_bytes) { return kBlobBytes / (6 * value_bytes); }  // 2816 (f32), 1408 (f64)

int64_t blob_count(int64_t n_edges, int64_t value_bytes) {
  const int64_t rows = blob_rows(value_bytes);
  return (n_edges + rows - 1) / rows;
}

// Morton bits per axis: about one cell per atom.
int morton_bits(int64_t n_nodes) {
  int bits = 1;
  while (bits < 10 && (int64_t(1) << (3 * (bits + 1))) <= n_nodes) ++bits;
  return bits;
}

// A plan starts with a header naming what it was built for.  A planned call
// whose graph sizes, value size or record and piece counts differ from the
// header reads nothing else of the plan: it writes NaN into every output and
// DPA4K_FORCE_PLAN_MISMATCH into the caller's status word (every index inside
// a plan is consistent with its own graph size, so a plan of another graph of
// the same sizes gives wrong sums, never an access out of bounds).
constexpr int64_t kPlanMagic = 0x4e4c5046'34415044LL;  // "DPA4FPLN"
constexpr int kHeaderWords = 6;  // magic, n_edges, n_nodes, value_bytes, n_records, n_pieces

struct BlobPlan {
  int64_t* header;        // [kHeaderWords]
  int32_t* perm;          // [N] atoms in spatial order ("positions" below index perm)
  int32_t* piece_first;   // [N+1] first piece of each position; [N] = pieces
  int32_t* piece_t;       // [N+B+1] first concatenated row of each piece; [pieces] = E
  int32_t* blob_piece;    // [B+1] first piece of each blob; [B] = pieces
  int32_t* blob_rec;      // [B+1] first record of each blob; [B] = records
  int32_t* blob_entry;    // [B+1] first entry of each blob; [B] = valid entries
  int32_t* row_edge;      // [E] edge of each concatenated row
  uint16_t* entry_row;    // [E] blob row of each entry (entries: valid src slots sorted by blob, source, slot)
  int32_t* rec_entry;     // [E+1] first entry of each record; [records] = valid entries
  int32_t* pos_records;   // [E] record ids grouped by the position of their source atom, in blob order
  int32_t* pos_rec;       // [N+1] records of position i: pos_records[pos_rec[i] .. pos_rec[i+1])
};

bool carve_blob_plan(void* plan, size_t plan_bytes, int64_t n_edges, int64_t n_nodes, int64_t value_bytes,
                     BlobPlan& out) {
  Carver carver{static_cast<char*>(plan), plan_bytes};
  const size_t e = static_cast<size_t>(n_edges > 0 ? n_edges : 1), n = static_cast<size_t>(n_nodes);
  const size_t b = static_cast<size_t>(blob_count(n_edges, value_bytes));
  out.header = carver.take<int64_t>(kHeaderWords);
  out.perm = carver.take<int32_t>(n);
  out.piece_first = carver.take<int32_t>(n + 1);
  out.piece_t = carver.take<int32_t>(n + b + 1);
  out.blob_piece = carver.take<int32_t>(b + 1);
  out.blob_rec = carver.take<int32_t>(b + 1);
  out.blob_entry = carver.take<int32_t>(b + 1);
  out.row_edge = carver.take<int32_t>(e);
  out.entry_row = carver.take<uint16_t>(e);
  out.rec_entry = carver.take<int32_t>(e + 1);
  out.pos_records = carver.take<int32_t>(e);
  out.pos_rec = carver.take<int32_t>(n + 1);
  return out.header && out.perm && out.piece_first && out.piece_t && out.blob_piece && out.blob_rec && out.blob_entry &&
         out.row_edge && out.entry_row && out.rec_entry && out.pos_records && out.pos_rec;
}

size_t blob_plan_bytes(int64_t n_edges, int64_t n_nodes, int64_t value_bytes) {
  const size_t e = static_cast<size_t>(n_edges > 0 ? n_edges : 1), n = static_cast<size_t>(n_nodes);
  const size_t b = static_cast<size_t>(blob_count(n_edges, value_bytes));
  return round_up_256(kHeaderWords * 8) + round_up_256(n * 4) + round_up_256((n + 1) * 4) +
         round_up_256((n + b + 1) * 4) + 3 * round_up_256((b + 1) * 4) + round_up_256(e * 4) + round_up_256(e * 2) + round_up_256((e + 1) * 4) +
         round_up_256(e * 4) + round_up_256((n + 1) * 4);
}

// Records buffer of a plan: the pieces' destination sums (3 doubles each), then the records (12 values each).
size_t records_bytes_for(int64_t n_records, int64_t n_pieces, int64_t value_bytes) {
  return round_up_256(static_cast<size_t>(n_pieces > 0 ? n_pieces : 1) * 3 * 8) +
         round_up_256(static_cast<size_t>(n_records > 0 ? n_records : 1) * 12 * static_cast<size_t>(value_bytes));
}

struct BuildScratch {
  int32_t *edge_src, *slot_atom, *tpos, *level, *rank, *cum, *flags, *counts, *scanned, *scan_blocks, *lengths,
      *rec_old, *src_counts, *cum_src, *pslot;
  uint16_t* entry_old;
  float *pos, *box_part, *box;
  int64_t *key, *order, *key_offsets, *key2;
  int32_t* sort_status;
  void* sort;
  size_t sort_bytes;
};

int64_t morton_keys_of(int64_t n_nodes) { return (int64_t(1) << (3 * morton_bits(n_nodes))) + 1; }

// Records of a blob are ordered by descending length (entries, capped at kLengthKeys - 1), so
// that the 64 records a wave takes are of similar length.
constexpr int64_t kLengthKeys = 64;

size_t sort_keys_of(int64_t n_edges, int64_t n_nodes) {
  const size_t blobs = static_cast<size_t>(blob_count(n_edges, 4) > blob_count(n_edges, 8) ? blob_count(n_edges, 4)
                                                                                            : blob_count(n_edges, 8));
  size_t keys = blobs * kLengthKeys + 1;
  keys = static_cast<size_t>(n_nodes) > keys ? static_cast<size_t>(n_nodes) : keys;
  const size_t cells = static_cast<size_t>(morton_keys_of(n_nodes));
  return cells > keys ? cells : keys;
}

size_t build_sort_bytes(int64_t n_edges, int64_t n_nodes) {
  const int64_t blobs = blob_count(n_edges, 4) > blob_count(n_edges, 8) ? blob_count(n_edges, 4)
                                                                         : blob_count(n_edges, 8);
  size_t most = dpa4k_group_by_key_workspace_size(n_nodes, morton_keys_of(n_nodes));
  const size_t slots = dpa4k_group_by_key_workspace_size(n_edges, blobs + 1);
  const size_t records = dpa4k_group_by_key_workspace_size(n_edges, n_nodes);
  const size_t lengths = dpa4k_group_by_key_workspace_size(n_edges, blobs * kLengthKeys);
  most = slots > most ? slots : most;
  most = lengths > most ? lengths : most;
  return records > most ? records : most;
}

bool carve_build(void* workspace, size_t bytes, int64_t n_edges, int64_t n_nodes, BuildScratch& out) {
  Carver carver{static_cast<char*>(workspace), bytes};
  const size_t e = static_cast<size_t>(n_edges > 0 ? n_edges : 1), n = static_cast<size_t>(n_nodes);
  const size_t m = e > n ? e : n;
  const size_t keys = sort_keys_of(n_edges, n_nodes);
  out.edge_src = carver.take<int32_t>(e);
  out.slot_atom = carver.take<int32_t>(e);
  out.tpos = carver.take<int32_t>(e);
  out.level = carver.take<int32_t>(n);
  out.rank = carver.take<int32_t>(n);
  out.cum = carver.take<int32_t>(n + 1);
  out.flags = carver.take<int32_t>(kMaxLevels + 8);
  out.counts = carver.take<int32_t>(m + 1);
  out.scanned = carver.take<int32_t>(m + 1);
  out.scan_blocks = carver.take<int32_t>((m + 1) / kScanBlock + 2);
  out.lengths = carver.take<int32_t>(m + 1);
  out.rec_old = carver.take<int32_t>(m + 1);
  out.src_counts = carver.take<int32_t>(n + 1);
  out.cum_src = carver.take<int32_t>(n + 1);
  out.pslot = carver.take<int32_t>(e);
  out.entry_old = carver.take<uint16_t>(m);
  out.key2 = carver.take<int64_t>(m);
  out.pos = carver.take<float>(3 * n);
  out.box_part = carver.take<float>(kBoxBlocks * 6);
  out.box = carver.take<float>(8);
  out.key = carver.take<int64_t>(m);
  out.order = carver.take<int64_t>(m);
  out.key_offsets = carver.take<int64_t>(keys + 2);
  out.sort_status = carver.take<int32_t>(1);
  out.sort_bytes = build_sort_bytes(n_edges, n_nodes);
  out.sort = carver.take<char>(out.sort_bytes);
  return out.edge_src && out.slot_atom && out.tpos && out.level && out.rank && out.cum && out.flags &&
         out.counts && out.scanned && out.scan_blocks && out.lengths && out.rec_old && out.src_counts &&
         out.cum_src && out.pslot && out.entry_old && out.key2 &&
         out.pos && out.box_part && out.box && out.key && out.order && out.key_offsets && out.sort_status && out.sort;
}

size_t build_workspace_bytes(int64_t n_edges, int64_t n_nodes) {
  const size_t e = static_cast<size_t>(n_edges > 0 ? n_edges : 1), n = static_cast<size_t>(n_nodes);
  const size_t m = e > n ? e : n;
  const size_t keys = sort_keys_of(n_edges, n_nodes);
  return 3 * round_up_256(e * 4) + 2 * round_up_256(n * 4) + round_up_256((n + 1) * 4) +
         round_up_256((kMaxLevels + 8) * 4) + 2 * round_up_256((m + 1) * 4) +
         round_up_256(((m + 1) / kScanBlock + 2) * 4) + 2 * round_up_256((m + 1) * 4) +
         2 * round_up_256((n + 1) * 4) + round_up_256(e * 4) + round_up_256(m * 2) +
         round_up_256(m * 8) + round_up_256(3 * n * 4) + round_up_256(kBoxBlocks * 6 * 4) +
         round_up_256(8 * 4) + 2 * round_up_256(m * 8) + round_up_256((keys + 2) * 8) + round_up_256(4) +
         round_up_256(build_sort_bytes(n_edges, n_nodes));
}

unsigned int stride_blocks(int64_t items) {
  const int64_t wanted = (items + 255) / 256;
  return static_cast<unsigned int>(wanted < 1 ? 1 : (wanted > 8192 ? 8192 : wanted));
}

#define DPA4K_GRID_STRIDE(i, n) \
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (n); \
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)

// ---- exclusive scan of int32 counts: out[0..n], out[n] = total ----

// Exclusive prefix of `value` over a 256-thread block; `total` gets the block's sum.
__device__ __forceinline__ int32_t block_exclusive_256(int32_t value, int32_t* wave_sums, int32_t& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int32_t inclusive = value;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t other = __shfl_up(inclusive, d, 64);
    inclusive += lane >= d ? other : 0;
  }
  if (lane == 63) wave_sums[wave] = inclusive;
  __syncthreads();
  int32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int32_t s = wave_sums[w];
    before += w < wave ? s : 0;
    sum += s;
  }
  __syncthreads();
  total = sum;
  return before + inclusive - value;
}

__global__ __launch_bounds__(256) void scan_reduce_kernel(const int32_t* __restrict__ in, int64_t n,
                                                          int32_t* __restrict__ block_sums) {
  __shared__ int32_t wave_sums[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanBlock + threadIdx.x * 4;
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) sum += base + i < n ? in[base + i] : 0;
  int32_t total;
  block_exclusive_256(sum, wave_sums, total);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// One block: exclusive scan of the block sums in place, chunk by chunk.
__global__ __launch_bounds__(256) void scan_blocks_kernel(int32_t* __restrict__ block_sums, int64_t blocks) {
  __shared__ int32_t wave_sums[4];
  int32_t carry = 0;
  for (int64_t base = 0; base < blocks; base += 256) {
    const int64_t i = base + threadIdx.x;
    const int32_t value = i < blocks ? block_sums[i] : 0;
    int32_t total;
    const int32_t before = block_exclusive_256(value, wave_sums, total);
    if (i < blocks) block_sums[i] = carry + before;
    carry += total;
  }
  if (threadIdx.x == 0) block_sums[blocks] = carry;
}

__global__ __launch_bounds__(256) void scan_apply_kernel(const int32_t* __restrict__ in, int64_t n,
                                                         const int32_t* __restrict__ block_sums,
                                                         int32_t* __restrict__ out, int64_t blocks) {
  __shared__ int32_t wave_sums[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanBlock + threadIdx.x * 4;
  int32_t v[4], sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = base + i < n ? in[base + i] : 0;
    sum += v[i];
  }
  int32_t total;
  int32_t running = block_sums[blockIdx.x] + block_exclusive_256(sum, wave_sums, total);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (base + i < n) out[base + i] = running;
    running += v[i];
  }
  if (blockIdx.x == blocks - 1 && threadIdx.x == 0) out[n] = block_sums[blocks];
}

int scan_exclusive(const int32_t* in, int32_t* out, int64_t n, int32_t* block_sums, hipStream_t stream) {
  const int64_t blocks = (n + kScanBlock - 1) / kScanBlock > 0 ? (n + kScanBlock - 1) / kScanBlock : 1;
  scan_reduce_kernel<<<static_cast<unsigned int>(blocks), 256, 0, stream>>>(in, n, block_sums);
  if (int s = launched("scan_reduce_kernel")) return s;
  scan_blocks_kernel<<<1, 256, 0, stream>>>(block_sums, blocks);
  if (int s = launched("scan_blocks_kernel")) return s;
  scan_apply_kernel<<<static_cast<unsigned int>(blocks), 256, 0, stream>>>(in, n, block_sums, out, blocks);
  return launched("scan_apply_kernel");
}

// ---- plan kernels ----

// flags[0] |= 1 when an offsets array is not a CSR of n_edges slots; flags[1] = the first atom with incoming edges.
__global__ __launch_bounds__(256) void plan_check_kernel(const int64_t* __restrict__ dst_offsets,
                                                         const int64_t* __restrict__ src_offsets, int64_t n_edges,
                                                         int64_t n_nodes, int32_t* __restrict__ flags) {
  DPA4K_GRID_STRIDE(k, n_nodes + 1) {
    bool bad = false;
    for (int side = 0; side < 2; ++side) {
      const int64_t* offsets = side == 0 ? dst_offsets : src_offsets;
      const int64_t here = offsets[k];
      if (k == 0) bad |= here != 0;
      if (k == n_nodes) bad |= here != n_edges;
      if (k < n_nodes) bad |= offsets[k + 1] < here;
    }
    if (bad) flags[0] = 1;
    if (k < n_nodes && dst_offsets[k] == 0 && dst_offsets[k + 1] > 0) flags[1] = static_cast<int32_t>(k);
  }
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ out, int64_t n, int32_t value) {
  DPA4K_GRID_STRIDE(i, n) out[i] = value;
}

// Atom of every source slot, and the source atom of every edge a slot names
// (the largest such atom when src_order names an edge twice).
__global__ __launch_bounds__(256) void plan_slot_atoms_kernel(const int64_t* __restrict__ src_offsets,
                                                              const int64_t* __restrict__ src_order,
                                                              int32_t* __restrict__ slot_atom,
                                                              int32_t* __restrict__ edge_src, int64_t n_edges,
                                                              int64_t n_nodes) {
  DPA4K_GRID_STRIDE(q, n_edges) {
    int64_t low = 0, high = n_nodes;  // the last atom k with src_offsets[k] <= q
    while (high - low > 1) {
      const int64_t mid = (low + high) / 2;
      if (src_offsets[mid] <= q) low = mid; else high = mid;
    }
    slot_atom[q] = static_cast<int32_t>(low);
    const int64_t e = src_order[q];
    if (static_cast<uint64_t>(e) < static_cast<uint64_t>(n_edges)) atomicMax(&edge_src[e], static_cast<int32_t>(low));
  }
}

__global__ __launch_bounds__(256) void plan_bfs_init_kernel(int32_t* __restrict__ level, float* __restrict__ pos,
                                                            const int32_t* __restrict__ flags, int64_t n_nodes) {
  const int32_t root = flags[1];
  DPA4K_GRID_STRIDE(k, n_nodes) {
    level[k] = k == root ? 0 : kUnreached;
    pos[3 * k] = pos[3 * k + 1] = pos[3 * k + 2] = 0.0f;
  }
}

// Level `depth` of the breadth-first tree: every unreached atom takes as its
// parent the source of its first incoming edge whose source sits at `depth`,
// and its position from that edge's vector.  Reads only levels set by earlier
// launches, so the tree does not depend on the order threads run in.
template <typename T>
__global__ __launch_bounds__(256) void plan_bfs_level_kernel(const int64_t* __restrict__ dst_offsets,
                                                             const int32_t* __restrict__ edge_src,
                                                             const T* __restrict__ edge_vec,
                                                             int32_t* __restrict__ level, float* __restrict__ pos,
                                                             int32_t* __restrict__ flags, int32_t depth,
                                                             int64_t n_nodes) {
  int32_t* progress = flags + 8;  // progress[d]: some atom joined level d + 1
  if (depth > 0 && progress[depth - 1] == 0) return;
  DPA4K_GRID_STRIDE(k, n_nodes) {
    if (level[k] != kUnreached) continue;
    for (int64_t e = dst_offsets[k]; e < dst_offsets[k + 1]; ++e) {
      const int32_t s = edge_src[e];
      if (s < 0 || level[s] != depth) continue;
      pos[3 * k] = pos[3 * s] - static_cast<float>(edge_vec[3 * e]);
      pos[3 * k + 1] = pos[3 * s + 1] - static_cast<float>(edge_vec[3 * e + 1]);
      pos[3 * k + 2] = pos[3 * s + 2] - static_cast<float>(edge_vec[3 * e + 2]);
      level[k] = depth + 1;
      progress[depth] = 1;
      break;
    }
  }
}

__device__ __forceinline__ void box_reduce(float (&box)[6], float* lds) {
  // lds: [6][256]
#pragma unroll
  for (int i = 0; i < 6; ++i) lds[i * 256 + threadIdx.x] = box[i];
  __syncthreads();
  for (int width = 128; width > 0; width >>= 1) {
    if (threadIdx.x < width) {
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        lds[i * 256 + threadIdx.x] = fminf(lds[i * 256 + threadIdx.x], lds[i * 256 + threadIdx.x + width]);
        lds[(i + 3) * 256 + threadIdx.x] =
            fmaxf(lds[(i + 3) * 256 + threadIdx.x], lds[(i + 3) * 256 + threadIdx.x + width]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) box[i] = lds[i * 256];
}

__global__ __launch_bounds__(256) void plan_box_kernel(const float* __restrict__ pos,
                                                       const int32_t* __restrict__ level, int64_t n_nodes,
                                                       float* __restrict__ box_part) {
  __shared__ float lds[6 * 256];
  float box[6] = {INFINITY, INFINITY, INFINITY, -INFINITY, -INFINITY, -INFINITY};
  DPA4K_GRID_STRIDE(k, n_nodes) {
    if (level[k] == kUnreached) continue;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      box[i] = fminf(box[i], pos[3 * k + i]);
      box[i + 3] = fmaxf(box[i + 3], pos[3 * k + i]);
    }
  }
  box_reduce(box, lds);
  if (threadIdx.x < 6) box_part[blockIdx.x * 6 + threadIdx.x] = box[threadIdx.x];
}

__global__ __launch_bounds__(256) void plan_box_final_kernel(const float* __restrict__ box_part, int parts,
                                                             float* __restrict__ box_out) {
  __shared__ float lds[6 * 256];
  float box[6] = {INFINITY, INFINITY, INFINITY, -INFINITY, -INFINITY, -INFINITY};
  for (int p = threadIdx.x; p < parts; p += 256) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      box[i] = fminf(box[i], box_part[p * 6 + i]);
      box[i + 3] = fmaxf(box[i + 3], box_part[p * 6 + i + 3]);
    }
  }
  box_reduce(box, lds);
  if (threadIdx.x < 6) box_out[threadIdx.x] = box[threadIdx.x];
}

// Morton key of each reached atom's cell; unreached atoms after every cell.
__global__ __launch_bounds__(256) void plan_morton_kernel(const float* __restrict__ pos,
                                                          const int32_t* __restrict__ level,
                                                          const float* __restrict__ box, int64_t n_nodes, int bits,
                                                          int64_t* __restrict__ key) {
  const float extent = fmaxf(fmaxf(box[3] - box[0], box[4] - box[1]), box[5] - box[2]);
  const float cells = static_cast<float>(1 << bits);
  const float scale = extent > 0.0f && extent < INFINITY ? cells / extent : 0.0f;
  DPA4K_GRID_STRIDE(k, n_nodes) {
    if (level[k] == kUnreached) {
      key[k] = int64_t(1) << (3 * bits);
      continue;
    }
    uint32_t q[3];
#pragma unroll
    for (int i = 0; i < 3; ++i)
      q[i] = static_cast<uint32_t>(fminf(fmaxf((pos[3 * k + i] - box[i]) * scale, 0.0f), cells - 1.0f));
    int64_t code = 0;
    for (int b = 0; b < bits; ++b)
#pragma unroll
      for (int i = 0; i < 3; ++i) code |= static_cast<int64_t>((q[i] >> b) & 1u) << (3 * b + (2 - i));
    key[k] = code;
  }
}

// perm, rank, and the destination and source degrees of each position of perm.
__global__ __launch_bounds__(256) void plan_perm_kernel(const int64_t* __restrict__ order,
                                                        const int64_t* __restrict__ dst_offsets,
                                                        const int64_t* __restrict__ src_offsets,
                                                        int32_t* __restrict__ perm, int32_t* __restrict__ rank,
                                                        int32_t* __restrict__ degree,
                                                        int32_t* __restrict__ src_degree, int64_t n_nodes) {
  DPA4K_GRID_STRIDE(i, n_nodes) {
    const int64_t a = order[i];
    perm[i] = static_cast<int32_t>(a);
    rank[a] = static_cast<int32_t>(i);
    degree[i] = static_cast<int32_t>(dst_offsets[a + 1] - dst_offsets[a]);
    src_degree[i] = static_cast<int32_t>(src_offsets[a + 1] - src_offsets[a]);
  }
}

// Pieces of position i of perm: one per window of `rows` concatenated rows its segment meets.
__global__ __launch_bounds__(256) void plan_piece_counts_kernel(const int32_t* __restrict__ cum,
                                                                int32_t* __restrict__ count, int64_t n_nodes,
                                                                int64_t rows) {
  DPA4K_GRID_STRIDE(i, n_nodes) {
    const int64_t begin = cum[i], end = cum[i + 1];
    count[i] = end > begin ? static_cast<int32_t>((end - 1) / rows - begin / rows + 1) : 0;
  }
}

__global__ __launch_bounds__(256) void plan_pieces_kernel(const int32_t* __restrict__ cum,
                                                          const int32_t* __restrict__ piece_first,
                                                          int32_t* __restrict__ piece_t,
                                                          int32_t* __restrict__ blob_piece, int64_t n_nodes,
                                                          int64_t rows, int64_t n_edges, int64_t blobs) {
  DPA4K_GRID_STRIDE(i, n_nodes) {
    const int64_t begin = cum[i], end = cum[i + 1];
    if (end <= begin) continue;
    const int64_t w0 = begin / rows;
    for (int64_t w = w0; w <= (end - 1) / rows; ++w) {
      const int64_t id = piece_first[i] + (w - w0);
      const int64_t start = begin > w * rows ? begin : w * rows;
      piece_t[id] = static_cast<int32_t>(start);
      if (start == w * rows) blob_piece[w] = static_cast<int32_t>(id);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int32_t pieces = piece_first[n_nodes];
    piece_t[pieces] = static_cast<int32_t>(n_edges);
    blob_piece[blobs] = pieces;
  }
}

// Concatenated row of every edge, and the edge of every row.
__global__ __launch_bounds__(256) void plan_rows_kernel(const int64_t* __restrict__ dst_offsets,
                                                        const int32_t* __restrict__ rank,
                                                        const int32_t* __restrict__ cum, int32_t* __restrict__ tpos,
                                                        int32_t* __restrict__ row_edge, int64_t n_edges,
                                                        int64_t n_nodes) {
  DPA4K_GRID_STRIDE(e, n_edges) {
    int64_t low = 0, high = n_nodes;  // the last atom k with dst_offsets[k] <= e
    while (high - low > 1) {
      const int64_t mid = (low + high) / 2;
      if (dst_offsets[mid] <= e) low = mid; else high = mid;
    }
    const int64_t t = cum[rank[low]] + (e - dst_offsets[low]);
    tpos[e] = static_cast<int32_t>(t);
    row_edge[t] = static_cast<int32_t>(e);
  }
}

// The source slots listed position by position: pslot[j] for j in the
// concatenation of the positions' source segments (cum_src its prefix).
// Sorting this list stably by blob puts a blob's records in the spatial order
// of their source atoms, so that atoms near each other in pass 2 find their
// records near each other (records pass 17.8 -> 15.5 us at config 4 f32,
// against the slots in atom-id order).
__global__ __launch_bounds__(256) void plan_source_slots_kernel(const int32_t* __restrict__ cum_src,
                                                                const int32_t* __restrict__ perm,
                                                                const int64_t* __restrict__ src_offsets,
                                                                int32_t* __restrict__ pslot, int64_t n_edges,
                                                                int64_t n_nodes) {
  DPA4K_GRID_STRIDE(j, n_edges) {
    int64_t low = 0, high = n_nodes;  // the last position i with cum_src[i] <= j (it has a slot)
    while (high - low > 1) {
      const int64_t mid = (low + high) / 2;
      if (cum_src[mid] <= j) low = mid; else high = mid;
    }
    pslot[j] = static_cast<int32_t>(src_offsets[perm[low]] + (j - cum_src[low]));
  }
}

// Blob of the edge of every listed source slot; `blobs` for a slot whose src_order entry is out of range.
__global__ __launch_bounds__(256) void plan_slot_keys_kernel(const int64_t* __restrict__ src_order,
                                                             const int32_t* __restrict__ pslot,
                                                             const int32_t* __restrict__ tpos,
                                                             int64_t* __restrict__ key, int64_t n_edges, int64_t rows,
                                                             int64_t blobs) {
  DPA4K_GRID_STRIDE(j, n_edges) {
    const int64_t e = src_order[pslot[j]];
    key[j] = static_cast<uint64_t>(e) < static_cast<uint64_t>(n_edges) ? tpos[e] / rows : blobs;
  }
}

// Entries (listed slots sorted stably by blob: by blob, source position,
// slot): their blob rows, and a 1 where a record starts (a new blob or a new
// source atom).
__global__ __launch_bounds__(256) void plan_entries_kernel(const int64_t* __restrict__ order,
                                                           const int64_t* __restrict__ key,
                                                           const int32_t* __restrict__ pslot,
                                                           const int64_t* __restrict__ src_order,
                                                           const int32_t* __restrict__ slot_atom,
                                                           const int32_t* __restrict__ tpos,
                                                           uint16_t* __restrict__ entry_row,
                                                           int32_t* __restrict__ starts, int64_t n_edges, int64_t rows,
                                                           int64_t blobs) {
  DPA4K_GRID_STRIDE(j, n_edges) {
    const int64_t listed = order[j];
    const int64_t blob = key[listed];
    const int32_t q = pslot[listed];
    const bool valid = blob < blobs;
    entry_row[j] = valid ? static_cast<uint16_t>(tpos[src_order[q]] - blob * rows) : uint16_t(0);
    bool start = valid;
    if (valid && j > 0) {
      const int64_t previous = order[j - 1];
      start = key[previous] != blob || slot_atom[pslot[previous]] != slot_atom[q];
    }
    starts[j] = start ? 1 : 0;
  }
}

__global__ __launch_bounds__(256) void plan_records_kernel(const int32_t* __restrict__ starts,
                                                           const int32_t* __restrict__ record_of,
                                                           const int64_t* __restrict__ key_offsets,
                                                           int32_t* __restrict__ rec_entry,
                                                           int32_t* __restrict__ blob_rec,
                                                           int32_t* __restrict__ blob_entry, int64_t n_edges,
                                                           int64_t blobs) {
  DPA4K_GRID_STRIDE(j, n_edges) {
    if (starts[j]) rec_entry[record_of[j]] = static_cast<int32_t>(j);
  }
  DPA4K_GRID_STRIDE(b, blobs + 1) {
    blob_rec[b] = record_of[key_offsets[b]];
    blob_entry[b] = static_cast<int32_t>(key_offsets[b]);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) rec_entry[record_of[n_edges]] = static_cast<int32_t>(key_offsets[blobs]);
}

// Key of each record (in source position order within its blob): its blob,
// then its length descending; the record's length and source atom on the side.
__global__ __launch_bounds__(256) void plan_length_keys_kernel(const int32_t* __restrict__ rec_old,
                                                               const int64_t* __restrict__ order,
                                                               const int64_t* __restrict__ slot_key,
                                                               const int32_t* __restrict__ pslot,
                                                               const int32_t* __restrict__ slot_atom,
                                                               int64_t* __restrict__ key, int32_t* __restrict__ length,
                                                               int32_t* __restrict__ rec_atom, int64_t records) {
  DPA4K_GRID_STRIDE(r, records) {
    const int32_t n = rec_old[r + 1] - rec_old[r];
    const int64_t listed = order[rec_old[r]];
    key[r] = slot_key[listed] * kLengthKeys + (kLengthKeys - 1 - (n < kLengthKeys - 1 ? n : kLengthKeys - 1));
    length[r] = n;
    rec_atom[r] = slot_atom[pslot[listed]];
  }
}

__global__ __launch_bounds__(256) void plan_gather_i32_kernel(const int64_t* __restrict__ order,
                                                              const int32_t* __restrict__ in,
                                                              int32_t* __restrict__ out, int64_t n) {
  DPA4K_GRID_STRIDE(k, n) out[k] = in[order[k]];
}

// Record k of the balanced order is old record order[k]: its entries move to
// [first[k], first[k + 1]); the key of its source atom's position goes to key[k].
__global__ __launch_bounds__(256) void plan_move_entries_kernel(const int64_t* __restrict__ order,
                                                                const int32_t* __restrict__ rec_old,
                                                                const uint16_t* __restrict__ entry_old,
                                                                const int32_t* __restrict__ first,
                                                                const int32_t* __restrict__ rec_atom,
                                                                const int32_t* __restrict__ rank,
                                                                uint16_t* __restrict__ entry_row,
                                                                int32_t* __restrict__ rec_entry,
                                                                int64_t* __restrict__ key, int64_t records) {
  DPA4K_GRID_STRIDE(k, records) {
    const int64_t old = order[k];
    const int32_t from = rec_old[old], count = rec_old[old + 1] - from, to = first[k];
    for (int32_t i = 0; i < count; ++i) entry_row[to + i] = entry_old[from + i];
    rec_entry[k] = to;
    key[k] = rank[rec_atom[old]];
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) rec_entry[records] = first[records];
}

// Records sorted stably by position.
__global__ __launch_bounds__(256) void plan_record_slots_kernel(const int64_t* __restrict__ order,
                                                                const int64_t* __restrict__ key_offsets,
                                                                int32_t* __restrict__ pos_records,
                                                                int32_t* __restrict__ pos_rec, int64_t records,
                                                                int64_t n_nodes) {
  DPA4K_GRID_STRIDE(k, records) pos_records[k] = static_cast<int32_t>(order[k]);
  DPA4K_GRID_STRIDE(i, n_nodes + 1) pos_rec[i] = static_cast<int32_t>(key_offsets[i]);
}

// ---- the two passes of a planned call ----

// v clamped to [low, high].
__device__ __forceinline__ int32_t clamp_i32(int32_t v, int32_t low, int32_t high) {
  return v < low ? low : (v > high ? high : v);
}

struct BlobView;
template <typename T>
__device__ __forceinline__ bool plan_matches(const BlobView& plan, int64_t n_edges, int64_t n_nodes,
                                             int32_t n_records, int32_t n_pieces);

struct BlobView {
  const int64_t* header;
  const int32_t *perm, *piece_first, *piece_t, *blob_piece, *blob_rec, *blob_entry, *row_edge, *rec_entry,
      *pos_records, *pos_rec;
  const uint16_t* entry_row;
};

// The six header words are read together: a chain of short-circuit compares
// waits for each load before issuing the next (records pass 17.8 -> 15.6 us
// at config 4 f32).
template <typename T>
__device__ __forceinline__ bool plan_matches(const BlobView& plan, int64_t n_edges, int64_t n_nodes,
                                             int32_t n_records, int32_t n_pieces) {
  int64_t h[kHeaderWords];
#pragma unroll
  for (int i = 0; i < kHeaderWords; ++i) h[i] = plan.header[i];
  return (h[0] == kPlanMagic) & (h[1] == n_edges) & (h[2] == n_nodes) & (h[3] == static_cast<int64_t>(sizeof(T))) &
         (h[4] == n_records) & (h[5] == n_pieces);
}

template <typename T>
__device__ __forceinline__ void store_record(T* __restrict__ out, const T (&acc)[12]) {
  if constexpr (sizeof(T) == 4) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4* v = reinterpret_cast<f32x4*>(out);  // 48-byte records: 16-byte aligned
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = f32x4{acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]};
  } else {
    typedef double f64x2 __attribute__((ext_vector_type(2)));
    f64x2* v = reinterpret_cast<f64x2*>(out);
#pragma unroll
    for (int i = 0; i < 6; ++i) v[i] = f64x2{acc[2 * i], acc[2 * i + 1]};
  }
}

// Destination sums of pieces [0, count) of a blob, kPieceLanes lanes per
// piece: piece p covers the blob's LDS rows [bound(p) - t0, bound(p + 1) -
// t0); lane l sums rows l, l + kPieceLanes, ... in order, then a fixed
// butterfly adds the lanes.
constexpr int kPieceLanes = 8;


template <typename T, typename Bound>
__device__ __forceinline__ void blob_pieces(const T* rows, int32_t count, int64_t t0, int32_t piece0, Bound bound,
                                            double* __restrict__ dst_rec) {
  const int group = threadIdx.x / kPieceLanes, sub = threadIdx.x % kPieceLanes;
  for (int32_t p = group; p < count; p += kBlobThreads / kPieceLanes) {
    const int32_t begin = static_cast<int32_t>(bound(p) - t0), end = static_cast<int32_t>(bound(p + 1) - t0);
    double s0 = 0.0, s1 = 0.0, s2 = 0.0;
    for (int32_t row = begin + sub; row < end; row += kPieceLanes) {
      s0 += static_cast<double>(rows[row * 6]);
      s1 += static_cast<double>(rows[row * 6 + 1]);
      s2 += static_cast<double>(rows[row * 6 + 2]);
    }
    s0 = group_sum<kPieceLanes>(s0);
    s1 = group_sum<kPieceLanes>(s1);
    s2 = group_sum<kPieceLanes>(s2);
    if (sub < 3) dst_rec[static_cast<int64_t>(piece0 + p) * 3 + sub] = sub == 0 ? s0 : (sub == 1 ? s1 : s2);
  }
}

// Twelve source sums of one record: entries [from, to), their blob rows from `row_of`.
// acc -= the twelve source products of one row, in the accumulator's precision.
template <typename A, typename T>
__device__ __forceinline__ void sub_source(A (&acc)[12], const T* r6) {
  const A g0 = r6[0], g1 = r6[1], g2 = r6[2], v0 = r6[3], v1 = r6[4], v2 = r6[5];
  acc[0] -= g0;
  acc[1] -= g1;
  acc[2] -= g2;
  if constexpr (sizeof(A) == 4) {  // float32 records: one rounding per product and sum (fused)
    acc[3] = __builtin_fmaf(-g0, v0, acc[3]);
    acc[4] = __builtin_fmaf(-g0, v1, acc[4]);
    acc[5] = __builtin_fmaf(-g0, v2, acc[5]);
    acc[6] = __builtin_fmaf(-g1, v0, acc[6]);
    acc[7] = __builtin_fmaf(-g1, v1, acc[7]);
    acc[8] = __builtin_fmaf(-g1, v2, acc[8]);
    acc[9] = __builtin_fmaf(-g2, v0, acc[9]);
    acc[10] = __builtin_fmaf(-g2, v1, acc[10]);
    acc[11] = __builtin_fmaf(-g2, v2, acc[11]);
  } else {
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
}

// Twelve source sums of one record: entries [from, to), their blob rows from
// `row_of`.  A record holds a few edges (6.5 on average at config 4) and is
// stored in the value type, so float32 records accumulate in float32 with
// fused products; float64 records in double.
template <typename T, typename RowOf>
__device__ __forceinline__ void blob_record(const T* rows, int32_t from, int32_t to, RowOf row_of,
                                            T* __restrict__ out) {
  T acc[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) acc[i] = T(0);
  int32_t j = from;
  const auto row = [&](int32_t k) { return rows + row_of(k) * 6; };
  for (; j + 2 <= to; j += 2) {  // two entries' reads in flight; the sums stay in entry order
    const T* a = row(j);
    const T* b = row(j + 1);
    T ra[6], rb[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      ra[i] = a[i];
      rb[i] = b[i];
    }
    sub_source(acc, ra);
    sub_source(acc, rb);
  }
  if (j < to) sub_source(acc, row(j));
  store_record(out, acc);
}

// Pass 1: one workgroup per blob.  Every global load of the blob is issued
// before any LDS work: the rows' edge ids, the blob's entries and piece
// bounds (contiguous in the plan), each thread's record bounds and slots,
// then the rows (g_e, v_e) themselves (consecutive threads read consecutive
// rows of a piece).  After one barrier eight lanes sum each piece's g and
// each thread a record's twelve products (the records of a blob come
// longest first, so a wave's records are of similar length), from LDS only,
// and the record is stored at its id (a blob's records are contiguous).  A blob with more entries than rows
// (src_order naming an edge twice) or more pieces than threads reads those
// from the plan instead: a branch uniform over the workgroup, so the common
// case's loops hold no global load.
template <typename T>
__global__ __launch_bounds__(kBlobThreads) void force_blob_kernel(const T* __restrict__ grad_edge,
                                                                  const T* __restrict__ edge_vec, BlobView plan,
                                                                  double* __restrict__ dst_rec,
                                                                  T* __restrict__ src_rec, int64_t n_edges,
                                                                  int64_t n_nodes, int64_t blobs, int32_t n_records,
                                                                  int32_t n_pieces) {
  constexpr int64_t kRows = blob_rows_of<T>();
  constexpr int kRounds = static_cast<int>((kRows + kBlobThreads - 1) / kBlobThreads);
  __shared__ T rows[kRows * 6];
  __shared__ uint16_t entries[kRows];
  __shared__ int32_t bounds[kBlobThreads];
  // each XCD takes a contiguous range of blobs (so of atom positions): pass 2 on
  // that XCD then reads the records its L2 received
  const int64_t blob = static_cast<int64_t>(blockIdx.y) * gridDim.x + xcd_block(blockIdx.x, gridDim.x);
  if (blob >= blobs || !plan_matches<T>(plan, n_edges, n_nodes, n_records, n_pieces)) return;
  const int tid = static_cast<int>(threadIdx.x);
  const int64_t t0 = blob * kRows;
  const int64_t count = n_edges - t0 < kRows ? n_edges - t0 : kRows;
  // a plan's own extents are consistent; the caller's record and piece counts bound them
  const int32_t edges = static_cast<int32_t>(n_edges);
  const int32_t entry0 = clamp_i32(plan.blob_entry[blob], 0, edges);
  const int32_t entry_count = clamp_i32(plan.blob_entry[blob + 1], entry0, edges) - entry0;
  const int32_t piece0 = clamp_i32(plan.blob_piece[blob], 0, n_pieces);
  const int32_t piece_count = clamp_i32(plan.blob_piece[blob + 1], piece0, n_pieces) - piece0;
  const int32_t rec0 = clamp_i32(plan.blob_rec[blob], 0, n_records);
  const int32_t rec1 = clamp_i32(plan.blob_rec[blob + 1], rec0, n_records);
  const bool staged_entries = entry_count <= kRows;
  const bool staged_pieces = piece_count < kBlobThreads;

  // thread t takes record t of the blob (records come longest first, so the
  // lanes of a wave take records of similar length); any records past the
  // first kBlobThreads are taken in the loop below
  const int32_t my_record = rec0 + tid;
  int32_t edge[kRounds], entry[kRounds];
  const int32_t bound = plan.piece_t[piece0 + (tid <= piece_count ? tid : 0)];
  const int32_t first = plan.rec_entry[my_record < rec1 ? my_record : rec0];
  const int32_t last = plan.rec_entry[(my_record < rec1 ? my_record : rec0) + 1];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int32_t i = r * kBlobThreads + tid;
    edge[r] = plan.row_edge[t0 + (i < count ? i : count - 1)];
    entry[r] = plan.entry_row[entry0 + (i < entry_count ? i : 0)];
  }
  Row3<T> g[kRounds], v[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    g[r] = load_row(grad_edge, edge[r]);
    v[r] = load_row(edge_vec, edge[r]);
  }
  if (tid <= piece_count && staged_pieces) bounds[tid] = bound;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int32_t i = r * kBlobThreads + tid;
    if (i < entry_count && staged_entries) entries[i] = static_cast<uint16_t>(entry[r]);
    if (i < count) {
      T* at = rows + i * 6;
      at[0] = g[r].x; at[1] = g[r].y; at[2] = g[r].z;
      at[3] = v[r].x; at[4] = v[r].y; at[5] = v[r].z;
    }
  }
  __syncthreads();

  if (staged_pieces)
    blob_pieces(rows, piece_count, t0, piece0, [&](int32_t p) { return bounds[p]; }, dst_rec);
  else
    blob_pieces(rows, piece_count, t0, piece0, [&](int32_t p) { return plan.piece_t[piece0 + p]; }, dst_rec);

  if (staged_entries) {
    auto row_of = [&](int32_t j) { return static_cast<int32_t>(entries[j - entry0]); };
    if (my_record < rec1) blob_record(rows, first, last, row_of, src_rec + static_cast<int64_t>(my_record) * 12);
    for (int32_t rec = rec0 + kBlobThreads + tid; rec < rec1; rec += kBlobThreads)
      blob_record(rows, plan.rec_entry[rec], plan.rec_entry[rec + 1], row_of, src_rec + static_cast<int64_t>(rec) * 12);
  } else {
    auto row_of = [&](int32_t j) { return static_cast<int32_t>(plan.entry_row[j]); };
    for (int32_t rec = rec0 + tid; rec < rec1; rec += kBlobThreads)
      blob_record(rows, plan.rec_entry[rec], plan.rec_entry[rec + 1], row_of, src_rec + static_cast<int64_t>(rec) * 12);
  }
}

// Pass 2: kRecordLanes lanes per position of perm; lane c < 12 adds
// component c of the position's pieces (c < 3) and of its records, in blob
// order, and writes it for the atom.  The group loads up to kRecordLanes
// record ids at once (one per lane) and then every record's 48 bytes.
template <typename T>
__global__ __launch_bounds__(256) void force_records_kernel(BlobView plan, const double* __restrict__ dst_rec,
                                                            const T* __restrict__ src_rec, T* __restrict__ force,
                                                            T* __restrict__ virial, int64_t n_edges, int64_t n_nodes,
                                                            int32_t n_records, int32_t n_pieces,
                                                            int32_t* __restrict__ status) {
  const int64_t block = static_cast<int64_t>(blockIdx.y) * gridDim.x + xcd_block(blockIdx.x, gridDim.x);
  const int64_t i = block * (256 / kRecordLanes) + threadIdx.x / kRecordLanes;
  const bool match = plan_matches<T>(plan, n_edges, n_nodes, n_records, n_pieces);
  if (status != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
    *status = match ? 0 : DPA4K_FORCE_PLAN_MISMATCH;
  if (i >= n_nodes) return;
  const int c = threadIdx.x & (kRecordLanes - 1);
  if (!match) {  // nothing of the plan is read: atom i of this position's slot gets NaN
    const T nan = __builtin_nan("");
    if (c < 3)
      force[i * 3 + c] = nan;
    else if (c < 12)
      virial[i * 9 + (c - 3)] = nan;
    return;
  }
  const int32_t atom = plan.perm[i];
  const int32_t piece0 = clamp_i32(plan.piece_first[i], 0, n_pieces);
  const int32_t piece1 = clamp_i32(plan.piece_first[i + 1], piece0, n_pieces);
  const int32_t rec0 = clamp_i32(plan.pos_rec[i], 0, n_records);
  const int32_t rec1 = clamp_i32(plan.pos_rec[i + 1], rec0, n_records);
  const int cc = c < 12 ? c : 0;
  double acc = 0.0;
  for (int32_t p = piece0; p < piece1; ++p) acc += c < 3 ? dst_rec[static_cast<int64_t>(p) * 3 + c] : 0.0;
  for (int32_t base = rec0; base < rec1; base += kRecordLanes) {
    const int32_t here = rec1 - base < kRecordLanes ? rec1 - base : kRecordLanes;
    const int32_t id = plan.pos_records[base + (c < here ? c : 0)];
    const int32_t mine = static_cast<uint32_t>(id) < static_cast<uint32_t>(n_records) ? id : 0;
    T part[kRecordLanes];
#pragma unroll
    for (int k = 0; k < kRecordLanes; ++k) {
      const int32_t record = __shfl(mine, k < here ? k : 0, kRecordLanes);
      part[k] = src_rec[static_cast<int64_t>(record) * 12 + cc];
    }
#pragma unroll
    for (int k = 0; k < kRecordLanes; ++k) acc += k < here && c < 12 ? static_cast<double>(part[k]) : 0.0;
  }
  if (c < 3)
    force[static_cast<int64_t>(atom) * 3 + c] = static_cast<T>(acc);
  else if (c < 12)
    virial[static_cast<int64_t>(atom) * 9 + (c - 3)] = static_cast<T>(acc);
}

int check_plan_shapes(int64_t n_edges, int64_t n_nodes, const char* what) {
  if (n_edges < 0) return fail(DPA4K_EINVAL, "%s: negative edge count", what);
  if (n_nodes <= 0) return fail(DPA4K_EINVAL, "%s requires at least one atom", what);
  if (n_edges > int64_t(0x7fffffff) - 1) return fail(DPA4K_EINVAL, "%s: at least 2^31 - 1 edges", what);
  if (n_nodes > int64_t(0x7fffffff) - 1) return fail(DPA4K_EINVAL, "%s: at least 2^31 - 1 atoms", what);
  return DPA4K_OK;
}

BlobView view_of(const BlobPlan& p) {
  return BlobView{p.header, p.perm, p.piece_first, p.piece_t,  p.blob_piece, p.blob_rec, p.blob_entry,
                  p.row_edge, p.rec_entry,   p.pos_records, p.pos_rec, p.entry_row};
}

template <typename T>
int run_planned(const T* grad_edge, const T* edge_vec, T* force, T* virial, int64_t n_edges, int64_t n_nodes,
                const void* plan, size_t plan_bytes, void* records, size_t records_bytes, int64_t n_records,
                int64_t n_pieces, int32_t* status, dpa4k_stream_t stream_handle) {
  clear_error();
  if (int s = check_plan_shapes(n_edges, n_nodes, "planned force assembly")) return s;
  if (force == nullptr || virial == nullptr || plan == nullptr || records == nullptr ||
      (n_edges > 0 && (grad_edge == nullptr || edge_vec == nullptr)))
    return fail(DPA4K_EINVAL, "planned force assembly: null pointer");
  const size_t needed = blob_plan_bytes(n_edges, n_nodes, sizeof(T));
  if (plan_bytes < needed)
    return fail(DPA4K_EINVAL, "planned force assembly: plan of %zu bytes is smaller than %zu", plan_bytes, needed);
  if (n_records < 0 || n_records > n_edges || n_pieces < 0 || n_pieces > n_nodes + blob_count(n_edges, sizeof(T)))
    return fail(DPA4K_EINVAL, "planned force assembly: record or piece count out of range");
  const size_t records_needed = records_bytes_for(n_records, n_pieces, sizeof(T));
  if (records_bytes < records_needed)
    return fail(DPA4K_EINVAL, "planned force assembly: records buffer of %zu bytes is smaller than %zu",
                records_bytes, records_needed);
  BlobPlan arrays;
  if (!carve_blob_plan(const_cast<void*>(plan), plan_bytes, n_edges, n_nodes, sizeof(T), arrays))
    return fail(DPA4K_EINVAL, "planned force assembly: plan too small");
  hipStream_t stream = as_stream(stream_handle);
  if (n_edges == 0) {
    if (status != nullptr)
      if (int s = zero_fill(status, sizeof(int32_t), stream)) return s;
    if (int s = zero_fill(force, static_cast<size_t>(n_nodes) * 3 * sizeof(T), stream)) return s;
    return zero_fill(virial, static_cast<size_t>(n_nodes) * 9 * sizeof(T), stream);
  }
  Carver carver{static_cast<char*>(records), records_bytes};
  double* dst_rec = carver.take<double>(static_cast<size_t>(n_pieces > 0 ? n_pieces : 1) * 3);
  T* src_rec = carver.take<T>(static_cast<size_t>(n_records > 0 ? n_records : 1) * 12);
  const BlobView view = view_of(arrays);
  const int64_t blobs = blob_count(n_edges, sizeof(T));
  force_blob_kernel<T><<<launch_grid(blobs, kBlobThreads), kBlobThreads, 0, stream>>>(
      grad_edge, edge_vec, view, dst_rec, src_rec, n_edges, n_nodes, blobs, static_cast<int32_t>(n_records),
      static_cast<int32_t>(n_pieces));
  if (int s = launched("force_blob_kernel")) return s;
  const int64_t groups = (n_nodes + (256 / kRecordLanes) - 1) / (256 / kRecordLanes);
  force_records_kernel<T><<<launch_grid(groups, 256), 256, 0, stream>>>(
      view, dst_rec, src_rec, force, virial, n_edges, n_nodes, static_cast<int32_t>(n_records),
      static_cast<int32_t>(n_pieces), status);
  return launched("force_records_kernel");
}

int read_back(const int32_t* device, int32_t* host, size_t count, hipStream_t stream) {
  if (int s = hip_status(hipMemcpyAsync(host, device, count * 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync"))
    return s;
  return hip_status(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

template <typename T>
int build_plan(const int64_t* dst_offsets, const int64_t* src_offsets, const int64_t* src_order, const T* edge_vec,
               int64_t n_edges, int64_t n_nodes, const BlobPlan& plan, const BuildScratch& w, int64_t* counts_out,
               hipStream_t stream) {
  const int64_t rows = blob_rows_of<T>();
  const int64_t blobs = blob_count(n_edges, sizeof(T));
  const unsigned int node_blocks = stride_blocks(n_nodes + 1), edge_blocks = stride_blocks(n_edges);
  // the header names the graph only once the plan is complete
  if (int s = zero_fill(plan.header, kHeaderWords * sizeof(int64_t), stream)) return s;
  // validity of both CSRs, and the breadth-first root
  fill_i32_kernel<<<1, 256, 0, stream>>>(w.flags, kMaxLevels + 8, 0);
  if (int s = launched("fill_i32_kernel")) return s;
  plan_check_kernel<<<node_blocks, 256, 0, stream>>>(dst_offsets, src_offsets, n_edges, n_nodes, w.flags);
  if (int s = launched("plan_check_kernel")) return s;
  int32_t head[2];
  if (int s = read_back(w.flags, head, 2, stream)) return s;
  if (head[0] != 0) return fail(DPA4K_EINVAL, "force assembly plan: the offsets are not a CSR of n_edges slots");

  fill_i32_kernel<<<edge_blocks, 256, 0, stream>>>(w.edge_src, n_edges, -1);
  if (int s = launched("fill_i32_kernel")) return s;
  plan_slot_atoms_kernel<<<edge_blocks, 256, 0, stream>>>(src_offsets, src_order, w.slot_atom, w.edge_src, n_edges,
                                                          n_nodes);
  if (int s = launched("plan_slot_atoms_kernel")) return s;

  // positions along a breadth-first tree (edge_vec given), then Morton keys
  plan_bfs_init_kernel<<<node_blocks, 256, 0, stream>>>(w.level, w.pos, w.flags, n_nodes);
  if (int s = launched("plan_bfs_init_kernel")) return s;
  if (edge_vec != nullptr) {
    for (int depth = 0; depth < kMaxLevels; ++depth) {
      plan_bfs_level_kernel<T><<<node_blocks, 256, 0, stream>>>(dst_offsets, w.edge_src, edge_vec, w.level, w.pos,
                                                                w.flags, depth, n_nodes);
      if (int s = launched("plan_bfs_level_kernel")) return s;
      if (depth % 8 == 7) {
        int32_t progress;
        if (int s = read_back(w.flags + 8 + depth, &progress, 1, stream)) return s;
        if (progress == 0) break;
      }
    }
  }
  plan_box_kernel<<<kBoxBlocks, 256, 0, stream>>>(w.pos, w.level, n_nodes, w.box_part);
  if (int s = launched("plan_box_kernel")) return s;
  plan_box_final_kernel<<<1, 256, 0, stream>>>(w.box_part, kBoxBlocks, w.box);
  if (int s = launched("plan_box_final_kernel")) return s;
  const int bits = morton_bits(n_nodes);
  plan_morton_kernel<<<node_blocks, 256, 0, stream>>>(w.pos, w.level, w.box, n_nodes, bits, w.key);
  if (int s = launched("plan_morton_kernel")) return s;
  if (int s = dpa4k_group_by_key_async(w.key, n_nodes, (int64_t(1) << (3 * bits)) + 1, w.order, w.key_offsets,
                                       w.sort_status, w.sort, w.sort_bytes, stream))
    return s;
  plan_perm_kernel<<<node_blocks, 256, 0, stream>>>(w.order, dst_offsets, src_offsets, plan.perm, w.rank, w.counts,
                                                    w.src_counts, n_nodes);
  if (int s = launched("plan_perm_kernel")) return s;
  if (int s = scan_exclusive(w.counts, w.cum, n_nodes, w.scan_blocks, stream)) return s;
  if (int s = scan_exclusive(w.src_counts, w.cum_src, n_nodes, w.scan_blocks, stream)) return s;

  // pieces and rows
  plan_piece_counts_kernel<<<node_blocks, 256, 0, stream>>>(w.cum, w.counts, n_nodes, rows);
  if (int s = launched("plan_piece_counts_kernel")) return s;
  if (int s = scan_exclusive(w.counts, plan.piece_first, n_nodes, w.scan_blocks, stream)) return s;
  plan_pieces_kernel<<<node_blocks, 256, 0, stream>>>(w.cum, plan.piece_first, plan.piece_t, plan.blob_piece, n_nodes,
                                                      rows, n_edges, blobs);
  if (int s = launched("plan_pieces_kernel")) return s;
  plan_rows_kernel<<<edge_blocks, 256, 0, stream>>>(dst_offsets, w.rank, w.cum, w.tpos, plan.row_edge, n_edges,
                                                    n_nodes);
  if (int s = launched("plan_rows_kernel")) return s;

  // entries and records
  plan_source_slots_kernel<<<edge_blocks, 256, 0, stream>>>(w.cum_src, plan.perm, src_offsets, w.pslot, n_edges,
                                                            n_nodes);
  if (int s = launched("plan_source_slots_kernel")) return s;
  plan_slot_keys_kernel<<<edge_blocks, 256, 0, stream>>>(src_order, w.pslot, w.tpos, w.key, n_edges, rows, blobs);
  if (int s = launched("plan_slot_keys_kernel")) return s;
  if (int s = dpa4k_group_by_key_async(w.key, n_edges, blobs + 1, w.order, w.key_offsets, w.sort_status, w.sort,
                                       w.sort_bytes, stream))
    return s;
  plan_entries_kernel<<<edge_blocks, 256, 0, stream>>>(w.order, w.key, w.pslot, src_order, w.slot_atom, w.tpos,
                                                       w.entry_old, w.counts, n_edges, rows, blobs);
  if (int s = launched("plan_entries_kernel")) return s;
  if (int s = scan_exclusive(w.counts, w.scanned, n_edges, w.scan_blocks, stream)) return s;
  plan_records_kernel<<<edge_blocks, 256, 0, stream>>>(w.counts, w.scanned, w.key_offsets, w.rec_old,
                                                       plan.blob_rec, plan.blob_entry, n_edges, blobs);
  if (int s = launched("plan_records_kernel")) return s;
  int32_t records, pieces;
  if (int s = read_back(w.scanned + n_edges, &records, 1, stream)) return s;
  if (int s = read_back(plan.piece_first + n_nodes, &pieces, 1, stream)) return s;

  // each blob's records by descending length (stable), their entries moved to match
  const unsigned int record_blocks = stride_blocks(records);
  plan_length_keys_kernel<<<record_blocks, 256, 0, stream>>>(w.rec_old, w.order, w.key, w.pslot, w.slot_atom, w.key2,
                                                             w.lengths, w.tpos, records);
  if (int s = launched("plan_length_keys_kernel")) return s;
  if (int s = dpa4k_group_by_key_async(w.key2, records, blobs * kLengthKeys, w.order, w.key_offsets, w.sort_status,
                                       w.sort, w.sort_bytes, stream))
    return s;
  plan_gather_i32_kernel<<<record_blocks, 256, 0, stream>>>(w.order, w.lengths, w.counts, records);
  if (int s = launched("plan_gather_i32_kernel")) return s;
  if (int s = scan_exclusive(w.counts, w.scanned, records, w.scan_blocks, stream)) return s;
  plan_move_entries_kernel<<<record_blocks, 256, 0, stream>>>(w.order, w.rec_old, w.entry_old, w.scanned, w.tpos,
                                                              w.rank, plan.entry_row, plan.rec_entry, w.key, records);
  if (int s = launched("plan_move_entries_kernel")) return s;

  // record ids grouped by position (stable: blob order within a position)
  if (int s = dpa4k_group_by_key_async(w.key, records, n_nodes, w.order, w.key_offsets, w.sort_status, w.sort,
                                       w.sort_bytes, stream))
    return s;
  plan_record_slots_kernel<<<stride_blocks(records > n_nodes + 1 ? records : n_nodes + 1), 256, 0, stream>>>(
      w.order, w.key_offsets, plan.pos_records, plan.pos_rec, records, n_nodes);
  if (int s = launched("plan_record_slots_kernel")) return s;
  const int64_t header[kHeaderWords] = {kPlanMagic, n_edges, n_nodes, static_cast<int64_t>(sizeof(T)), records,
                                        pieces};
  if (int s = hip_status(hipMemcpyAsync(plan.header, header, sizeof(header), hipMemcpyHostToDevice, stream),
                         "hipMemcpyAsync"))
    return s;
  counts_out[0] = records;
  counts_out[1] = pieces;
  return hip_status(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

#undef DPA4K_GRID_STRIDE

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
  if (n_edges < 0 || n_nodes <= 0 || (value_bytes != 4 && value_bytes != 8)) return 0;
  return dpa4k::blob_plan_bytes(n_edges, n_nodes, value_bytes);
}

extern "C" size_t dpa4k_force_assembly_plan_workspace_size(int64_t n_edges, int64_t n_nodes) {
  if (n_edges < 0 || n_nodes <= 0) return 0;
  return dpa4k::build_workspace_bytes(n_edges, n_nodes);
}

extern "C" size_t dpa4k_force_assembly_records_size(int64_t n_records, int64_t n_pieces, int64_t value_bytes) {
  if (n_records < 0 || n_pieces < 0 || (value_bytes != 4 && value_bytes != 8)) return 0;
  return dpa4k::records_bytes_for(n_records, n_pieces, value_bytes);
}

extern "C" int dpa4k_force_assembly_plan(const int64_t* dst_offsets, const int64_t* src_offsets,
                                         const int64_t* src_order, const void* edge_vec, int64_t n_edges,
                                         int64_t n_nodes, int64_t value_bytes, void* plan, size_t plan_bytes,
                                         void* workspace, size_t workspace_bytes, int64_t* counts,
                                         dpa4k_stream_t stream_handle) {
  using namespace dpa4k;
  clear_error();
  if (int s = check_plan_shapes(n_edges, n_nodes, "force assembly plan")) return s;
  if (value_bytes != 4 && value_bytes != 8) return fail(DPA4K_EINVAL, "force assembly plan: values of 4 or 8 bytes");
  if (dst_offsets == nullptr || src_offsets == nullptr || plan == nullptr || counts == nullptr ||
      (n_edges > 0 && src_order == nullptr))
    return fail(DPA4K_EINVAL, "force assembly plan: null pointer");
  const size_t needed = blob_plan_bytes(n_edges, n_nodes, value_bytes);
  if (plan_bytes < needed)
    return fail(DPA4K_EINVAL, "force assembly plan: buffer of %zu bytes is smaller than %zu", plan_bytes, needed);
  const size_t scratch_needed = build_workspace_bytes(n_edges, n_nodes);
  if (workspace == nullptr || workspace_bytes < scratch_needed)
    return fail(DPA4K_EWORKSPACE, "force assembly plan: workspace of %zu bytes is smaller than %zu", workspace_bytes,
                scratch_needed);
  counts[0] = counts[1] = 0;
  if (n_edges == 0) return DPA4K_OK;
  BlobPlan arrays;
  BuildScratch scratch;
  if (!carve_blob_plan(plan, plan_bytes, n_edges, n_nodes, value_bytes, arrays) ||
      !carve_build(workspace, workspace_bytes, n_edges, n_nodes, scratch))
    return fail(DPA4K_EINVAL, "force assembly plan: buffers too small");
  hipStream_t stream = as_stream(stream_handle);
  if (value_bytes == 4)
    return build_plan<float>(dst_offsets, src_offsets, src_order, static_cast<const float*>(edge_vec), n_edges,
                             n_nodes, arrays, scratch, counts, stream);
  return build_plan<double>(dst_offsets, src_offsets, src_order, static_cast<const double*>(edge_vec), n_edges,
                            n_nodes, arrays, scratch, counts, stream);
}

extern "C" int dpa4k_force_assembly_f32_planned(const float* grad_edge, const float* edge_vec, float* force,
                                                float* virial, int64_t n_edges, int64_t n_nodes, const void* plan,
                                                size_t plan_bytes, void* records, size_t records_bytes,
                                                int64_t n_records, int64_t n_pieces, int32_t* status,
                                                dpa4k_stream_t stream) {
  return dpa4k::run_planned<float>(grad_edge, edge_vec, force, virial, n_edges, n_nodes, plan, plan_bytes, records,
                                   records_bytes, n_records, n_pieces, status, stream);
}

extern "C" int dpa4k_force_assembly_f64_planned(const double* grad_edge, const double* edge_vec, double* force,
                                                double* virial, int64_t n_edges, int64_t n_nodes, const void* plan,
                                                size_t plan_bytes, void* records, size_t records_bytes,
                                                int64_t n_records, int64_t n_pieces, int32_t* status,
                                                dpa4k_stream_t stream) {
  return dpa4k::run_planned<double>(grad_edge, edge_vec, force, virial, n_edges, n_nodes, plan, plan_bytes, records,
                                    records_bytes, n_records, n_pieces, status, stream);
}

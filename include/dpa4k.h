/*
 * dpa4k.h -- C ABI of the MI355X (gfx950) DPA4/SeZM operator library
 * (libdpa4k.so, built from bysj_amd/csrc/).
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - Plain pointers and sizes only.  Every pointer is a device pointer into
 *    HBM of the current HIP device, except where a parameter says "host".
 *  - Tensors are dense, row-major and contiguous; shapes are given in the
 *    comment of each function ([E, C] means E rows of C elements).
 *  - Index tensors (offsets, orders, dst, src, radial_slot) are int64.
 *  - `stream` is a hipStream_t passed as void*; NULL is the null stream.  All
 *    work is enqueued on it.  Only the functions marked "synchronises" wait
 *    for the stream; every other function returns as soon as its kernels are
 *    enqueued.
 *  - The library never allocates device memory.  Functions that need scratch
 *    memory take a caller-provided workspace and have a *_workspace_size
 *    query.
 *  - Return value: DPA4K_OK (0) on success, otherwise an error code; the
 *    message of the last error raised on the calling thread is returned by
 *    dpa4k_last_error().  No C++ exception crosses this boundary.
 *  - CSR contract (segment operators): `offsets[N+1]` is the exclusive prefix
 *    sum of the per-segment edge counts (offsets[0] == 0, offsets[N] == E,
 *    non-decreasing).  Segment n owns the slots [offsets[n], offsets[n+1]);
 *    slot s addresses edge `order[s]` when `order` is given and edge `s`
 *    otherwise.  Outputs indexed by edge are written in the natural edge
 *    order.  Offsets are clamped to [0, E] and order entries outside [0, E)
 *    are skipped on the device, so a malformed CSR yields wrong values but
 *    never an out-of-bounds access.
 *  - Every reduction runs in a fixed order that depends only on the shapes
 *    and the CSR, never on timing: results are bitwise reproducible from
 *    run to run.  No floating-point atomics are used anywhere.
 *
 * Each declaration names the reference interface it replaces
 * (lipengfei1409/bysj, file:line).
 */
#ifndef DPA4K_H
#define DPA4K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dpa4k_stream_t;

enum {
  DPA4K_OK = 0,
  DPA4K_EINVAL = 1,    /* bad argument (shape, size, pointer, index range) */
  DPA4K_EHIP = 2,      /* a HIP runtime call or kernel launch failed        */
  DPA4K_EWORKSPACE = 3 /* workspace missing or smaller than required        */
};

/* Message of the last error on this thread ("" if none).  No reference
 * counterpart: replaces TORCH_CHECK's exception text (csrc/checks.h:6-20). */
const char* dpa4k_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int dpa4k_abi_version(void);
#define DPA4K_ABI_VERSION 10

/* ------------------------------------------------------------------------
 * CSR construction
 * ---------------------------------------------------------------------- */

/* Replaces kernels.segment.segment_offsets (python/kernels/segment.py:46-57).
 * offsets[N+1] = [0, cumsum(bincount(keys, minlength=N))].  Bit-exact.
 * Synchronises once, at the end: returns DPA4K_EINVAL ("... values must be
 * within the node range") when a key lies outside [0, N), matching the
 * reference's dst.min()/dst.max() check (:54).  1 <= N <= 2^32,
 * 0 <= E < 2^32.  workspace >= dpa4k_segment_offsets_workspace_size(E, N)
 * bytes.  Keys that are already non-decreasing are not sorted; others are
 * grouped by a stable counting sort on the device. */
size_t dpa4k_segment_offsets_workspace_size(int64_t n_edges, int64_t n_nodes);
int dpa4k_segment_offsets(const int64_t* keys, int64_t n_edges, int64_t n_nodes,
                          int64_t* offsets, void* workspace,
                          size_t workspace_bytes, dpa4k_stream_t stream);

/* Replaces kernels.segment.group_by_source (python/kernels/segment.py:60-71):
 * order[E] = stable argsort(keys), offsets[N+1] as above.  Bit-exact (a
 * stable order is unique).  Synchronises once (same range check as above). */
size_t dpa4k_group_by_key_workspace_size(int64_t n_edges, int64_t n_nodes);
int dpa4k_group_by_key(const int64_t* keys, int64_t n_edges, int64_t n_nodes,
                       int64_t* order, int64_t* offsets, void* workspace,
                       size_t workspace_bytes, dpa4k_stream_t stream);

/* Asynchronous forms of the two builders above (no reference counterpart:
 * the reference's check synchronises).  They enqueue the whole build on
 * `stream` and return without waiting, so a caller may capture them in a HIP
 * graph.  `status` (device int32, cleared by the call) receives the bits
 *   DPA4K_CSR_OUT_OF_RANGE  a key lies outside [0, N): offsets and order are
 *                           then unspecified (nothing outside them is written);
 *   DPA4K_CSR_UNSORTED      the keys were not already non-decreasing.
 * The caller must read it before trusting the result.  Same workspace. */
#define DPA4K_CSR_OUT_OF_RANGE 1
#define DPA4K_CSR_UNSORTED 2
int dpa4k_segment_offsets_async(const int64_t* keys, int64_t n_edges,
                                int64_t n_nodes, int64_t* offsets,
                                int32_t* status, void* workspace,
                                size_t workspace_bytes, dpa4k_stream_t stream);
int dpa4k_group_by_key_async(const int64_t* keys, int64_t n_edges,
                             int64_t n_nodes, int64_t* order, int64_t* offsets,
                             int32_t* status, void* workspace,
                             size_t workspace_bytes, dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * segment_sum
 * ---------------------------------------------------------------------- */

/* Replaces segment_sum_forward_hip (csrc/segment_sum.cpp:214).
 * out[n, c] = node_scale[n] * sum_{slots of n} edge_scale[e] * src[e, c]
 * src[E, C], edge_scale[E] or NULL, node_scale[N] or NULL, order[E] or NULL,
 * out[N, C].  C >= 1.  Each output element is accumulated sequentially in
 * slot order (product rounded, then added), so the result equals the
 * sequential fp32 chain `zeros -> index_add_ -> mul` bit for bit. */
int dpa4k_segment_sum_forward(const float* src, const int64_t* offsets,
                              const float* edge_scale, const float* node_scale,
                              const int64_t* order, float* out,
                              int64_t n_edges, int64_t n_nodes, int64_t channels,
                              dpa4k_stream_t stream);

/* Replaces segment_sum_backward_hip (csrc/segment_sum.cpp:271), adding the
 * edge_scale gradient the reference leaves out (python/kernels/segment.py:221-230):
 *   grad_src[e, c]      = (grad_out[n, c] * node_scale[n]) * edge_scale[e]
 *   grad_edge_scale[e]  = sum_c (grad_out[n, c] * node_scale[n]) * src[e, c]
 *   grad_node_scale[n]  = sum_c grad_out[n, c] * (sum_{slots} edge_scale * src)[n, c]
 * with n the segment owning edge e.  grad_edge_scale / grad_node_scale may be
 * NULL (not computed); grad_src must cover [E, C].  The reference's `dst`
 * argument is not needed: the CSR (offsets, order) identifies each edge's
 * segment, which the grouping contract makes equal to dst[e]. */
int dpa4k_segment_sum_backward(const float* grad_out, const float* src,
                               const int64_t* offsets, const float* edge_scale,
                               const float* node_scale, const int64_t* order,
                               float* grad_src, float* grad_edge_scale,
                               float* grad_node_scale, int64_t n_edges,
                               int64_t n_nodes, int64_t channels,
                               dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * segment_softmax
 * ---------------------------------------------------------------------- */

/* Replaces segment_softmax_forward_hip (csrc/segment_softmax.cpp:235).
 * Per segment and channel: l_e = logit[e, c] + 2 ln(max(env[e], 1e-30)) for
 * env[e] > 0 (other edges carry no mass), m = max(null_logit[n, c], max_e l_e),
 * w_e = exp(l_e - m), D = exp(null - m) + sum_e w_e, alpha = w_e / D,
 * null_alpha = exp(null - m) / D; a segment with no mass gives zeros.
 * Evaluated in base 2 with the hardware exp2/log2/reciprocal (relative error
 * below 1e-6 against the natural-base chain).
 * logit[E, C], env[E], null_logit[N, C] or NULL, order[E] or NULL,
 * alpha[E, C], null_alpha[N, C] (required iff null_logit is given). */
int dpa4k_segment_softmax_forward(const float* logit, const float* env,
                                  const int64_t* offsets, const float* null_logit,
                                  const int64_t* order, float* alpha,
                                  float* null_alpha, int64_t n_edges,
                                  int64_t n_nodes, int64_t channels,
                                  dpa4k_stream_t stream);

/* Replaces segment_softmax_backward_hip (csrc/segment_softmax.cpp:279).
 *   S = sum_e alpha * grad_alpha + null_alpha * grad_null_alpha
 *   grad_logit = alpha (grad_alpha - S); grad_null_logit = null_alpha (grad_null_alpha - S)
 *   grad_env[e] = (sum_c grad_logit[e, c]) * 2 / env[e]  (0 where !(env > 0))
 * null_alpha, grad_null_alpha and grad_null_logit are all given or all NULL. */
int dpa4k_segment_softmax_backward(const float* alpha, const float* grad_alpha,
                                   const float* env, const int64_t* offsets,
                                   const float* null_alpha,
                                   const float* grad_null_alpha,
                                   const int64_t* order, float* grad_logit,
                                   float* grad_null_logit, float* grad_env,
                                   int64_t n_edges, int64_t n_nodes,
                                   int64_t channels, dpa4k_stream_t stream);

/* Degree plan of a CSR for the segment softmax (no reference counterpart: it
 * is the degree-binned schedule of the gfx950 kernels).  Lists, in ascending
 * order, the segments longer than the register capacity of the kernel that
 * runs `channels` channels; the planned entry points below give each of them
 * a workgroup of its own ahead of the short segments.  Build it once per
 * graph and reuse it for every forward and backward on the same offsets and
 * channel count.  plan >= dpa4k_segment_softmax_plan_size(N) bytes of device
 * memory (8-byte aligned); *n_long and *plan_capacity (host) receive the
 * number of listed segments and the degree threshold the list was built for.
 * Synchronises (to read them back). */
size_t dpa4k_segment_softmax_plan_size(int64_t n_nodes);
int dpa4k_segment_softmax_plan(const int64_t* offsets, int64_t n_edges,
                               int64_t n_nodes, int64_t channels, void* plan,
                               size_t plan_bytes, int64_t* n_long,
                               int64_t* plan_capacity, dpa4k_stream_t stream);

/* dpa4k_segment_softmax_forward / _backward with a plan from
 * dpa4k_segment_softmax_plan on the same offsets, and the n_long and
 * plan_capacity it returned (0 <= n_long <= N).  Same results as the
 * unplanned calls, bit for bit.  When plan_capacity does not match the
 * kernel chosen for these channels and pointer alignments, the plan is
 * ignored and the call runs unplanned. */
int dpa4k_segment_softmax_forward_planned(
    const float* logit, const float* env, const int64_t* offsets,
    const float* null_logit, const int64_t* order, float* alpha,
    float* null_alpha, int64_t n_edges, int64_t n_nodes, int64_t channels,
    const void* plan, int64_t n_long, int64_t plan_capacity,
    dpa4k_stream_t stream);
int dpa4k_segment_softmax_backward_planned(
    const float* alpha, const float* grad_alpha, const float* env,
    const int64_t* offsets, const float* null_alpha,
    const float* grad_null_alpha, const int64_t* order, float* grad_logit,
    float* grad_null_logit, float* grad_env, int64_t n_edges, int64_t n_nodes,
    int64_t channels, const void* plan, int64_t n_long, int64_t plan_capacity,
    dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * force_assembly
 * ---------------------------------------------------------------------- */

/* Replaces force_assembly_hip (csrc/force_assembly.cpp:106).
 *   force[k]         = sum_{dst slots of k} g_e - sum_{src slots of k} g_e
 *   virial[k, 3r+c]  = - sum_{src slots of k} g_e[r] * v_e[c]
 * grad_edge[E, 3], edge_vec[E, 3], dst_offsets[N+1] addressing the natural
 * (dst-grouped) edge order, src_offsets[N+1] + src_order[E] grouping the
 * edges by source; force[N, 3], virial[N, 9].  N >= 1.  Accumulates in
 * double in a fixed order; the f32 variant rounds once on output. */
int dpa4k_force_assembly_f32(const float* grad_edge, const float* edge_vec,
                             const int64_t* dst_offsets,
                             const int64_t* src_offsets,
                             const int64_t* src_order, float* force,
                             float* virial, int64_t n_edges, int64_t n_nodes,
                             dpa4k_stream_t stream);

/* fp64 extension of the above (the reference is fp32-only,
 * csrc/force_assembly.cpp:110-111): double inputs, double outputs. */
int dpa4k_force_assembly_f64(const double* grad_edge, const double* edge_vec,
                             const int64_t* dst_offsets,
                             const int64_t* src_offsets,
                             const int64_t* src_order, double* force,
                             double* virial, int64_t n_edges, int64_t n_nodes,
                             dpa4k_stream_t stream);

/* Planned force assembly (no reference counterpart; same sums as the two
 * entry points above, in another fixed order: equal to them within rounding,
 * and reproducible run to run).  A plan of one graph (both CSRs and
 * src_order) is built once:
 *   - atom positions are recovered from `edge_vec` (a hint: r_dst = r_src -
 *     v_e along a breadth-first tree; NULL keeps the natural atom order) and
 *     the atoms are sorted by their Morton cell;
 *   - the destination segments, concatenated in that order, are cut into
 *     blobs of 2816 (float32) or 1408 (float64) rows; a segment crossing a
 *     blob boundary becomes one piece per blob;
 *   - within a blob, the edges of one source atom form a record.
 * A planned call stages each blob's rows (g_e, v_e) in LDS, writes one
 * destination sum per piece and twelve source sums per record, then adds
 * each atom's pieces and records in blob order.  The build synchronises
 * `stream` (it reads the record and piece counts back, returned in
 * counts[0] and counts[1]) and fails with DPA4K_EINVAL unless both offsets
 * arrays are CSRs of n_edges slots.  Slots of src_order out of [0, E) are
 * skipped, as in the direct kernels.  A plan starts with a header naming
 * the edge count, atom count, value size and the record and piece counts
 * it was built with.  A planned call checks it on the device: for a plan
 * whose header differs from the call (another graph's size, dtype or
 * counts, or a build that did not finish), it reads nothing else of the
 * plan, writes NaN into every element of force and virial and sets
 * `*status` (a device int32, may be NULL) to DPA4K_FORCE_PLAN_MISMATCH;
 * otherwise it sets `*status` to 0.  The call itself returns DPA4K_OK in
 * both cases (it never synchronises): read `status` before trusting the
 * outputs.  A plan of another graph with identical sizes and counts gives
 * wrong sums, never an access out of bounds; the plan's own indices are
 * bounded by the given counts.  The calls write the caller's records
 * buffer (dpa4k_force_assembly_records_size bytes): calls sharing one must
 * not overlap.  value_bytes = 4 (float32) or 8 (float64); a plan serves the
 * dtype it was built for.  E < 2^31 - 1, N >= 1.  The plan needs
 * dpa4k_force_assembly_plan_size bytes (about 14 * E) and its build a
 * workspace of dpa4k_force_assembly_plan_workspace_size bytes. */
size_t dpa4k_force_assembly_plan_size(int64_t n_edges, int64_t n_nodes,
                                      int64_t value_bytes);
size_t dpa4k_force_assembly_plan_workspace_size(int64_t n_edges,
                                                int64_t n_nodes);
size_t dpa4k_force_assembly_records_size(int64_t n_records, int64_t n_pieces,
                                         int64_t value_bytes);
int dpa4k_force_assembly_plan(const int64_t* dst_offsets,
                              const int64_t* src_offsets,
                              const int64_t* src_order, const void* edge_vec,
                              int64_t n_edges, int64_t n_nodes,
                              int64_t value_bytes, void* plan,
                              size_t plan_bytes, void* workspace,
                              size_t workspace_bytes, int64_t* counts,
                              dpa4k_stream_t stream);
int dpa4k_force_assembly_f32_planned(const float* grad_edge,
                                     const float* edge_vec, float* force,
                                     float* virial, int64_t n_edges,
                                     int64_t n_nodes, const void* plan,
                                     size_t plan_bytes, void* records,
                                     size_t records_bytes, int64_t n_records,
                                     int64_t n_pieces, int32_t* status,
                                     dpa4k_stream_t stream);
int dpa4k_force_assembly_f64_planned(const double* grad_edge,
                                     const double* edge_vec, double* force,
                                     double* virial, int64_t n_edges,
                                     int64_t n_nodes, const void* plan,
                                     size_t plan_bytes, void* records,
                                     size_t records_bytes, int64_t n_records,
                                     int64_t n_pieces, int32_t* status,
                                     dpa4k_stream_t stream);
#define DPA4K_FORCE_PLAN_MISMATCH 4

/* ------------------------------------------------------------------------
 * Edge-stream elementwise chain
 * ---------------------------------------------------------------------- */

/* No reference implementation: the reference designs this fusion as its
 * candidate C4 (docs/task2-hip-fusion-plan.md:280-300, "designed, not
 * implemented"), to replace chains of add_/mul/copy_ passes over [E, R, C]
 * edge tensors in DeepMD's SeZM blocks.  One pass computes
 *   acc[e, r, c] = sum_{k < n_terms, left to right} (a_k * b_k) * coef_k
 *   out[e, r, c] = act(acc[e, r, c])
 * over E edges, R rows and C channels; out is a contiguous [E, R, C] fp32
 * array.  Each operand is an fp32 view: element (e, r, c) sits at
 * data + e * stride[0] + r * stride[1] + c * stride[2], strides >= 0, and a
 * zero stride broadcasts it along that axis (a per-edge scalar, a per-row
 * gate, a per-channel weight).  The caller guarantees that every element the
 * strides address lies in the operand's allocation.  b may be NULL, or b[k]
 * have data NULL: factor 1.  Every product is rounded before the next
 * operation, so with DPA4K_ACT_NONE the result equals the eager fp32 chain
 * t = a * b; t = t * coef; acc = t_0 + t_1 + ... bit for bit.  Activations:
 *   DPA4K_ACT_SILU  x * sigmoid(x);
 *   DPA4K_ACT_GATE  SeZM's gated activation: gate_row (host array of R
 *                   ints, R <= DPA4K_EDGE_STREAM_MAX_GATE_ROWS) maps each row
 *                   to a gate index; rows with gate_row[r] < 0 take silu, the
 *                   others x * sigmoid(gate[e, gate_row[r], c]), gate being
 *                   an operand view over (edge, gate index, channel).
 * out may be the same array as a contiguous [E, R, C] operand (in-place
 * accumulation); it must not overlap any other operand.  1 <= n_terms <=
 * DPA4K_EDGE_STREAM_MAX_TERMS.  Enqueued on `stream`, no allocation. */
#define DPA4K_EDGE_STREAM_MAX_TERMS 4
#define DPA4K_EDGE_STREAM_MAX_GATE_ROWS 64
enum { DPA4K_ACT_NONE = 0, DPA4K_ACT_SILU = 1, DPA4K_ACT_GATE = 2 };
typedef struct dpa4k_edge_operand {
  const float* data;
  int64_t stride[3]; /* element strides over (edge, row, channel) */
} dpa4k_edge_operand;
int dpa4k_edge_stream_combine(const dpa4k_edge_operand* a,
                              const dpa4k_edge_operand* b, const float* coef,
                              int n_terms, int activation,
                              const dpa4k_edge_operand* gate,
                              const int32_t* gate_row, float* out,
                              int64_t n_edges, int64_t n_rows,
                              int64_t channels, dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * GIE zonal scatter
 * ---------------------------------------------------------------------- */

/* Grouping step of the GIE operator (no reference counterpart: the
 * reference scatters with atomics on the unsorted dst, csrc/gie.cpp:68-87).
 * Builds the destination CSR of an unsorted dst: offsets[N+1] and order[E]
 * (the identity when dst is already non-decreasing).  Also checks
 * 0 <= dst < N and 0 <= radial_slot < S.  Synchronises.
 * host_info (host pointer, may be NULL) receives a bit set:
 *   1 = dst was non-decreasing (the kernels may then take a NULL order),
 *   2 = every radial slot is referenced by at most one row,
 *   bits 16..23 = the most rows that reference one slot (capped at 255).
 * The GIE kernels below take this word as `slot_info` to pick their layout;
 * 0 means "unknown" and selects kernels that assume nothing about the map.
 * Out-of-range indices return DPA4K_EINVAL. */
size_t dpa4k_gie_group_workspace_size(int64_t n_edges, int64_t n_nodes);
int dpa4k_gie_group(const int64_t* dst, const int64_t* radial_slot,
                    int64_t n_edges, int64_t n_nodes, int64_t n_rows,
                    int64_t n_radial, int64_t* offsets, int64_t* order,
                    int32_t* host_info, void* workspace, size_t workspace_bytes,
                    dpa4k_stream_t stream);

/* Replaces gie_zonal_scatter_forward_hip (csrc/gie.cpp:148), given the CSR
 * from dpa4k_gie_group:
 *   out[n, 0, :]   = 0 * inv[n]
 *   out[n, r+1, c] = inv[n] * sum_{slots of n} zonal[e, r] * radial[e, slot[r], c]
 * (normalise after the sum).  zonal[E, R], radial[E, S, C], radial_slot[R],
 * inv_sqrt_deg[N], out[N, R+1, C].  Sequential per-element accumulation:
 * equals the fp32 chain `gather -> mul -> index_add_ -> mul` bit for bit.
 * slot_info: dpa4k_gie_group's host_info for this radial_slot, or 0.  With
 * shared slots and at most 8 rows per slot it selects a kernel that reads
 * each radial element once per edge (same output); it must then describe
 * radial_slot truthfully. */
int dpa4k_gie_zonal_scatter_forward_csr(const float* zonal, const float* radial,
                                        const int64_t* offsets,
                                        const int64_t* order,
                                        const int64_t* radial_slot,
                                        const float* inv_sqrt_deg, float* out,
                                        int64_t n_edges, int64_t n_nodes,
                                        int64_t n_rows, int64_t n_radial,
                                        int64_t channels, int32_t slot_info,
                                        dpa4k_stream_t stream);

/* Replaces gie_zonal_scatter_backward_hip (csrc/gie.cpp:178), given the CSR:
 *   grad_zonal[e, r]     = sum_c inv[n] grad[n, r+1, c] radial[e, slot[r], c]
 *   grad_radial[e, s, c] = sum_{r: slot[r]=s} inv[n] grad[n, r+1, c] zonal[e, r]
 *   grad_inv[n]          = sum_{r, c} grad[n, r+1, c] pre[n, r+1, c]
 * with pre the unnormalised destination sum (recomputed, not saved).  Any
 * of the three outputs may be NULL.  grad_radial is written in full (zeros
 * for unreferenced slots).  slot_info: dpa4k_gie_group's host_info for this
 * radial_slot, or 0; bit 2 (distinct slots) or bits 16..23 in [2, 8]
 * (shared slots, C = 8 * k with k a power of two, k <= 16 and S * k <= 64)
 * select register-only kernels, anything else the general one.  It must
 * describe radial_slot truthfully. */
int dpa4k_gie_zonal_scatter_backward_csr(
    const float* grad_output, const float* zonal, const float* radial,
    const int64_t* offsets, const int64_t* order, const int64_t* radial_slot,
    const float* inv_sqrt_deg, float* grad_zonal, float* grad_radial,
    float* grad_inv_sqrt_deg, int64_t n_edges, int64_t n_nodes, int64_t n_rows,
    int64_t n_radial, int64_t channels, int32_t slot_info,
    dpa4k_stream_t stream);

/* One-call forms with the reference's signature (csrc/gie.cpp:148,178):
 * group + forward/backward.  Synchronise (grouping step). */
int dpa4k_gie_zonal_scatter_forward(const float* zonal, const float* radial,
                                    const int64_t* dst,
                                    const int64_t* radial_slot,
                                    const float* inv_sqrt_deg, float* out,
                                    int64_t n_edges, int64_t n_nodes,
                                    int64_t n_rows, int64_t n_radial,
                                    int64_t channels, void* workspace,
                                    size_t workspace_bytes,
                                    dpa4k_stream_t stream);
int dpa4k_gie_zonal_scatter_backward(
    const float* grad_output, const float* zonal, const float* radial,
    const int64_t* dst, const int64_t* radial_slot, const float* inv_sqrt_deg,
    float* grad_zonal, float* grad_radial, float* grad_inv_sqrt_deg,
    int64_t n_edges, int64_t n_nodes, int64_t n_rows, int64_t n_radial,
    int64_t channels, void* workspace, size_t workspace_bytes,
    dpa4k_stream_t stream);
/* Workspace of the one-call forms (CSR arrays + grouping scratch). */
size_t dpa4k_gie_workspace_size(int64_t n_edges, int64_t n_nodes);

/* Fused GIE zonal scatter -> RMSNorm (no reference counterpart: the
 * reference runs gie_zonal_scatter_forward_hip, csrc/gie.cpp:148, and then
 * rmsnorm_forward_hip, csrc/rmsnorm.cpp:99).  For each node, x = the GIE
 * output row [R + 1, C] (as dpa4k_gie_zonal_scatter_forward_csr), flattened
 * to W = (R + 1) * C floats, and y = x * (1 / sqrt(mean(x^2) + eps)) *
 * scale (as dpa4k_rmsnorm_forward); y[N, W], inverse_rms[N], and x[N, W]
 * when x_out is not NULL (the backward needs it).  Bit-identical to the two
 * entry points run back to back.  scale may be NULL.  Needs channels % 4 ==
 * 0, W <= 2048 + C (dpa4k_gie_rmsnorm_supported) and 16-byte aligned
 * radial, scale, y and x_out. */
int dpa4k_gie_rmsnorm_supported(int64_t n_rows, int64_t channels);
int dpa4k_gie_rmsnorm_forward_csr(const float* zonal, const float* radial,
                                  const int64_t* offsets, const int64_t* order,
                                  const int64_t* radial_slot,
                                  const float* inv_sqrt_deg, const float* scale,
                                  float eps, float* y, float* x_out,
                                  float* inverse_rms, int64_t n_edges,
                                  int64_t n_nodes, int64_t n_rows,
                                  int64_t n_radial, int64_t channels,
                                  dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * RMSNorm
 * ---------------------------------------------------------------------- */

/* Replaces rmsnorm_forward_hip (csrc/rmsnorm.cpp:99).
 * y = x * (1 / sqrt(mean(x^2) + eps)) * scale over rows of width W.
 * x[rows, W], scale[W] or NULL, y[rows, W], inverse_rms[rows].  W >= 1,
 * eps finite and > 0. */
int dpa4k_rmsnorm_forward(const float* x, const float* scale, float* y,
                          float* inverse_rms, int64_t rows, int64_t width,
                          float eps, dpa4k_stream_t stream);

/* Replaces rmsnorm_backward_hip (csrc/rmsnorm.cpp:123).
 *   u = grad * scale;  grad_x = inv u - x inv^3 mean(x u)
 *   grad_scale[w] = sum_rows grad * x * inv      (if grad_scale != NULL)
 * grad_scale is reduced over rows in a fixed two-stage order (no atomics);
 * it needs workspace >= dpa4k_rmsnorm_backward_workspace_size(rows, W). */
size_t dpa4k_rmsnorm_backward_workspace_size(int64_t rows, int64_t width);
int dpa4k_rmsnorm_backward(const float* grad, const float* x,
                           const float* scale, const float* inverse_rms,
                           float* grad_x, float* grad_scale, int64_t rows,
                           int64_t width, void* workspace,
                           size_t workspace_bytes, dpa4k_stream_t stream);

/* dpa4k_rmsnorm_backward without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * It calls no hipMalloc/hipFree: the column partials of grad_scale live in a
 * library-owned static device array of DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES
 * (768 rows of at most 4096 floats, 12 MiB), one per device, held until the
 * process ends; its address is looked up once per device on the first call.
 * Same kernels as dpa4k_rmsnorm_backward, so the results are the same bit
 * for bit.  Every row of partials a call uses is written before it is read:
 * nothing needs clearing between calls.  Calls that overlap on one device
 * (concurrent streams or threads) race on the array and must be serialised
 * by the caller.  Returns DPA4K_EINVAL if a shape would need more partials
 * than the array holds (no shape the kernels accept does). */
#define DPA4K_RMSNORM_NOALLOC_SCRATCH_BYTES 12582912
int dpa4k_rmsnorm_backward_noalloc(const float* grad, const float* x,
                                   const float* scale, const float* inverse_rms,
                                   float* grad_x, float* grad_scale,
                                   int64_t rows, int64_t width,
                                   dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * Stream calibration (measurement aid; no reference counterpart)
 * ---------------------------------------------------------------------- */

/* Streams read_floats floats of src and writes the first write_floats of
 * them to dst (write_floats == 0: read only; dst then receives at most one
 * word per workgroup and needs 8192 floats).  Counts are multiples of 4,
 * write_floats <= read_floats, buffers 16-byte aligned.  bench.py times it
 * to report the read and copy ceilings of the part beside each roofline. */
int dpa4k_stream_calibrate(const float* src, int64_t read_floats, float* dst,
                           int64_t write_floats, dpa4k_stream_t stream);

/* ------------------------------------------------------------------------
 * Launch shape (testing aid; no reference counterpart)
 * ---------------------------------------------------------------------- */

/* HIP launches fewer than 2^32 work-items along each grid dimension, so a
 * launch that needs more blocks than one row holds (16,777,215 blocks of 256
 * threads) continues in rows along y.  This lowers the blocks per row to
 * `blocks` (0 restores the hardware limit) for every later launch in the
 * process, so that tests reach the multi-row grids at small sizes.  Results
 * do not depend on it.  Not meant to be changed while other threads launch. */
int dpa4k_set_launch_row_limit(int64_t blocks);

#ifdef __cplusplus
}
#endif

#endif /* DPA4K_H */

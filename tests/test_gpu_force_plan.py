"""The planned (blob) force assembly against the direct kernel, the oracle and an exact plan restatement.

The planned path (dpa4k_force_assembly_plan + dpa4k_force_assembly_f*_planned)
adds the same terms as the direct gather kernel in another fixed order: the
destination sums of each piece, then each record's source sums, in blob
order.  The two paths therefore agree within rounding, and the planned one
is reproducible run to run.  Its layout is checked exactly against a NumPy
restatement of the plan's definition: positions along the breadth-first tree
(float32 arithmetic, as the kernels do it), Morton cells, blobs of
2816 / 1408 concatenated rows, pieces, entries (source slots in the spatial
order of their atoms) and records.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from bysj_amd import workloads
from bysj_amd.kernels import _C
from oracle import loops
from oracle import segment as ref
from parity import announce, assert_bitwise, assert_close_scaled, assert_fp64

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
ROWS = {4: 2816, 8: 1408}  # blob rows per value size (67,584 bytes of LDS)


def _random_graph(atoms, edges, seed, src_hubs=(), dst_hubs=()):
    gen = torch.Generator().manual_seed(seed)
    dst = torch.randint(0, atoms, (edges,), generator=gen)
    for hub, count in dst_hubs:  # atoms with many incoming edges: segments split over blobs
        dst[torch.randperm(edges, generator=gen)[:count]] = hub
    dst = torch.sort(dst).values
    src = torch.randint(0, atoms, (edges,), generator=gen)
    for hub, count in src_hubs:  # atoms that are the source of many edges
        src[torch.randperm(edges, generator=gen)[:count]] = hub
    g = torch.randn(edges, 3, generator=gen, dtype=torch.float64)
    v = torch.randn(edges, 3, generator=gen, dtype=torch.float64)
    order, src_offsets = ref.group_by_source(src, atoms)
    return {"grad_edge": g, "edge_vec": v, "src": src, "dst": dst, "dst_offsets": ref.segment_offsets(dst, atoms),
            "src_offsets": src_offsets, "src_order": order}


def _chain(atoms, seed, components=1):
    """Atoms on lines, each bonded to its neighbours both ways: a breadth-first tree as deep as a
    component is long; with several components the later ones are never reached from the root."""
    gen = torch.Generator().manual_seed(seed)
    per = atoms // components
    dst, src = [], []
    for k in range(atoms):
        start = (k // per) * per
        for other in (k - 1, k + 1):
            if start <= other < min(start + per, atoms):
                dst.append(k)
                src.append(other)
    dst, src = torch.tensor(dst), torch.tensor(src)
    edges = dst.numel()
    position = torch.arange(atoms, dtype=torch.float64)[:, None] * torch.tensor([1.0, 0.3, -0.2], dtype=torch.float64)
    v = position[src] - position[dst]
    g = torch.randn(edges, 3, generator=gen, dtype=torch.float64)
    order, src_offsets = ref.group_by_source(src, atoms)
    return {"grad_edge": g, "edge_vec": v, "src": src, "dst": dst, "dst_offsets": ref.segment_offsets(dst, atoms),
            "src_offsets": src_offsets, "src_order": order}


def _water(atoms, seed, spatial):
    graph = workloads.water_graph(atoms, seed=seed, spatial_order=spatial)
    return workloads.force_config(graph, seed=seed, device="cpu", dtype=torch.float64)


CASES = {
    "water_random_numbering": lambda: _water(4096, 5, False),
    "water_morton_numbering": lambda: _water(4096, 5, True),
    "source_hubs": lambda: _random_graph(700, 20000, 11, src_hubs=((3, 600), (650, 250))),
    "destination_hubs_split_over_blobs": lambda: _random_graph(900, 30000, 29, dst_hubs=((5, 7000), (400, 3000))),
    "three_atoms": lambda: _random_graph(3, 5, 12),
    "two_blobs_and_one_edge": lambda: _random_graph(300, 2 * 2816 + 1, 13),
    "chain_of_3000_atoms": lambda: _chain(3000, 41),
    "three_chains_two_unreached": lambda: _chain(3000, 43, components=3),
}


# ---------------------------------------------------------------------------
# the plan, restated
# ---------------------------------------------------------------------------

def _morton_bits(atoms):
    bits = 1
    while bits < 10 and (1 << (3 * (bits + 1))) <= atoms:
        bits += 1
    return bits


def _plan_restated(case, value_bytes, hint=True):
    """Every array of the plan from its definition (see dpa4k_force_assembly_plan)."""
    dst_off = case["dst_offsets"].numpy()
    src_off = case["src_offsets"].numpy()
    order = case["src_order"].numpy()
    atoms, edges = dst_off.size - 1, order.size
    rows = ROWS[value_bytes]
    blobs = -(-edges // rows)
    slot_atom = np.repeat(np.arange(atoms), np.diff(src_off))
    valid = (order >= 0) & (order < edges)
    edge_src = np.full(edges, -1, dtype=np.int64)
    np.maximum.at(edge_src, order[valid], slot_atom[valid])
    dst_of = np.repeat(np.arange(atoms), np.diff(dst_off))

    # breadth-first positions: an unreached atom joins level d + 1 through its first incoming
    # edge whose source is at level d; r_k = r_s - v_e in float32
    unreached = np.iinfo(np.int32).max
    level = np.full(atoms, unreached, dtype=np.int64)
    pos = np.zeros((atoms, 3), dtype=np.float32)
    vec = case["edge_vec"].numpy().astype(np.float64 if value_bytes == 8 else np.float32).astype(np.float32)
    level[int(dst_of[0])] = 0
    depth = 0
    while hint:
        before = level.copy()
        moved = False
        for k in np.nonzero(before == unreached)[0]:
            for e in range(dst_off[k], dst_off[k + 1]):
                s = edge_src[e]
                if s >= 0 and before[s] == depth:
                    pos[k] = pos[s] - vec[e]
                    level[k] = depth + 1
                    moved = True
                    break
        if not moved:
            break
        depth += 1
    reached = level != unreached
    bits = _morton_bits(atoms)
    cells = np.float32(1 << bits)
    lo = pos[reached].min(0)
    hi = pos[reached].max(0)
    extent = np.float32(max(hi[0] - lo[0], hi[1] - lo[1], hi[2] - lo[2]))
    scale = cells / extent if 0 < extent < np.inf else np.float32(0)
    q = np.minimum(np.maximum((pos - lo) * np.float32(scale), np.float32(0)), cells - np.float32(1)).astype(np.int64)
    key = np.zeros(atoms, dtype=np.int64)
    for b in range(bits):
        for i in range(3):
            key |= ((q[:, i] >> b) & 1) << (3 * b + (2 - i))
    key[~reached] = 1 << (3 * bits)
    perm = np.argsort(key, kind="stable")
    rank = np.empty(atoms, dtype=np.int64)
    rank[perm] = np.arange(atoms)
    degree = np.diff(dst_off)[perm]
    cum = np.concatenate([[0], np.cumsum(degree)])

    piece_t, piece_count, blob_piece = [], [], np.zeros(blobs + 1, dtype=np.int64)
    for i in range(atoms):
        begin, end = cum[i], cum[i + 1]
        piece_count.append(0 if end <= begin else (end - 1) // rows - begin // rows + 1)
        if end > begin:
            for w in range(begin // rows, (end - 1) // rows + 1):
                start = max(begin, w * rows)
                if start == w * rows:
                    blob_piece[w] = len(piece_t)
                piece_t.append(start)
    pieces = len(piece_t)
    blob_piece[blobs] = pieces
    piece_first = np.concatenate([[0], np.cumsum(piece_count)])
    tpos = cum[rank[dst_of]] + (np.arange(edges) - dst_off[dst_of])
    row_edge = np.empty(edges, dtype=np.int64)
    row_edge[tpos] = np.arange(edges)

    # entries: the source slots listed position by position, sorted stably by the blob of their edge
    listed = np.concatenate([np.arange(src_off[a], src_off[a + 1]) for a in perm] + [np.zeros(0, np.int64)])
    listed = listed[valid[listed]]
    sorted_slots = listed[np.argsort(tpos[order[listed]] // rows, kind="stable")]
    entry_blob = tpos[order[sorted_slots]] // rows
    entry_row = tpos[order[sorted_slots]] - entry_blob * rows
    entry_atom = slot_atom[sorted_slots]
    start = np.ones(sorted_slots.size, dtype=bool)
    start[1:] = (entry_blob[1:] != entry_blob[:-1]) | (entry_atom[1:] != entry_atom[:-1])
    rec_first = np.concatenate([np.nonzero(start)[0], [sorted_slots.size]])
    records = rec_first.size - 1
    rec_blob = entry_blob[rec_first[:-1]]
    blob_rec = np.searchsorted(rec_blob, np.arange(blobs + 1), side="left")
    blob_entry = np.searchsorted(entry_blob, np.arange(blobs + 1), side="left")
    # each blob's records by descending length (capped at 63), stable; their entries follow
    length = np.diff(rec_first)
    balanced = np.argsort(rec_blob * 64 + (63 - np.minimum(length, 63)), kind="stable")
    entry_row = np.concatenate([entry_row[rec_first[r]:rec_first[r + 1]] for r in balanced] + [entry_row[:0]])
    rec_entry = np.concatenate([[0], np.cumsum(length[balanced])])
    rec_position = rank[entry_atom[rec_first[:-1]]][balanced]
    pos_records = np.argsort(rec_position, kind="stable")  # record ids grouped by position, in blob order
    pos_rec = np.concatenate([[0], np.cumsum(np.bincount(rec_position, minlength=atoms))])
    return {"perm": perm, "piece_first": piece_first, "piece_t": np.append(piece_t, edges), "blob_piece": blob_piece,
            "blob_rec": blob_rec, "blob_entry": blob_entry, "row_edge": row_edge, "entry_row": entry_row,
            "rec_entry": rec_entry, "pos_records": pos_records, "pos_rec": pos_rec, "records": records, "pieces": pieces}


def _decode_plan(plan: _C.ForcePlan):
    """The plan buffer's arrays (carved in order, each 256-byte aligned)."""
    atoms, edges = plan.n_nodes, plan.n_edges
    blobs = -(-edges // ROWS[plan.value_bytes])
    e = max(edges, 1)
    layout = [("header", 6, np.int64), ("perm", atoms, np.int32), ("piece_first", atoms + 1, np.int32),
              ("piece_t", atoms + blobs + 1, np.int32), ("blob_piece", blobs + 1, np.int32),
              ("blob_rec", blobs + 1, np.int32), ("blob_entry", blobs + 1, np.int32), ("row_edge", e, np.int32),
              ("entry_row", e, np.uint16), ("rec_entry", e + 1, np.int32), ("pos_records", e, np.int32),
              ("pos_rec", atoms + 1, np.int32)]
    raw = plan.plan.cpu().numpy()
    out, at = {}, 0
    for name, count, dtype in layout:
        size = count * np.dtype(dtype).itemsize
        out[name] = raw[at:at + size].view(dtype)
        at += -(-size // 256) * 256
    return out


def _check_plan_layout(plan, case):
    expected = _plan_restated(case, plan.value_bytes)
    got = _decode_plan(plan)
    assert plan.n_records == expected["records"] and plan.n_pieces == expected["pieces"]
    magic = int.from_bytes(b"DPA4FPLN", "little")  # the header names what the plan was built for
    np.testing.assert_array_equal(got["header"], [magic, plan.n_edges, plan.n_nodes, plan.value_bytes,
                                                  plan.n_records, plan.n_pieces])
    lengths = {"piece_t": expected["pieces"] + 1, "rec_entry": expected["records"] + 1,
               "pos_records": expected["records"], "entry_row": expected["rec_entry"][-1]}
    for name in ("perm", "piece_first", "piece_t", "blob_piece", "blob_rec", "blob_entry", "row_edge", "entry_row",
                 "rec_entry", "pos_records", "pos_rec"):
        n = lengths.get(name, expected[name].size)
        np.testing.assert_array_equal(got[name][:n], expected[name][:n], err_msg=f"plan: {name}")


def _on_device(case):
    return {k: v.to(DEV) for k, v in case.items()}


def _run(d, dtype, plan=None):
    """Force and virial of a case already on the device (a plan is tied to those very offsets tensors)."""
    return _C.force_assembly(d["grad_edge"].to(dtype), d["edge_vec"].to(dtype), d["dst_offsets"], d["src_offsets"],
                             d["src_order"], plan=plan)


def _plan(d, dtype):
    return _C.force_assembly_plan(d["dst_offsets"], d["src_offsets"], d["src_order"], d["edge_vec"].to(dtype),
                                  value_bytes=torch.empty((), dtype=dtype).element_size())


@pytest.mark.parametrize("name", list(CASES))
def test_planned_force_matches_the_direct_kernel_and_its_restated_plan(name):
    case = CASES[name]()
    atoms = case["dst_offsets"].numel() - 1
    announce("force plan", name, atoms, case["src_order"].numel())
    d = _on_device(case)
    for dtype in (torch.float32, torch.float64):
        plan = _plan(d, dtype)
        _check_plan_layout(plan, case)
        direct = _run(d, dtype)
        planned = _run(d, dtype, plan)
        again = _run(d, dtype, plan)
        for label, a, b, c in zip(("force", "virial"), direct, planned, again):
            if dtype == torch.float32:
                assert_close_scaled(b, a, what=f"{name} {label}: planned vs direct")
            else:
                assert_fp64(b, a, f"{name} {label}: planned vs direct")
            assert_bitwise(c, b, f"{name} {dtype} {label}: planned run to run")


def test_planned_force_against_the_oracle_and_truth():
    case = _random_graph(500, 30000, 17, src_hubs=((7, 400),), dst_hubs=((9, 4000),))
    announce("force plan vs oracle")
    d = _on_device(case)
    force, virial = _run(d, torch.float32, _plan(d, torch.float32))
    g, v = case["grad_edge"].float(), case["edge_vec"].float()
    e_force, e_virial = ref.force_assembly_reference(g, v, case["src"], case["dst"], case["dst_offsets"],
                                                     case["src_offsets"])
    t_force, t_virial = loops.force_assembly_loop(g, v, case["src"], case["dst"], 500)
    assert_close_scaled(force, e_force, what="fp32 force vs oracle")
    assert_close_scaled(virial, e_virial, what="fp32 virial vs oracle")
    assert_close_scaled(force, t_force, what="fp32 force vs truth")
    assert_close_scaled(virial, t_virial, what="fp32 virial vs truth")
    force64, virial64 = _run(d, torch.float64, _plan(d, torch.float64))
    t_force, t_virial = loops.force_assembly_loop(case["grad_edge"], case["edge_vec"], case["src"], case["dst"], 500)
    assert_fp64(force64, t_force, "fp64 force vs truth")
    assert_fp64(virial64, t_virial, "fp64 virial vs truth")


def _invalid_slots():
    case = _random_graph(200, 9000, 19)
    order = case["src_order"].clone()
    order[5], order[700], order[-1] = -1, order.numel() + 7, -3
    return dict(case, src_order=order)


def _one_edge_named_by_every_slot():
    """src_order names edge 0 from every slot: one blob holds every entry (more than it stages in LDS)
    and more records than its threads take in their first rounds."""
    case = _random_graph(4000, 12000, 37)
    return dict(case, src_order=torch.zeros_like(case["src_order"]))


@pytest.mark.parametrize("make", [_invalid_slots, _one_edge_named_by_every_slot],
                         ids=["out_of_range_slots", "one_edge_named_by_every_slot"])
def test_planned_force_takes_source_slots_like_the_direct_kernel(make):
    case = make()
    announce("force plan, unusual src_order", make.__name__)
    d = _on_device(case)
    for dtype in (torch.float32, torch.float64):
        plan = _plan(d, dtype)
        _check_plan_layout(plan, case)
        for label, a, b in zip(("force", "virial"), _run(d, dtype), _run(d, dtype, plan)):
            if dtype == torch.float32:
                assert_close_scaled(b, a, what=f"{label}: planned vs direct")
            else:
                assert_fp64(b, a, f"{label}: planned vs direct")


def test_planned_force_without_a_geometry_hint_keeps_the_natural_order():
    case = _water(2048, 3, False)
    announce("force plan without a hint")
    d = _on_device(case)
    plan = _C.force_assembly_plan(d["dst_offsets"], d["src_offsets"], d["src_order"], None, value_bytes=4)
    np.testing.assert_array_equal(_decode_plan(plan)["perm"], np.arange(2048), err_msg="identity order")
    for label, a, b in zip(("force", "virial"), _run(d, torch.float32), _run(d, torch.float32, plan)):
        assert_close_scaled(b, a, what=f"{label} without a hint")


def test_planned_force_without_edges_and_plan_checks():
    announce("force plan, empty graph and checks")
    offsets = torch.zeros(5, dtype=torch.int64, device=DEV)
    order = torch.empty(0, dtype=torch.int64, device=DEV)
    empty = torch.empty((0, 3), device=DEV)
    plan = _C.force_assembly_plan(offsets, offsets, order, empty, value_bytes=4)
    force, virial = _C.force_assembly(empty, empty, offsets, offsets, order, plan=plan)
    assert force.shape == (4, 3) and virial.shape == (4, 9)
    assert force.count_nonzero().item() == 0 and virial.count_nonzero().item() == 0
    d = _on_device(_random_graph(50, 800, 23))
    plan = _plan(d, torch.float32)
    with pytest.raises(RuntimeError, match="another graph, device or dtype"):
        _run(d, torch.float64, plan)  # a float32 plan does not serve float64 rows
    with pytest.raises(RuntimeError, match="another graph"):
        _run(_on_device(_random_graph(50, 801, 23)), torch.float32, plan)
    copy = dict(d, dst_offsets=d["dst_offsets"].clone())  # the same values in another tensor
    with pytest.raises(RuntimeError, match="another graph"):
        _run(copy, torch.float32, plan)
    bad = {k: v.clone() for k, v in d.items()}
    bad["dst_offsets"][10] = 10 ** 6  # not a CSR of the edge list
    with pytest.raises(ValueError, match="not a CSR"):
        _C.force_assembly_plan(bad["dst_offsets"], bad["src_offsets"], bad["src_order"], bad["edge_vec"].float())


def test_operator_plans_compact_graphs_only():
    """kernels.force_assembly keeps a plan for water graphs in float32 (either numbering) and in float64 with
    random numbering, and none for float64 with Morton numbering or for a graph whose edge vectors carry no
    geometry (records about as many as edges)."""
    from bysj_amd import kernels
    from bysj_amd.kernels import segment as segment_ops

    announce("force plan policy")
    segment_ops._FORCE_PLANS.clear()
    kept = {}
    for spatial in (False, True):
        case = _water(16384, 6, spatial)
        assert case["src_order"].numel() >= segment_ops._ForcePlanCache.MIN_EDGES
        d = {k: v.to(DEV) for k, v in case.items()}
        for dtype in (torch.float32, torch.float64):
            args = (d["grad_edge"].to(dtype), d["edge_vec"].to(dtype), d["src"], d["dst"], d["dst_offsets"],
                    d["src_offsets"], d["src_order"])
            force, virial = kernels.force_assembly(*args)
            plan = segment_ops._FORCE_PLANS._entries[(id(d["src_order"]), dtype)][2]
            direct = _C.force_assembly(args[0], args[1], d["dst_offsets"], d["src_offsets"], d["src_order"])
            if dtype == torch.float64 and spatial:
                assert plan is None, "float64 with Morton numbering keeps the direct kernel"
                assert_bitwise(force, direct[0], "operator force, direct")
                continue
            assert plan is not None, f"a plan for the water graph (spatial={spatial}, {dtype})"
            assert plan.n_records * segment_ops._ForcePlanCache.MIN_EDGES_PER_RECORD <= plan.n_edges
            check = assert_close_scaled if dtype == torch.float32 else assert_fp64
            check(force, direct[0], what=f"operator force (spatial={spatial}, {dtype})")
            check(virial, direct[1], what=f"operator virial (spatial={spatial}, {dtype})")
        kept[spatial] = d
    scattered = {k: v.to(DEV) for k, v in _random_graph(4096, 1 << 17, 31).items()}
    args = (scattered["grad_edge"].float(), scattered["edge_vec"].float(), scattered["src"], scattered["dst"],
            scattered["dst_offsets"], scattered["src_offsets"], scattered["src_order"])
    force, _ = kernels.force_assembly(*args)
    assert segment_ops._FORCE_PLANS._entries[(id(scattered["src_order"]), torch.float32)][2] is None
    assert_bitwise(force, _C.force_assembly(args[0], args[1], args[4], args[5], args[6])[0], "unplanned operator")
    # an in-place write to src_order drops the cached plan; the next call plans again
    d = kept[False]
    before = segment_ops._FORCE_PLANS._entries[(id(d["src_order"]), torch.float32)][2]
    d["src_order"].add_(0)
    kernels.force_assembly(d["grad_edge"].float(), d["edge_vec"].float(), d["src"], d["dst"], d["dst_offsets"],
                           d["src_offsets"], d["src_order"])
    after = segment_ops._FORCE_PLANS._entries[(id(d["src_order"]), torch.float32)][2]
    assert after is not None and after is not before
    segment_ops._FORCE_PLANS.clear()


def test_planned_call_reports_a_plan_that_does_not_match_it():
    """Through the C ABI: a plan whose header differs from the call (record count, or a buffer that no build
    finished) yields NaN in every output and DPA4K_FORCE_PLAN_MISMATCH in the status word; a matching call
    clears the word."""
    from bysj_amd.kernels import _lib

    announce("force plan mismatch through the C ABI")
    library = _lib.load()
    d = _on_device(_random_graph(300, 9000, 47))
    g, v = d["grad_edge"].float(), d["edge_vec"].float()
    plan = _plan(d, torch.float32)
    status = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    force = torch.empty((300, 3), device=DEV)
    virial = torch.empty((300, 9), device=DEV)

    def call(plan_buffer, n_records):
        stream = torch.cuda.current_stream().cuda_stream
        rc = library.dpa4k_force_assembly_f32_planned(
            g.data_ptr(), v.data_ptr(), force.data_ptr(), virial.data_ptr(), 9000, 300, plan_buffer.data_ptr(),
            plan_buffer.numel(), plan.records.data_ptr(), plan.records.numel(), n_records, plan.n_pieces,
            status.data_ptr(), stream)
        assert rc == _lib.OK, library.dpa4k_last_error()
        torch.cuda.synchronize()
        return int(status.item())

    assert call(plan.plan, plan.n_records - 1) == 4  # DPA4K_FORCE_PLAN_MISMATCH
    assert torch.isnan(force).all() and torch.isnan(virial).all()
    assert call(torch.zeros_like(plan.plan), plan.n_records) == 4  # no build finished in this buffer
    assert torch.isnan(force).all() and torch.isnan(virial).all()
    assert call(plan.plan, plan.n_records) == 0
    direct = _run(d, torch.float32)
    assert_close_scaled(force, direct[0], what="matching call: force")
    assert_close_scaled(virial, direct[1], what="matching call: virial")


def test_planned_float32_records_stay_within_their_stated_bound():
    """Records sum their few terms in float32 (fused products); against the fp64 truth every output component
    stays within L * 2^-24 * (the atom's sum of absolute terms) plus the final rounding, L the longest record."""
    case = _water(4096, 8, False)
    announce("force plan float32 record bound")
    d = _on_device(case)
    plan = _plan(d, torch.float32)
    longest = int(np.diff(_decode_plan(plan)["rec_entry"][:plan.n_records + 1]).max())
    force, virial = _run(d, torch.float32, plan)
    g = case["grad_edge"].float().double()
    v = case["edge_vec"].float().double()
    atoms = case["dst_offsets"].numel() - 1
    t_force, t_virial = (torch.from_numpy(t) for t in loops.force_assembly_loop(g, v, case["src"], case["dst"], atoms))
    # the sum of absolute terms per output component: |g| on both sides, |g_r v_c| on the source side
    a_force = torch.zeros(atoms, 3, dtype=torch.float64).index_add_(0, case["dst"], g.abs())
    a_force.index_add_(0, case["src"], g.abs())
    a_virial = torch.zeros(atoms, 9, dtype=torch.float64).index_add_(
        0, case["src"], (g.abs().unsqueeze(2) * v.abs().unsqueeze(1)).reshape(-1, 9))
    unit = 2.0 ** -24
    for label, got, truth, absolute in (("force", force, t_force, a_force), ("virial", virial, t_virial, a_virial)):
        error = (got.double().cpu() - truth).abs()
        bound = (longest + 2) * unit * absolute + unit * truth.abs()
        assert bool((error <= bound).all()), f"{label}: worst excess {float((error - bound).max()):.3e}"

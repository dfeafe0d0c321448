"""Synthetic inputs of the benchmark configurations.

Graphs are built on the host from one seeded numpy PCG64 generator, drawn in
a fixed order; dense features are drawn with a seeded torch generator on the
device that will consume them (large feature tensors are not staged through
host memory).  All destination lists are sorted, so ``offsets`` addresses the
natural edge order directly.

config 1  segment_sum   N=1,024 nodes, in-degree max(1, Poisson(40)), src [E, 128] ~ N(0, 1)
config 2  softmax       N=16,384, 1 % hubs of degree 512, rest Poisson(48); logits [E, 8] ~ N(0, 4)
                        with 0.1 % of entries set to +-40, env ~ U(0.1, 1.1), null ~ N(0, 1)
config 3  GIE + RMSNorm water-like periodic box, N=24,576 atoms at 0.1 / A^3, r_c = 6 A
                        (~90 neighbours); zonal [E, 15], radial [E, 16, 64], slots 1..15;
                        RMSNorm over rows of 1,024 with eps 1e-6, scale ~ U(0.5, 1.5)
config 4  force         the config-3 generator at N=65,536; grad_edge [E, 3] ~ N(0, 0.5),
                        edge_vec = minimum-image vectors; fp32 and fp64
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass

import numpy as np
import torch


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def offsets_from_degrees(degrees: np.ndarray) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(degrees)]).astype(np.int64)


def poisson_degrees(n_nodes: int, mean: float, seed: int, *, minimum: int = 1,
                    hub_fraction: float = 0.0, hub_degree: int = 0) -> np.ndarray:
    """Per-node in-degrees: max(minimum, Poisson(mean)), with a seeded hub subset."""
    generator = rng(seed)
    degrees = np.maximum(minimum, generator.poisson(mean, size=n_nodes)).astype(np.int64)
    hubs = int(round(hub_fraction * n_nodes))
    if hubs:
        degrees[generator.permutation(n_nodes)[:hubs]] = hub_degree
    return degrees


def dst_from_degrees(degrees: np.ndarray) -> np.ndarray:
    return np.repeat(np.arange(degrees.shape[0], dtype=np.int64), degrees)


@dataclass
class WaterGraph:
    """Directed minimum-image neighbour graph, edges sorted by (dst, src)."""

    n_atoms: int
    box: float
    positions: np.ndarray   # [N, 3] float64
    types: np.ndarray       # [N] int64, 0 = O, 1 = H
    src: np.ndarray         # [E] int64
    dst: np.ndarray         # [E] int64, non-decreasing
    edge_vec: np.ndarray    # [E, 3] float64, position[src] - position[dst] (minimum image)

    @property
    def n_edges(self) -> int:
        return int(self.dst.shape[0])

    def degrees(self) -> np.ndarray:
        return np.bincount(self.dst, minlength=self.n_atoms).astype(np.int64)

    def offsets(self) -> np.ndarray:
        return offsets_from_degrees(self.degrees())


def morton_order(positions: np.ndarray, box: float, bin_size: float) -> np.ndarray:
    """Permutation sorting atoms by the Z-order (Morton) key of their spatial bin,
    the kind of periodic spatial sort MD engines apply to their atom arrays."""
    bins = np.minimum((positions // bin_size).astype(np.int64), max(1, int(box // bin_size)) - 1)
    key = np.zeros(positions.shape[0], dtype=np.int64)
    for bit in range(21):
        for axis in range(3):
            key |= ((bins[:, axis] >> bit) & 1) << (3 * bit + axis)
    return np.argsort(key, kind="stable")


def water_graph(n_atoms: int, seed: int, *, rcut: float = 6.0, density: float = 0.1,
                spatial_order: bool = False, device: str | torch.device = "cpu") -> WaterGraph:
    """Uniform random positions in a periodic cube; O:H = 1:2 types shuffled by the seed.

    Atom indices follow the draw order (no spatial locality) unless
    ``spatial_order`` renumbers them by the Morton key of rcut/2 bins.
    Positions and the cell lists come from the seeded host generator; the
    candidate pairs of the 27 neighbouring cells are filtered with torch on
    ``device`` (the GPU builds a 65k-atom box in about a second).  Every
    step is exact or correctly rounded IEEE arithmetic in a fixed order
    (difference, minimum image, ``(dx^2 + dy^2) + dz^2``), and the edges end
    sorted by the unique key ``(dst, src)``, so every device yields the same
    graph bit for bit.
    """
    generator = rng(seed)
    box = (n_atoms / density) ** (1.0 / 3.0)
    types = np.ones(n_atoms, dtype=np.int64)
    types[: n_atoms // 3] = 0
    types = types[generator.permutation(n_atoms)]
    positions = generator.uniform(0.0, box, size=(n_atoms, 3))
    if spatial_order:
        permutation = morton_order(positions, box, rcut / 2.0)
        positions, types = positions[permutation], types[permutation]

    n_cell = int(box // rcut)
    if n_cell < 3:
        raise ValueError("water_graph needs a box of at least three cut-off lengths per side")
    cell_size = box / n_cell
    cell_xyz = np.minimum((positions // cell_size).astype(np.int64), n_cell - 1)
    cell = (cell_xyz[:, 0] * n_cell + cell_xyz[:, 1]) * n_cell + cell_xyz[:, 2]
    by_cell = np.argsort(cell, kind="stable")
    counts = np.bincount(cell, minlength=n_cell ** 3)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    width = int(counts.max())

    dev = torch.device(device)
    positions_t = torch.from_numpy(positions).to(dev)
    cell_xyz_t = torch.from_numpy(cell_xyz).to(dev)
    counts_t = torch.from_numpy(counts).to(dev)
    starts_t = torch.from_numpy(starts).to(dev)
    by_cell_t = torch.from_numpy(by_cell).to(dev)
    lane = torch.arange(width, device=dev)
    shifts = torch.tensor(list(itertools.product((-1, 0, 1), repeat=3)), device=dev)
    cutoff2 = rcut * rcut
    chunk = max(1024, (1 << 26) // (27 * width * 8))  # about 200 MB of candidate vectors per chunk
    keys, vectors = [], []
    for begin in range(0, n_atoms, chunk):
        atoms = torch.arange(begin, min(n_atoms, begin + chunk), device=dev)
        neighbour_xyz = (cell_xyz_t[atoms][:, None, :] + shifts[None, :, :]) % n_cell          # [A, 27, 3]
        neighbour = (neighbour_xyz[..., 0] * n_cell + neighbour_xyz[..., 1]) * n_cell + neighbour_xyz[..., 2]
        valid = lane < counts_t[neighbour][..., None]                                         # [A, 27, W]
        other = by_cell_t[torch.clamp(starts_t[neighbour][..., None] + lane, max=n_atoms - 1)]
        delta = positions_t[other] - positions_t[atoms][:, None, None, :]
        delta = delta - box * torch.round(delta / box)
        distance2 = (delta[..., 0] * delta[..., 0] + delta[..., 1] * delta[..., 1]) + delta[..., 2] * delta[..., 2]
        keep = valid & (distance2 < cutoff2) & (other != atoms[:, None, None])
        a, s, w = torch.nonzero(keep, as_tuple=True)
        keys.append(atoms[a] * n_atoms + other[a, s, w])
        vectors.append(delta[a, s, w])
    key, order = torch.sort(torch.cat(keys))
    vector = torch.cat(vectors)[order]
    dst = (key // n_atoms).cpu().numpy()
    src = (key % n_atoms).cpu().numpy()
    return WaterGraph(n_atoms, box, positions, types, src, dst, vector.cpu().numpy())


# ---------------------------------------------------------------------------
# configurations as device tensors
# ---------------------------------------------------------------------------

def _generator(device, seed):
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    return generator


def segment_sum_config(n_nodes: int = 1024, channels: int = 128, seed: int = 0, device="cpu",
                       scales: bool = False):
    degrees = poisson_degrees(n_nodes, 40.0, seed)
    dst = torch.from_numpy(dst_from_degrees(degrees)).to(device)
    offsets = torch.from_numpy(offsets_from_degrees(degrees)).to(device)
    generator = _generator(device, seed)
    src = torch.randn((dst.numel(), channels), generator=generator, device=device)
    case = {"src": src, "dst": dst, "offsets": offsets, "edge_scale": None, "node_scale": None}
    if scales:
        case["edge_scale"] = torch.rand((dst.numel(),), generator=generator, device=device) + 0.5
        case["node_scale"] = torch.rand((n_nodes,), generator=generator, device=device) + 0.5
    return case


def segment_softmax_features(n_edges: int, n_nodes: int, channels: int = 8, seed: int = 0, device="cpu",
                             null: bool = True, masked_fraction: float = 0.0):
    """Config-2 features of one graph: logits ~ N(0, 4) with 0.1 % of entries at +-40,
    env ~ U(0.1, 1.1) (a fraction set to -0.5 when masked_fraction > 0), null ~ N(0, 1)."""
    generator = _generator(device, seed)
    logit = torch.randn((n_edges, channels), generator=generator, device=device) * 2.0
    flat = logit.view(-1)
    extreme = torch.rand(flat.shape, generator=generator, device=device) < 1e-3
    sign = torch.where(torch.rand(flat.shape, generator=generator, device=device) < 0.5, -40.0, 40.0)
    flat[extreme] = sign[extreme]
    env = torch.rand((n_edges,), generator=generator, device=device) + 0.1
    if masked_fraction > 0:
        env[torch.rand((n_edges,), generator=generator, device=device) < masked_fraction] = -0.5
    null_logit = torch.randn((n_nodes, channels), generator=generator, device=device) if null else None
    return {"logit": logit, "env": env, "null_logit": null_logit}


def segment_softmax_config(n_nodes: int = 16384, channels: int = 8, seed: int = 0, device="cpu",
                           null: bool = True, masked_fraction: float = 0.0):
    degrees = poisson_degrees(n_nodes, 48.0, seed, hub_fraction=0.01, hub_degree=512)
    edges = int(degrees.sum())
    dst = torch.from_numpy(dst_from_degrees(degrees)).to(device)
    offsets = torch.from_numpy(offsets_from_degrees(degrees)).to(device)
    features = segment_softmax_features(edges, n_nodes, channels, seed, device, null, masked_fraction)
    return {"dst": dst, "offsets": offsets, **features}


def gie_config(graph: WaterGraph, seed: int = 0, device="cpu", *, primary: bool = True, channels: int = 64):
    """zonal [E, 15]; radial [E, 16, C] with slots 1..15 (primary) or [E, 3, C] with slot = l - 1."""
    edges = graph.n_edges
    dst = torch.from_numpy(graph.dst).to(device)
    generator = _generator(device, seed)
    zonal = torch.randn((edges, 15), generator=generator, device=device)
    if primary:
        radial = torch.randn((edges, 16, channels), generator=generator, device=device)
        slots = torch.arange(1, 16, dtype=torch.int64, device=device)
    else:
        radial = torch.randn((edges, 3, channels), generator=generator, device=device)
        slots = torch.tensor([0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2], dtype=torch.int64, device=device)
    inv = torch.rsqrt(torch.from_numpy(graph.degrees()).to(device=device, dtype=torch.float32) + 1.0)
    scale = torch.rand((16 * channels,), generator=generator, device=device) + 0.5
    return {"zonal": zonal, "radial": radial, "dst": dst, "radial_slot": slots, "inv_sqrt_deg": inv,
            "rms_scale": scale, "eps": 1e-6}


def force_config(graph: WaterGraph, seed: int = 0, device="cpu", dtype=torch.float32):
    edges = graph.n_edges
    generator = _generator(device, seed)
    grad_edge = (torch.randn((edges, 3), generator=generator, device=device, dtype=torch.float64)
                 * np.sqrt(0.5)).to(dtype)
    edge_vec = torch.from_numpy(graph.edge_vec).to(device=device, dtype=dtype)
    src = torch.from_numpy(graph.src).to(device)
    dst = torch.from_numpy(graph.dst).to(device)
    src_order = torch.from_numpy(np.argsort(graph.src, kind="stable").astype(np.int64)).to(device)
    src_offsets = torch.from_numpy(offsets_from_degrees(np.bincount(graph.src, minlength=graph.n_atoms))).to(device)
    dst_offsets = torch.from_numpy(graph.offsets()).to(device)
    return {"grad_edge": grad_edge, "edge_vec": edge_vec, "src": src, "dst": dst,
            "dst_offsets": dst_offsets, "src_offsets": src_offsets, "src_order": src_order}

"""Seeded synthetic sparse inputs for the SpTRSV / SpILU0 solver paths.

Every generator is vectorised NumPy, fully determined by its arguments and a
seed, and returns int32 pointer/index arrays with float64 values, which is the
layout the decorated loops of the reference consume
(reference: README.md:85-92, compiler/demo/sptrsv.py:26-43,
compiler/demo/spilu0.py:21-47).

Storage conventions (they matter for the loops, which index the diagonal by
position):

* CSC lower-triangular factors store the diagonal FIRST in every column.
* CSR lower-triangular factors store the diagonal LAST in every row.
* Full CSR matrices (ILU0) have sorted column indices in every row.
"""

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Workload:
    """One named problem instance."""

    name: str
    kind: str                 # "sptrsv_csc" | "sptrsv_csr" | "ilu0_csr"
    n: int
    indptr: np.ndarray        # int32[n + 1]
    indices: np.ndarray       # int32[nnz]
    data: np.ndarray          # float64[nnz]
    rhs: np.ndarray | None    # float64[n] (None for ILU0)
    execution_mode: str       # executor the configuration is quoted on
    seed: int
    meta: dict = field(default_factory=dict)

    @property
    def nnz(self):
        return int(self.indptr[-1])

    @property
    def algorithmic_bytes(self):
        """Bytes every implementation must move at least once.

        SpTRSV: 12*nnz (fp64 value + int32 index) + 4*(n+1) pointers + 8n
        right-hand side + 8n solution.  ILU0 in place: values read and written
        (16*nnz), indices (4*nnz) and pointers (4*(n+1)).
        """
        if self.kind == "ilu0_csr":
            return 20 * self.nnz + 4 * self.n + 4
        return 12 * self.nnz + 20 * self.n + 4

    @property
    def true_flops(self):
        """Floating-point operations of the sequential loop: SpTRSV one
        division per row and a multiply-add per off-diagonal entry; ILU0
        counted on the pattern (``ilu0_true_flops``)."""
        if self.kind == "ilu0_csr":
            if "true_flops" not in self.meta:
                self.meta["true_flops"] = ilu0_true_flops(
                    self.indptr, self.indices, self.n)
            return self.meta["true_flops"]
        return 2 * (self.nnz - self.n) + self.n

    @property
    def reference_style_flops(self):
        """The reference harness counts n + 2*nnz for SpTRSV and 2*nnz for
        ILU0 (benchmark/sptrsv_benchmark.py:626,
        benchmark/spilu0_benchmark.py:767)."""
        if self.kind == "ilu0_csr":
            return 2 * self.nnz
        return self.n + 2 * self.nnz


def ilu0_true_flops(indptr, indices, n):
    """Operation count of in-place ILU0 on a CSR pattern with sorted rows
    (compiler/demo/spilu0.py:21-47): for every entry (i, k) below the
    diagonal one division, and one multiply-subtract (2 flops) for every
    j > k that rows i and k both hold.  Counted with sparse pattern algebra:
    (L U)[i, j] = number of pivots k < i with (i, k) and (k, j > k) present,
    summed over the positions of the pattern itself."""
    from scipy import sparse
    ones = np.ones(len(indices), dtype=np.int64)
    pattern = sparse.csr_matrix((ones, indices, indptr), shape=(n, n))
    lower = sparse.tril(pattern, k=-1, format="csr")
    upper = sparse.triu(pattern, k=1, format="csr")
    updates = (lower @ upper).multiply(pattern).sum()
    return int(lower.nnz) + 2 * int(updates)


def _grid_coordinates(shape):
    """Natural (x fastest) ordering of a 1-, 2- or 3-D grid."""
    dims = tuple(int(d) for d in shape)
    total = int(np.prod(dims))
    ids = np.arange(total, dtype=np.int64)
    coords = []
    stride = 1
    strides = []
    for d in dims:
        coords.append((ids // stride) % d)
        strides.append(stride)
        stride *= d
    return ids, coords, strides, dims


def stencil_lower_csc(shape, diagonal, off_diagonal=-1.0):
    """Lower triangle (with diagonal) of the (2d+1)-point Laplacian stencil.

    Natural ordering; column ``i`` holds row ``i`` (the diagonal, first) and
    the rows ``i + stride_d`` of its forward neighbours, ascending.
    """
    ids, coords, strides, dims = _grid_coordinates(shape)
    n = ids.size
    present = [coords[d] < dims[d] - 1 for d in range(len(dims))]
    counts = 1 + sum(p.astype(np.int64) for p in present)
    indptr = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = np.empty(nnz, dtype=np.int32)
    data = np.empty(nnz, dtype=np.float64)
    cursor = indptr[:-1].copy()
    indices[cursor] = ids
    data[cursor] = diagonal
    cursor += 1
    for d in range(len(dims)):
        mask = present[d]
        where = cursor[mask]
        indices[where] = ids[mask] + strides[d]
        data[where] = off_diagonal
        cursor[mask] += 1
    return indptr.astype(np.int32), indices, data


def stencil9_csr(nx, ny, diagonal=8.0, off_diagonal=-1.0, perturbation=0.01,
                 seed=0):
    """Full 9-point 2-D stencil matrix in CSR with sorted rows."""
    rng = np.random.default_rng(seed)
    ids = np.arange(nx * ny, dtype=np.int64)
    x = ids % nx
    y = ids // nx
    offsets = [(-1, -1), (0, -1), (1, -1), (-1, 0), (0, 0), (1, 0),
               (-1, 1), (0, 1), (1, 1)]
    masks = []
    for dx, dy in offsets:
        masks.append(
            (x + dx >= 0) & (x + dx < nx) & (y + dy >= 0) & (y + dy < ny)
        )
    counts = sum(m.astype(np.int64) for m in masks)
    indptr = np.zeros(nx * ny + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = np.empty(nnz, dtype=np.int32)
    is_diagonal = np.zeros(nnz, dtype=bool)
    cursor = indptr[:-1].copy()
    for (dx, dy), mask in zip(offsets, masks):
        where = cursor[mask]
        indices[where] = ids[mask] + dx + dy * nx
        if dx == 0 and dy == 0:
            is_diagonal[where] = True
        cursor[mask] += 1
    data = off_diagonal + rng.uniform(-perturbation, perturbation, nnz)
    data[is_diagonal] = diagonal
    return indptr.astype(np.int32), indices, data


POWER_LAW_SCALE = 3.3


def power_law_lower_csr(n, alpha=2.1, max_count=512, seed=0,
                        scale=POWER_LAW_SCALE):
    """Random lower-triangular CSR factor with a heavy-tailed row length.

    Row ``i`` has ``k_i = min(i, clip(floor(scale * U^(-1/(alpha-1))), 1,
    max_count))`` off-diagonals (a Pareto tail with exponent ``alpha``;
    ``scale`` is fixed so the mean is about 16).  Columns are DISTINCT, drawn
    by mapping a sorted with-replacement sample of ``[0, i - k_i]`` to a
    strictly increasing sequence (``c_j = s_j + j``); they are distinct because
    the reference's DAG has set semantics, so duplicate columns would make the
    unique in-degree differ from the entry count.  Values ~ U[-1, 1]; the
    diagonal ``1 + sum|row|`` is stored last in the row.
    """
    rng = np.random.default_rng(seed)
    u = rng.random(n)
    counts = np.clip(
        np.floor(scale * (1.0 - u) ** (-1.0 / (alpha - 1.0))), 1, max_count
    ).astype(np.int64)
    counts = np.minimum(counts, np.arange(n, dtype=np.int64))
    row_nnz = counts + 1
    indptr = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(row_nnz, out=indptr[1:])
    nnz = int(indptr[-1])
    off_total = int(counts.sum())
    rows = np.repeat(np.arange(n, dtype=np.int64), counts)
    span = (rows - counts[rows] + 1).astype(np.float64)
    sample = np.floor(rng.random(off_total) * span).astype(np.int64)
    order = np.argsort(rows * np.int64(n + 1) + sample, kind="stable")
    sample = sample[order]
    off_start = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(counts, out=off_start[1:])
    within = np.arange(off_total, dtype=np.int64) - off_start[rows]
    columns = sample + within
    values = rng.uniform(-1.0, 1.0, off_total)
    indices = np.empty(nnz, dtype=np.int32)
    data = np.empty(nnz, dtype=np.float64)
    destination = indptr[rows] + within
    indices[destination] = columns
    data[destination] = values
    diagonal_position = indptr[1:] - 1
    indices[diagonal_position] = np.arange(n, dtype=np.int32)
    row_abs = np.bincount(rows, weights=np.abs(values), minlength=n)
    data[diagonal_position] = 1.0 + row_abs
    return indptr.astype(np.int32), indices, data


def banded_lower_csc(n, bandwidth=8, low=-0.1, high=0.1, seed=0):
    """Banded lower-triangular CSC factor: column ``i`` holds the unit diagonal
    first, then rows ``i+1 .. min(i+bandwidth, n-1)``."""
    rng = np.random.default_rng(seed)
    ids = np.arange(n, dtype=np.int64)
    below = np.minimum(bandwidth, n - 1 - ids)
    indptr = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(below + 1, out=indptr[1:])
    nnz = int(indptr[-1])
    columns = np.repeat(ids, below + 1)
    within = np.arange(nnz, dtype=np.int64) - indptr[columns]
    indices = (columns + within).astype(np.int32)
    data = rng.uniform(low, high, nnz)
    data[indptr[:-1]] = 1.0
    return indptr.astype(np.int32), indices, data


def poisson2d_csc(nx=64, ny=64, seed=1):
    """Configuration 1: 2-D 5-point Poisson lower factor, CSC."""
    indptr, indices, data = stencil_lower_csc((nx, ny), 4.0)
    rhs = np.random.default_rng(seed).random(nx * ny)
    return Workload(
        f"poisson2d_{nx}x{ny}_csc", "sptrsv_csc", nx * ny, indptr, indices,
        data, rhs, "sync_free", seed, {"grid": (nx, ny), "levels": nx + ny - 1},
    )


def laplace3d_csc(nx=128, ny=128, nz=128, seed=2):
    """Configuration 2: 3-D 7-point Laplacian lower factor, CSC."""
    indptr, indices, data = stencil_lower_csc((nx, ny, nz), 6.0)
    rhs = np.random.default_rng(seed).random(nx * ny * nz)
    return Workload(
        f"laplace3d_{nx}x{ny}x{nz}_csc", "sptrsv_csc", nx * ny * nz, indptr,
        indices, data, rhs, "wavefront", seed,
        {"grid": (nx, ny, nz), "levels": nx + ny + nz - 2},
    )


def power_law_csr(n=1_000_000, seed=3):
    """Configuration 3: power-law random lower factor, CSR."""
    indptr, indices, data = power_law_lower_csr(n, seed=seed)
    rhs = np.random.default_rng(seed + 1000).standard_normal(n)
    return Workload(
        f"powerlaw_{n}_csr", "sptrsv_csr", n, indptr, indices, data, rhs,
        "sync_free", seed, {},
    )


def stencil9_ilu0(nx=1024, ny=1024, seed=4):
    """Configuration 4: 2-D 9-point stencil, CSR, for in-place ILU0."""
    indptr, indices, data = stencil9_csr(nx, ny, seed=seed)
    return Workload(
        f"stencil9_{nx}x{ny}_ilu0", "ilu0_csr", nx * ny, indptr, indices,
        data, None, "wavefront", seed,
        {"grid": (nx, ny), "levels": nx + 2 * ny - 2},
    )


def banded_csc(n=4_194_304, bandwidth=8, seed=5):
    """Configuration 5: long-chain banded lower factor, CSC."""
    indptr, indices, data = banded_lower_csc(n, bandwidth, seed=seed)
    rhs = np.random.default_rng(seed + 1000).random(n)
    return Workload(
        f"banded{bandwidth}_{n}_csc", "sptrsv_csc", n, indptr, indices, data,
        rhs, "sync_free", seed, {"bandwidth": bandwidth, "levels": n},
    )


CONFIGURATIONS = {
    "c1": poisson2d_csc,
    "c2": laplace3d_csc,
    "c3": power_law_csr,
    "c4": stencil9_ilu0,
    "c5": banded_csc,
}


def configuration(name, **overrides):
    """Build one of the five named configurations (optionally down-sized)."""
    return CONFIGURATIONS[name](**overrides)

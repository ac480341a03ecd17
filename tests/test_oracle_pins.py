"""Pins for the CPU oracle (no GPU).

The oracle is only trusted after it reproduces (a) every known-answer vector
the reference's own tests hold for this path, (b) closed forms and library
routines that a plausible mistake would violate, and (c) a literal set-based
restatement of the generated inspector on random small inputs.
"""

import json
import os

import numpy as np
import pytest

from lcd_amd import workloads
from oracle import lcd_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden",
                      "reference_vectors.json")


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as handle:
        return json.load(handle)


def test_reference_dag_vectors(golden):
    for case in golden["dag_cases"]:
        if case["rule"] == "ilu0_csc":       # two rules, one relational
            rules = O.rules_ilu0_csc(case["ptr"], case["idx"])
        else:
            rules = [getattr(O, "rule_" + case["rule"])(case["ptr"],
                                                        case["idx"])]
        dag = O.dag_build(rules, case["n"])
        assert dag.successors() == case["dag"], case["name"]
        assert dag.dep_count.tolist() == case["dep_count"], case["name"]
        if "dag_ptr" in case:
            assert dag.dag_ptr.tolist() == case["dag_ptr"]
            assert dag.dag_index.tolist() == case["dag_index"]
        if "wavefronts" in case:
            assert dag.wavefront_list() == case["wavefronts"], case["name"]
        if "wavefront_ptr" in case:
            assert dag.wavefronts.tolist() == case["wavefronts_flat"]
            assert dag.wavefront_ptr.tolist() == case["wavefront_ptr"]


def test_reference_cycle_vector(golden):
    dag = O.dag_from_successors(golden["cyclic_dag"]["successors"])
    assert dag.scheduled < dag.n      # the reference raises "may contain a cycle"


def test_reference_lookup_vectors(golden):
    for case in golden["lookup_cases"]:
        status, positions = O.lookup_positions(case["ptr"], case["idx"])
        if "error" in case:
            assert status == 2
        else:
            assert status == 0 and positions.tolist() == case["positions"]


@pytest.mark.parametrize("seed", range(6))
def test_inspector_matches_literal_restatement(seed):
    """Random, unsorted segments with duplicates; all rule shapes."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 60))
    counts = rng.integers(0, 7, n)
    ptr = np.zeros(n + 1, dtype=np.int32)
    np.cumsum(counts, out=ptr[1:])
    idx = rng.integers(0, n, int(ptr[-1])).astype(np.int32)
    sorted_idx = idx.copy()
    for s in range(n):
        sorted_idx[ptr[s]:ptr[s + 1]].sort()
    rules = [
        O.make_rule(ptr, idx, True, guard=O.GUARD_GREATER),
        O.make_rule(ptr, idx, False, guard=O.GUARD_GREATER),
        O.make_rule(ptr, idx, True, guard=O.GUARD_NOT_EQUAL),
        O.make_rule(ptr, sorted_idx, False, guard=O.GUARD_NONE,
                    break_at_owner=True),
    ]
    for rule in rules:
        acyclic = rule["guard"] == O.GUARD_GREATER or rule["break_at_owner"]
        dag = O.dag_build([rule], n)
        successors, dep_count, edge_count = O.literal_extract_dag(
            rule, n, "sync_free", edge_multiplicity=True)
        assert dag.successors() == successors
        assert dag.dep_count.tolist() == dep_count
        assert dag.edge_count.tolist() == edge_count
        levels = O.literal_wavefronts_from_dag(successors, dep_count)
        assert dag.wavefront_list() == levels
        if acyclic:
            assert dag.scheduled == n
            # Kahn levels are longest-path levels
            level_of = dag.level_of
            for v, nbrs in enumerate(successors):
                for w in nbrs:
                    assert level_of[w] > level_of[v]
            for w in range(n):
                preds = [v for v in range(n) if w in successors[v]]
                expected = 1 + max((level_of[v] for v in preds), default=-1)
                assert level_of[w] == expected


def test_offsets_select_the_segment_part():
    """lower/upper offsets: CSC skips the leading diagonal, CSR the trailing."""
    csc = O.dag_build([O.rule_sptrsv_csc([0, 2, 3], [0, 1, 1])], 2)
    assert csc.successors() == [[1], []]
    csr = O.dag_build([O.rule_sptrsv_csr([0, 1, 3], [0, 0, 1])], 2)
    assert csr.successors() == [[1], []]
    # without the offsets the diagonal is examined too (and rejected by the
    # strict guard), so the result is the same; a wrong sign would add (1,0)
    wrong = O.dag_build([O.make_rule([0, 1, 3], [0, 0, 1], True)], 2)
    assert wrong.successors() == [[], []]


@pytest.mark.parametrize("shape", [(7, 5), (4, 5, 3), (9,)])
def test_stencil_closed_forms(shape):
    """Level of a grid node is the sum of its coordinates; in-degree counts
    its lower neighbours; successors are id + stride."""
    ptr, idx, _ = workloads.stencil_lower_csc(shape, 2.0 * len(shape))
    n = int(np.prod(shape))
    dag = O.dag_build([O.rule_sptrsv_csc(ptr, idx)], n)
    ids = np.arange(n)
    coords, stride = [], 1
    for d in shape:
        coords.append((ids // stride) % d)
        stride *= d
    np.testing.assert_array_equal(dag.level_of, sum(coords))
    np.testing.assert_array_equal(dag.dep_count,
                                  sum((c > 0).astype(int) for c in coords))
    assert dag.levels == sum(shape) - len(shape) + 1
    assert dag.edges == sum(
        (shape[d] - 1) * n // shape[d] for d in range(len(shape)))
    # inside a level node ids ascend
    for k in range(dag.levels):
        level = dag.wavefronts[dag.wavefront_ptr[k]:dag.wavefront_ptr[k + 1]]
        assert np.all(np.diff(level) > 0)


def test_configuration_sizes_match_the_published_table():
    c1 = workloads.configuration("c1")
    assert (c1.n, c1.nnz, c1.algorithmic_bytes) == (4096, 12160, 227844)
    c5 = workloads.configuration("c5", n=4096)
    assert c5.nnz == 4096 * 9 - 36
    c4 = workloads.configuration("c4", nx=32, ny=16)
    assert c4.nnz == 32 * 16 + 2 * 31 * 16 + 2 * 32 * 15 + 4 * 31 * 15
    c3 = workloads.configuration("c3", n=5000)
    for row in (1, 17, 4999):
        cols = c3.indices[c3.indptr[row]:c3.indptr[row + 1]]
        assert cols[-1] == row and np.all(np.diff(cols) > 0)
        values = c3.data[c3.indptr[row]:c3.indptr[row + 1]]
        assert values[-1] == pytest.approx(1 + np.abs(values[:-1]).sum())


def test_banded_and_ilu_closed_forms():
    ptr, idx, _ = workloads.banded_lower_csc(300, 8)
    dag = O.dag_build([O.rule_sptrsv_csc(ptr, idx)], 300)
    np.testing.assert_array_equal(dag.dep_count,
                                  np.minimum(np.arange(300), 8))
    np.testing.assert_array_equal(dag.level_of, np.arange(300))
    nx, ny = 9, 7
    ptr, idx, _ = workloads.stencil9_csr(nx, ny)
    dag = O.dag_build([O.rule_ilu0_csr(ptr, idx)], nx * ny)
    ids = np.arange(nx * ny)
    x, y = ids % nx, ids // nx
    np.testing.assert_array_equal(dag.level_of, x + 2 * y)
    assert dag.levels == nx + 2 * ny - 2


def test_sptrsv_against_scipy_and_dense():
    from scipy.sparse import csc_matrix, csr_matrix
    from scipy.sparse.linalg import spsolve_triangular
    work = workloads.configuration("c2", nx=6, ny=5, nz=4)
    matrix = csc_matrix((work.data, work.indices, work.indptr),
                        shape=(work.n, work.n))
    x = O.sptrsv_csc(work.indptr, work.indices, work.data, work.rhs, work.n)
    np.testing.assert_allclose(
        x, spsolve_triangular(matrix.tocsr(), work.rhs, lower=True),
        rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(x, np.linalg.solve(matrix.toarray(), work.rhs),
                               rtol=1e-12, atol=1e-13)
    np.testing.assert_array_equal(
        x, O.literal_sptrsv_csc(work.indptr, work.indices, work.data,
                                work.rhs, work.n))
    work = workloads.configuration("c3", n=300)
    matrix = csr_matrix((work.data, work.indices, work.indptr),
                        shape=(work.n, work.n))
    x = O.sptrsv_csr(work.indptr, work.indices, work.data, work.rhs, work.n)
    np.testing.assert_allclose(x, np.linalg.solve(matrix.toarray(), work.rhs),
                               rtol=1e-11, atol=1e-12)
    np.testing.assert_array_equal(
        x, O.literal_sptrsv_csr(work.indptr, work.indices, work.data,
                                work.rhs, work.n))
    # special cases: diagonal matrix, unit bidiagonal recurrence
    n = 50
    d = np.linspace(1, 2, n)
    b = np.arange(n, dtype=float)
    np.testing.assert_array_equal(
        O.sptrsv_csc(np.arange(n + 1), np.arange(n), d, b, n), b / d)
    ptr, idx, val = workloads.banded_lower_csc(n, 1, seed=3)
    x = O.sptrsv_csc(ptr, idx, val, b, n)
    expected = np.zeros(n)
    for i in range(n):
        expected[i] = b[i] - (val[ptr[i - 1] + 1] * expected[i - 1] if i else 0)
    np.testing.assert_allclose(x, expected, rtol=1e-14)


def test_ilu0_against_dense_lu_and_pattern_identity():
    rng = np.random.default_rng(2)
    n = 20
    dense = rng.uniform(-1, 1, (n, n)) + n * np.eye(n)
    indptr = np.arange(0, n * n + 1, n, dtype=np.int32)
    indices = np.tile(np.arange(n, dtype=np.int32), n)
    factors = O.ilu0_csr(dense.ravel(), indices, indptr).reshape(n, n)
    doolittle = dense.copy()
    for k in range(n):
        doolittle[k + 1:, k] /= doolittle[k, k]
        doolittle[k + 1:, k + 1:] -= np.outer(doolittle[k + 1:, k],
                                              doolittle[k, k + 1:])
    np.testing.assert_allclose(factors, doolittle, rtol=1e-12, atol=1e-13)
    # sparse pattern: (L U)[i, j] == A[i, j] on the pattern
    work = workloads.configuration("c4", nx=11, ny=9)
    from scipy.sparse import csr_matrix
    result = O.ilu0_csr(work.data, work.indices, work.indptr)
    np.testing.assert_array_equal(
        result, O.literal_ilu0_csr(work.data.copy(), work.indices.tolist(),
                                   work.indptr.tolist()))
    a = csr_matrix((work.data, work.indices, work.indptr),
                   shape=(work.n, work.n)).toarray()
    f = csr_matrix((result, work.indices, work.indptr),
                   shape=(work.n, work.n)).toarray()
    product = (np.tril(f, -1) + np.eye(work.n)) @ np.triu(f)
    mask = a != 0
    np.testing.assert_allclose(product[mask], a[mask], rtol=1e-12, atol=1e-12)
    # tridiagonal: Thomas recurrence
    n = 12
    main, off = np.full(n, 4.0), np.full(n - 1, -1.0)
    tri = csr_matrix(np.diag(main) + np.diag(off, 1) + np.diag(off, -1))
    tri.sort_indices()
    out = O.ilu0_csr(tri.data, tri.indices, tri.indptr)
    pivots = [4.0]
    for _ in range(n - 1):
        pivots.append(4.0 - 1.0 / pivots[-1])
    diag = csr_matrix((out, tri.indices, tri.indptr), shape=(n, n)).diagonal()
    np.testing.assert_allclose(diag, pivots, rtol=1e-14)


def test_ilu0_csc_against_dense_lu_row_form_and_inspector():
    from scipy.sparse import csc_matrix, csr_matrix
    # dense pattern: ILU0 is LU without pivoting, whatever the storage
    rng = np.random.default_rng(12)
    n = 17
    dense = rng.uniform(-1, 1, (n, n)) + n * np.eye(n)
    indptr = np.arange(0, n * n + 1, n, dtype=np.int32)
    indices = np.tile(np.arange(n, dtype=np.int32), n)
    factors = O.ilu0_csc(dense.T.ravel(), indices, indptr).reshape(n, n).T
    doolittle = dense.copy()
    for k in range(n):
        doolittle[k + 1:, k] /= doolittle[k, k]
        doolittle[k + 1:, k + 1:] -= np.outer(doolittle[k + 1:, k],
                                              doolittle[k, k + 1:])
    np.testing.assert_allclose(factors, doolittle, rtol=1e-12, atol=1e-13)
    # sparse, unsymmetric pattern: the column form and the row form compute
    # the same incomplete factor (different operation order, so a tolerance)
    pattern = (rng.random((40, 40)) < 0.15) | np.eye(40, dtype=bool)
    a = np.where(pattern, rng.uniform(-1, 1, (40, 40)), 0.0) + 8 * np.eye(40)
    by_column, by_row = csc_matrix(a), csr_matrix(a)
    by_column.sort_indices(), by_row.sort_indices()
    column_factor = csc_matrix(
        (O.ilu0_csc(by_column.data, by_column.indices, by_column.indptr),
         by_column.indices, by_column.indptr), shape=a.shape).toarray()
    row_factor = csr_matrix(
        (O.ilu0_csr(by_row.data, by_row.indices, by_row.indptr),
         by_row.indices, by_row.indptr), shape=a.shape).toarray()
    np.testing.assert_allclose(column_factor, row_factor, rtol=1e-12,
                               atol=1e-14)
    assert np.array_equal(column_factor != 0, a != 0)
    # zero pivot: the column is left unscaled and pushes no update
    singular = np.array([[0.0, 1.0], [2.0, 3.0]])
    ptr, idx = np.array([0, 2, 4], np.int32), np.array([0, 1, 0, 1], np.int32)
    np.testing.assert_array_equal(
        O.ilu0_csc(singular.T.ravel(), idx, ptr), singular.T.ravel())
    # inspector: both rules against the literal set-based enumeration
    rules = O.rules_ilu0_csc(by_column.indptr, by_column.indices)
    dag = O.dag_build(rules, 40)
    successors, dep_count = O.literal_extract_dag(rules, 40)
    assert dag.successors() == successors
    assert dag.successors() == [list(range(k + 1, 40)) for k in range(40)]
    assert dag.dep_count.tolist() == dep_count == list(range(40))
    assert dag.levels == 40


def test_band_chains_against_literal():
    rng = np.random.default_rng(4)
    for band_width in (1, 2, 3, 5):
        work = workloads.configuration("c2", nx=5, ny=4, nz=3)
        dag = O.dag_build([O.rule_sptrsv_csc(work.indptr, work.indices)],
                          work.n)
        nodes, ptr, bands = dag.band_chains(band_width)
        expected = O.literal_band_chains(
            dag.wavefronts.tolist(), dag.wavefront_ptr.tolist(),
            dag.dag_ptr.tolist(), dag.dag_index.tolist(), band_width)
        assert nodes.tolist() == expected[0]
        assert ptr.tolist() == expected[1]
        assert bands.tolist() == expected[2]
    del rng


def _components_per_band(dag, band_width):
    """Chain tasks from first principles: cut the level sets into bands of
    ``band_width`` levels, take the subgraph the band's nodes induce, and let
    SciPy label its connected components (undirected).  A chain is one
    component, members in band order (level, then id); chains are listed by
    their first member."""
    from scipy.sparse import coo_matrix
    from scipy.sparse.csgraph import connected_components
    sources = np.repeat(np.arange(dag.n), np.diff(dag.dag_ptr))
    targets = dag.dag_index
    nodes, ptr, bands = [], [0], [0]
    for first in range(0, dag.levels, band_width):
        last = min(first + band_width, dag.levels)
        band = dag.wavefronts[dag.wavefront_ptr[first]:dag.wavefront_ptr[last]]
        position = np.full(dag.n, -1)
        position[band] = np.arange(len(band))
        inside = (position[sources] >= 0) & (position[targets] >= 0)
        graph = coo_matrix(
            (np.ones(int(inside.sum())),
             (position[sources[inside]], position[targets[inside]])),
            shape=(len(band), len(band)))
        count, label = connected_components(graph, directed=False)
        first_member = np.full(count, len(band))
        np.minimum.at(first_member, label, np.arange(len(band)))
        for component in np.argsort(first_member):
            members = band[label == component]
            nodes.extend(members.tolist())
            ptr.append(len(nodes))
        bands.append(len(ptr) - 1)
    return nodes, ptr, bands


@pytest.mark.parametrize("case", ["stencil", "ilu", "random", "banded"])
def test_band_chains_are_connected_components(case):
    rng = np.random.default_rng(21)
    if case == "stencil":
        work = workloads.configuration("c2", nx=6, ny=5, nz=4)
        rule = O.rule_sptrsv_csc(work.indptr, work.indices)
        n = work.n
    elif case == "ilu":
        work = workloads.configuration("c4", nx=9, ny=7)
        rule = O.rule_ilu0_csr(work.indptr, work.indices)
        n = work.n
    elif case == "banded":
        work = workloads.configuration("c5", n=300)
        rule = O.rule_sptrsv_csc(work.indptr, work.indices)
        n = work.n
    else:
        n = 400
        counts = rng.integers(0, 3, n)
        ptr = np.zeros(n + 1, dtype=np.int32)
        np.cumsum(counts, out=ptr[1:])
        idx = np.minimum(np.repeat(np.arange(n), counts)
                         + rng.integers(1, 60, int(ptr[-1])),
                         n - 1).astype(np.int32)
        rule = O.make_rule(ptr, idx, True, guard=O.GUARD_GREATER)
    dag = O.dag_build([rule], n)
    for band_width in (1, 2, 3, 7, 10 ** 6):
        nodes, ptr, bands = dag.band_chains(band_width)
        expected = _components_per_band(dag, band_width)
        assert nodes.tolist() == expected[0], (case, band_width)
        assert ptr.tolist() == expected[1], (case, band_width)
        assert bands.tolist() == expected[2], (case, band_width)


def test_ilu0_flop_count():
    """The oracle's operation count of ILU0 against the dense closed form
    (every k < i: one division and n - 1 - k multiply-subtracts) and against
    the sparse pattern algebra of the workload generator."""
    n = 9
    indptr = np.arange(0, n * n + 1, n, dtype=np.int32)
    indices = np.tile(np.arange(n, dtype=np.int32), n)
    closed = sum(1 + 2 * (n - 1 - k) for i in range(n) for k in range(i))
    assert O.ilu0_csr_flops(indices, indptr) == closed
    assert workloads.ilu0_true_flops(indptr, indices, n) == closed
    # tridiagonal: one division and one update per row after the first
    rows = 50
    work_ptr = np.concatenate([[0], np.cumsum(
        [2] + [3] * (rows - 2) + [2])]).astype(np.int32)
    work_idx = np.concatenate(
        [[0, 1]] + [[i - 1, i, i + 1] for i in range(1, rows - 1)]
        + [[rows - 2, rows - 1]]).astype(np.int32)
    assert O.ilu0_csr_flops(work_idx, work_ptr) == 3 * (rows - 1)
    for nx, ny in ((7, 5), (16, 11)):
        work = workloads.configuration("c4", nx=nx, ny=ny)
        assert O.ilu0_csr_flops(work.indices, work.indptr) == work.true_flops


def test_gauss_seidel_is_repeated_forward_substitution():
    work = workloads.configuration("c4", nx=6, ny=5)
    from scipy.sparse import csr_matrix, tril
    matrix = csr_matrix((work.data, work.indices, work.indptr),
                        shape=(work.n, work.n))
    strict = tril(matrix, -1, format="csr")
    strict.sort_indices()
    diagonal = matrix.diagonal()
    b = np.linspace(0, 1, work.n)
    x = O.gauss_seidel_csr(strict.indptr, strict.indices, strict.data,
                           diagonal, b, np.zeros(work.n), work.n, 1)
    lower = (strict + csr_matrix(np.diag(diagonal))).toarray()
    np.testing.assert_allclose(x, np.linalg.solve(lower, b), rtol=1e-12)

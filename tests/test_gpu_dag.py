"""On-device inspector vs the CPU oracle: bit-exact edges, counts, levels."""

import json
import os

import numpy as np
import pytest

from lcd_amd import hip_runtime, workloads

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden",
                      "reference_vectors.json")


def _check_dag(device, oracle, rule, n, force_kahn=False):
    expected = oracle.dag_build([rule], n)
    dag = device.dag_build([rule], n, levels=True, force_kahn=force_kahn)
    assert dag.n == n
    assert dag.edges == expected.edges
    np.testing.assert_array_equal(dag.host("dag_ptr"), expected.dag_ptr)
    np.testing.assert_array_equal(dag.host("dag_index"), expected.dag_index)
    np.testing.assert_array_equal(dag.host("dep_count"), expected.dep_count)
    np.testing.assert_array_equal(dag.host("edge_count"), expected.edge_count)
    assert dag.levels == expected.levels
    assert dag.scheduled == expected.scheduled == n
    np.testing.assert_array_equal(dag.host("level_of"), expected.level_of)
    np.testing.assert_array_equal(dag.host("wavefronts"), expected.wavefronts)
    np.testing.assert_array_equal(dag.host("wavefront_ptr"),
                                  expected.wavefront_ptr)
    return dag, expected


def _rule_for(oracle, work):
    if work.kind == "sptrsv_csc":
        return oracle.rule_sptrsv_csc(work.indptr, work.indices)
    if work.kind == "sptrsv_csr":
        return oracle.rule_sptrsv_csr(work.indptr, work.indices)
    return oracle.rule_ilu0_csr(work.indptr, work.indices)


SMALL = [
    ("c1", {}),
    ("c2", dict(nx=24, ny=20, nz=18)),
    ("c3", dict(n=30000)),
    ("c4", dict(nx=96, ny=80)),
    ("c5", dict(n=50000)),
]


@pytest.mark.parametrize("name,overrides", SMALL)
@pytest.mark.parametrize("force_kahn", [False, True])
def test_dag_matches_oracle(device, oracle, name, overrides, force_kahn):
    if force_kahn and name == "c5":
        overrides = dict(n=3000)   # one launch per level: keep the chain short
    work = workloads.configuration(name, **overrides)
    print("dag", name, overrides, "kahn" if force_kahn else "sweep", flush=True)
    dag, _ = _check_dag(device, oracle, _rule_for(oracle, work), work.n,
                        force_kahn)
    assert dag.level_algorithm == (1 if force_kahn else 2)
    if "levels" in work.meta and not overrides.get("n"):
        grid = work.meta.get("grid")
        if grid is not None and name in ("c1", "c2"):
            assert dag.levels == sum(grid) - len(grid) + 1


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_dag_matches_oracle_at_full_size(device, oracle, name):
    """BASELINE.json's sizes: edges, unique in-degrees, multiplicities, CSR
    successors, levels and level sets bit-exact against the oracle, plus the
    closed forms the stencils and the band have."""
    work = workloads.configuration(name)
    print("dag full size", name, work.n, work.nnz, flush=True)
    dag, expected = _check_dag(device, oracle, _rule_for(oracle, work), work.n)
    grid = work.meta.get("grid")
    if name in ("c1", "c2"):
        assert dag.levels == sum(grid) - len(grid) + 1
        coordinates = np.unravel_index(np.arange(work.n), grid[::-1])
        np.testing.assert_array_equal(dag.host("level_of"),
                                      sum(coordinates).astype(np.int32))
    elif name == "c4":
        nx, ny = grid
        assert dag.levels == nx + 2 * ny - 2
    elif name == "c5":
        assert dag.levels == work.n
        np.testing.assert_array_equal(
            dag.host("dep_count"),
            np.minimum(np.arange(work.n), work.meta["bandwidth"]))
    assert dag.edges == expected.edges == int(dag.host("dep_count").sum())
    dag.destroy()


@pytest.mark.parametrize("name,overrides", SMALL)
def test_band_chains_match_oracle(device, oracle, name, overrides):
    """Chain tasks (band_width > 1): connected components inside bands of
    levels, listed by first member, members in (level, id) order."""
    if name == "c5":
        overrides = dict(n=4000)
    work = workloads.configuration(name, **overrides)
    rule = _rule_for(oracle, work)
    dag = device.dag_build([rule], work.n, levels=True)
    expected = oracle.dag_build([rule], work.n)
    for width in (1, 2, 3, 7, 64, 10 ** 6):
        print("chains", name, overrides, width, flush=True)
        tasks, bands = dag.band_chains(width)
        nodes, ptr, band_ptr = expected.band_chains(width)
        assert tasks == len(ptr) - 1 and bands == len(band_ptr) - 1
        np.testing.assert_array_equal(dag.host("task_nodes"), nodes)
        np.testing.assert_array_equal(dag.host("task_ptr"), ptr)
        np.testing.assert_array_equal(dag.host("band_ptr"), band_ptr)
    # width 1: every node is its own chain, bands are the levels
    dag.band_chains(1)
    np.testing.assert_array_equal(dag.host("task_nodes"), dag.host("wavefronts"))
    np.testing.assert_array_equal(dag.host("task_ptr"), np.arange(work.n + 1))
    np.testing.assert_array_equal(dag.host("band_ptr"), dag.host("wavefront_ptr"))
    with pytest.raises(Exception, match="positive integer"):
        dag.band_chains(0)


def test_band_chains_of_a_random_dag(device, oracle):
    rng = np.random.default_rng(11)
    n = 5000
    counts = rng.integers(0, 4, n)
    ptr = np.zeros(n + 1, dtype=np.int32)
    np.cumsum(counts, out=ptr[1:])
    idx = np.minimum(np.repeat(np.arange(n), counts)
                     + rng.integers(1, 40, int(ptr[-1])), n - 1).astype(np.int32)
    rule = oracle.make_rule(ptr, idx, True, guard=oracle.GUARD_GREATER)
    dag = device.dag_build([rule], n, levels=True)
    expected = oracle.dag_build([rule], n)
    for width in (2, 5, 33):
        dag.band_chains(width)
        nodes, task_ptr, band_ptr = expected.band_chains(width)
        np.testing.assert_array_equal(dag.host("task_nodes"), nodes)
        np.testing.assert_array_equal(dag.host("task_ptr"), task_ptr)
        np.testing.assert_array_equal(dag.host("band_ptr"), band_ptr)


def test_chain_rule_matches_oracle(device, oracle):
    """LCDHIP_RULE_NEXT: seg -> seg + offset, alone and beside a segment
    rule (duplicates of an edge the other rule already yields are merged)."""
    for n, offset in ((1, 1), (2, 1), (1000, 1), (1000, 3), (5, 7)):
        expected = oracle.dag_build([oracle.rule_next(offset)], n)
        dag = device.dag_build([oracle.rule_next(offset)], n, levels=True)
        assert dag.edges == expected.edges == max(n - offset, 0)
        for name in ("dag_ptr", "dag_index", "dep_count", "edge_count",
                     "level_of", "wavefronts", "wavefront_ptr"):
            np.testing.assert_array_equal(dag.host(name),
                                          getattr(expected, name))
    work = workloads.configuration("c5", n=3000)
    rules = [oracle.rule_sptrsv_csc(work.indptr, work.indices),
             oracle.rule_next(1)]
    expected = oracle.dag_build(rules, work.n)
    dag = device.dag_build(rules, work.n, levels=True)
    assert dag.edges == expected.edges
    np.testing.assert_array_equal(dag.host("dag_index"), expected.dag_index)
    np.testing.assert_array_equal(dag.host("edge_count"), expected.edge_count)
    np.testing.assert_array_equal(dag.host("level_of"), expected.level_of)
    with pytest.raises(hip_runtime.HIPRuntimeError, match="chain rule"):
        device.dag_build([dict(relation=2, lower_offset=0)], 10)


@pytest.mark.parametrize("gap", [1, 63, 64, 1234, 2999])
def test_levels_behind_a_chain_prefix(device, oracle, gap):
    """The level sweep skips the longest prefix in which every node follows
    its predecessor in the numbering (level = id there); behind the first
    node that does not, levels come from the sweep."""
    import scipy.sparse as sp
    work = workloads.configuration("c5", n=3000)
    matrix = sp.csc_matrix((work.data, work.indices, work.indptr),
                           shape=(work.n, work.n)).tolil()
    matrix[gap:, gap - 1] = 0.0        # node `gap` loses the predecessor gap - 1
    matrix = matrix.tocsc()
    matrix.eliminate_zeros()
    matrix.sort_indices()
    rule = oracle.rule_sptrsv_csc(matrix.indptr.astype(np.int32),
                                  matrix.indices.astype(np.int32))
    print("chain prefix", gap, flush=True)
    dag, expected = _check_dag(device, oracle, rule, work.n)
    assert dag.levels < work.n


def test_golden_vectors(device, oracle):
    with open(GOLDEN) as handle:
        golden = json.load(handle)
    for case in golden["dag_cases"]:
        if case["rule"] == "ilu0_csc":
            rules = oracle.rules_ilu0_csc(case["ptr"], case["idx"])
        else:
            rules = [getattr(oracle, "rule_" + case["rule"])(case["ptr"],
                                                             case["idx"])]
        dag = device.dag_build(rules, case["n"], levels=True)
        assert dag.successors() == case["dag"], case["name"]
        assert dag.host("dep_count").tolist() == case["dep_count"], case["name"]
        if "dag_ptr" in case:
            assert dag.host("dag_ptr").tolist() == case["dag_ptr"]
            assert dag.host("dag_index").tolist() == case["dag_index"]
        if "wavefronts" in case:
            assert dag.wavefront_list() == case["wavefronts"], case["name"]


@pytest.mark.parametrize("n,offset", [(1, 1), (2, 1), (67, 1), (300, 1),
                                      (300, 7), (5, 9)])
def test_relational_rule(device, oracle, n, offset):
    """``seg -> every j >= seg + offset`` beside a segment rule (the two
    rules of CSC ILU0), against the oracle's enumeration."""
    print("relational rule", n, offset, flush=True)
    work = workloads.configuration("c3", n=n, seed=n + offset)
    rules = [oracle.make_rule(work.indptr, work.indices, False,
                              upper_offset=-1),
             oracle.rule_later(offset)]
    expected = oracle.dag_build(rules, n)
    for force_kahn in (False, True):
        dag = device.dag_build(rules, n, levels=True, force_kahn=force_kahn)
        for name in ("dag_ptr", "dag_index", "dep_count", "edge_count",
                     "level_of", "wavefronts", "wavefront_ptr"):
            np.testing.assert_array_equal(dag.host(name),
                                          getattr(expected, name), name)
        assert dag.topological_ids
    if offset == 1:
        assert dag.levels == n and dag.edges == n * (n - 1) // 2
    with pytest.raises(hip_runtime.HIPRuntimeError):
        device.dag_build(rules, n, incoming=True)
    with pytest.raises(hip_runtime.HIPRuntimeError):
        device.dag_build([dict(relation=1, lower_offset=0)], n)
    with pytest.raises(hip_runtime.HIPRuntimeError):
        device.dag_build([oracle.rule_later(1)], 70000)


@pytest.mark.parametrize("lanes,tile_rows", [(4, 512), (2, 100), (8, None)])
def test_task_records(device, oracle, lanes, tile_rows):
    """Fixed-size records of the incoming listing in executor order."""
    print("task records", lanes, tile_rows, flush=True)
    work = workloads.configuration("c2", nx=12, ny=10, nz=9)
    rule = oracle.rule_sptrsv_csc(work.indptr, work.indices)
    dag = device.dag_build([rule], work.n, levels=True, incoming=True)
    if tile_rows:
        dag.tile_order(tile_rows)
    if not tile_rows:
        with pytest.raises(hip_runtime.HIPRuntimeError):
            dag.task_records(lanes, tiled=True)     # no tile order yet
    rec_in, rec_src, rec_pos = (
        a.copy_to_host()
        for a in dag.task_records(lanes, tiled=bool(tile_rows)))
    order = dag.host("tile_nodes" if tile_rows else "wavefronts")
    in_ptr, in_src, in_pos = (dag.host(name)
                              for name in ("in_ptr", "in_src", "in_pos"))
    np.testing.assert_array_equal(rec_in.reshape(-1, 2)[:, 0], in_ptr[order])
    np.testing.assert_array_equal(rec_in.reshape(-1, 2)[:, 1],
                                  in_ptr[order + 1])
    expected_src = np.zeros((work.n, lanes), dtype=np.int32)
    expected_pos = np.zeros((work.n, lanes), dtype=np.int32)
    for q, node in enumerate(order):
        count = min(in_ptr[node + 1] - in_ptr[node], lanes)
        expected_src[q, :count] = in_src[in_ptr[node]:in_ptr[node] + count]
        expected_pos[q, :count] = in_pos[in_ptr[node]:in_ptr[node] + count]
    np.testing.assert_array_equal(rec_src.reshape(-1, lanes), expected_src)
    np.testing.assert_array_equal(rec_pos.reshape(-1, lanes), expected_pos)
    assert dag.record_overflow == int(np.sum(np.diff(in_ptr) > lanes))
    with pytest.raises(hip_runtime.HIPRuntimeError):
        dag.task_records(0)
    plain = device.dag_build([rule], work.n, levels=True)
    with pytest.raises(hip_runtime.HIPRuntimeError):
        plain.task_records(lanes)          # no incoming listing


@pytest.mark.parametrize("grid,box", [((12, 10, 9), (4, 5, 3)),
                                      ((12, 10, 9), (8, 4, 4)),     # ragged
                                      ((16, 6, 1), (4, 2, 1)),
                                      ((7, 5, 3), (7, 5, 3))])
def test_box_order_and_position_records(device, oracle, grid, box):
    """Tiles over boxes of a grid: the task order is (box, level, id) with
    boxes in (z, y, x) order -- restated here with numpy from the level sets
    -- its inverse, and task records that name sources by their place in that
    order; every source comes before its consumer."""
    print("box order", grid, box, flush=True)
    nx, ny, nz = grid
    work = workloads.configuration("c2", nx=nx, ny=ny, nz=nz)
    rule = oracle.rule_sptrsv_csc(work.indptr, work.indices)
    dag = device.dag_build([rule], work.n, levels=True, incoming=True)
    with pytest.raises(hip_runtime.HIPRuntimeError):
        dag.task_records(4, tiled=hip_runtime.RECORDS_TILE_POSITIONS)
    order = dag.box_order(grid, box).copy_to_host()
    ids = np.arange(work.n)
    x, y, z = ids % nx, ids // nx % ny, ids // (nx * ny)
    boxes_x, boxes_y = -(-nx // box[0]), -(-ny // box[1])
    box_of = ((z // box[2]) * boxes_y + y // box[1]) * boxes_x + x // box[0]
    level_of = dag.host("level_of")
    expected = np.lexsort((ids, level_of, box_of))
    np.testing.assert_array_equal(order, expected)
    position = dag.host("tile_pos")
    np.testing.assert_array_equal(position[order], ids)
    lanes = 4
    rec_in, rec_src, rec_pos = (
        a.copy_to_host() for a in dag.task_records(
            lanes, tiled=hip_runtime.RECORDS_TILE_POSITIONS))
    in_ptr, in_src, in_pos = (dag.host(name)
                              for name in ("in_ptr", "in_src", "in_pos"))
    expected_src = np.zeros((work.n, lanes), dtype=np.int32)
    expected_pos = np.zeros((work.n, lanes), dtype=np.int32)
    for q, node in enumerate(order):
        count = min(in_ptr[node + 1] - in_ptr[node], lanes)
        sources = in_src[in_ptr[node]:in_ptr[node] + count]
        expected_src[q, :count] = position[sources]
        assert np.all(position[sources] < q)
        expected_pos[q, :count] = in_pos[in_ptr[node]:in_ptr[node] + count]
    np.testing.assert_array_equal(rec_src.reshape(-1, lanes), expected_src)
    np.testing.assert_array_equal(rec_pos.reshape(-1, lanes), expected_pos)
    assert dag.record_overflow == 0
    with pytest.raises(hip_runtime.HIPRuntimeError):
        dag.box_order((nx, ny, nz + 1), box)         # not n nodes
    with pytest.raises(hip_runtime.HIPRuntimeError):
        dag.box_order(grid, (0, 1, 1))


def test_position_records_refuse_an_order_that_is_not_topological(device,
                                                                  oracle):
    """A grid read with the wrong line length: an x step of the real grid
    then leads from a box to an earlier one, and the records say so instead
    of leaving an executor to wait for ever."""
    nx, ny, nz = 8, 4, 3
    work = workloads.configuration("c2", nx=nx, ny=ny, nz=nz)
    rule = oracle.rule_sptrsv_csc(work.indptr, work.indices)
    dag = device.dag_build([rule], work.n, levels=True, incoming=True)
    # boxes of four consecutive ids: any order by id is topological
    dag.box_order((nx * ny, nz, 1), (4, 1, 1))
    dag.task_records(4, tiled=hip_runtime.RECORDS_TILE_POSITIONS)  # still fine
    # lines of four: the edge 3 -> 4 goes from box 1 back to box 0
    dag.box_order((4, 2, 12), (2, 2, 1))
    with pytest.raises(hip_runtime.HIPRuntimeError, match="topological"):
        dag.task_records(4, tiled=hip_runtime.RECORDS_TILE_POSITIONS)


def test_edge_offsets(device, oracle):
    """destination - source over the unique edges: 1, nx and nx * ny on the
    7-point grid, with the counts of a full stencil; what the scheduler reads
    a structured grid from."""
    from lcd_amd.scheduler import structured_grid
    nx, ny, nz = 12, 10, 9
    work = workloads.configuration("c2", nx=nx, ny=ny, nz=nz)
    rule = oracle.rule_sptrsv_csc(work.indptr, work.indices)
    dag = device.dag_build([rule], work.n, levels=True)
    offsets, counts, distinct = dag.edge_offsets(8)
    assert (offsets, distinct) == ([1, nx, nx * ny], 3)
    assert counts == [(nx - 1) * ny * nz, nx * (ny - 1) * nz,
                      nx * ny * (nz - 1)]
    assert dag.edge_offsets(2) == ([1, nx], counts[:2], 3)
    assert dag.edge_offsets(0) == ([], [], 3)
    assert structured_grid(dag) == (nx, ny, nz)
    # a general matrix: every offset against a numpy histogram
    work = workloads.configuration("c3", n=500, seed=4)
    rule = oracle.rule_sptrsv_csr(work.indptr, work.indices)
    dag = device.dag_build([rule], work.n, levels=True)
    ptr, index = dag.host("dag_ptr"), dag.host("dag_index")
    sources = np.repeat(np.arange(work.n), np.diff(ptr))
    values, expected = np.unique(index - sources, return_counts=True)
    offsets, counts, distinct = dag.edge_offsets(len(values) + 3)
    assert distinct == len(values)
    assert offsets == values.tolist() and counts == expected.tolist()
    assert structured_grid(dag) is None
    empty = device.dag_build([], 5, levels=True)
    assert empty.edge_offsets(4) == ([], [], 0)


def test_incoming_positions(device, oracle):
    """Per destination, the positions whose entries produce its edges, by
    (source, position), duplicates kept."""
    rng = np.random.default_rng(3)
    n = 3000
    counts = rng.integers(0, 9, n)
    ptr = np.zeros(n + 1, dtype=np.int32)
    np.cumsum(counts, out=ptr[1:])
    idx = rng.integers(0, n, int(ptr[-1])).astype(np.int32)
    rule = oracle.make_rule(ptr, idx, True, lower_offset=1,
                            guard=oracle.GUARD_GREATER)
    dag = device.dag_build([rule], n, levels=True, incoming=True)
    expected = [[] for _ in range(n)]
    for seg in range(n):
        for p in range(ptr[seg] + 1, ptr[seg + 1]):
            if idx[p] > seg:
                expected[idx[p]].append((seg, p))
    in_ptr, in_pos = dag.host("in_ptr"), dag.host("in_pos")
    np.testing.assert_array_equal(np.diff(in_ptr), dag.host("edge_count"))
    for v in range(n):
        want = [p for _, p in sorted(expected[v])]
        assert in_pos[in_ptr[v]:in_ptr[v + 1]].tolist() == want
    in_src = dag.host("in_src")
    want_src = [seg for v in range(n) for seg, _ in sorted(expected[v])]
    assert in_src.tolist() == want_src
    # out_slot inverts the listing; positions without an edge hold -1
    out_slot = dag.host("out_slot")
    assert len(out_slot) == len(idx)
    np.testing.assert_array_equal(out_slot[in_pos], np.arange(len(in_pos)))
    assert int((out_slot >= 0).sum()) == len(in_pos)
    assert set(out_slot[out_slot < 0].tolist()) <= {-1}
    work = workloads.configuration("c2", nx=12, ny=10, nz=9)
    dag = device.dag_build([oracle.rule_sptrsv_csc(work.indptr, work.indices)],
                           work.n, incoming=True)
    in_ptr, in_pos = dag.host("in_ptr"), dag.host("in_pos")
    assert in_ptr[-1] == dag.edges == len(in_pos)
    np.testing.assert_array_equal(work.indices[in_pos],
                                  np.repeat(np.arange(work.n), np.diff(in_ptr)))


def test_random_unsorted_duplicates(device, oracle):
    """Unsorted segments with repeated entries: set semantics + multiplicity."""
    rng = np.random.default_rng(7)
    n = 5000
    counts = rng.integers(0, 12, n)
    ptr = np.zeros(n + 1, dtype=np.int32)
    np.cumsum(counts, out=ptr[1:])
    idx = rng.integers(0, n, int(ptr[-1])).astype(np.int32)
    for owner_is_source in (True, False):
        rule = oracle.make_rule(ptr, idx, owner_is_source,
                                guard=oracle.GUARD_GREATER)
        _check_dag(device, oracle, rule, n)
        _check_dag(device, oracle, rule, n, force_kahn=True)


def test_non_topological_ids_use_frontier_levels(device, oracle):
    """Edges from high to low ids force the frontier algorithm."""
    rng = np.random.default_rng(11)
    n = 4000
    perm = rng.permutation(n)
    work_ptr, work_idx, _ = workloads.banded_lower_csc(n, 3)
    # relabel node v as perm[v]: segments stay, endpoints are permuted
    inverse = np.argsort(perm)
    order = inverse  # new id k holds old column inverse[k]
    counts = (work_ptr[1:] - work_ptr[:-1])[order]
    ptr = np.zeros(n + 1, dtype=np.int32)
    np.cumsum(counts, out=ptr[1:])
    idx = np.concatenate([
        perm[work_idx[work_ptr[c]:work_ptr[c + 1]]] for c in order
    ]).astype(np.int32)
    rule = oracle.make_rule(ptr, idx, True, lower_offset=1,
                            guard=oracle.GUARD_NOT_EQUAL)
    dag, _ = _check_dag(device, oracle, rule, n)
    assert not dag.topological_ids and dag.level_algorithm == 1


def test_cycle_is_reported(device, oracle):
    from lcd_amd.dag_preprocessing import (DAGPreprocessingError,
                                           execution_data_from_device_dag)
    ptr = np.array([0, 1, 2], dtype=np.int32)
    idx = np.array([1, 0], dtype=np.int32)
    rule = oracle.make_rule(ptr, idx, True, guard=oracle.GUARD_NONE)
    dag = device.dag_build([rule], 2, levels=True)
    assert dag.scheduled == 0 and dag.levels == 0
    with pytest.raises(DAGPreprocessingError, match="may contain a cycle"):
        execution_data_from_device_dag(dag, "wavefront", True)


def test_out_of_range_endpoint(device, oracle):
    from lcd_amd import hip_runtime
    ptr = np.array([0, 1, 2], dtype=np.int32)
    idx = np.array([1, 7], dtype=np.int32)
    rule = oracle.make_rule(ptr, idx, True, guard=oracle.GUARD_NONE)
    with pytest.raises(hip_runtime.HIPRuntimeError) as info:
        device.dag_build([rule], 2)
    assert info.value.code == hip_runtime.ERR_DAG_BOUNDS


def test_empty_and_edgeless(device, oracle):
    ptr = np.zeros(1, dtype=np.int32)
    idx = np.zeros(0, dtype=np.int32)
    dag = device.dag_build(
        [oracle.make_rule(ptr, idx, True, guard=oracle.GUARD_NONE)], 0)
    assert dag.n == 0 and dag.edges == 0 and dag.levels == 0
    n = 1000
    ptr = np.arange(n + 1, dtype=np.int32)
    idx = np.arange(n, dtype=np.int32)   # diagonal only
    dag = device.dag_build([oracle.rule_sptrsv_csc(ptr, idx)], n)
    assert dag.edges == 0 and dag.levels == 1
    np.testing.assert_array_equal(dag.host("wavefronts"), np.arange(n))


def test_lookup_table(device, oracle):
    from lcd_amd import hip_runtime
    work = workloads.configuration("c4", nx=64, ny=48)
    status, expected = oracle.lookup_positions(work.indptr, work.indices)
    assert status == 0
    table = device.lookup_build(work.indptr, work.indices).copy_to_host()
    np.testing.assert_array_equal(table, expected)
    table = device.lookup_build([0, 2, 3, 5], [0, 2, 0, 1, 2]).copy_to_host()
    assert table.tolist() == [0, -1, 4]
    with pytest.raises(hip_runtime.HIPRuntimeError) as info:
        device.lookup_build([0, 2], [1, 0])
    assert info.value.code == hip_runtime.ERR_LOOKUP_ORDER


def test_pair_lookup_table(device):
    """For every pair of entries (a, b) of a segment: where segment
    indices[a] holds the index indices[b] -- what ILU0 searches per pivot and
    updated entry -- against a literal search over the rows."""
    from lcd_amd import hip_runtime

    def literal(indptr, indices):
        n = len(indptr) - 1
        lengths = np.diff(indptr)
        base = np.zeros(n + 1, dtype=np.int64)
        np.cumsum(lengths.astype(np.int64) ** 2, out=base[1:])
        table = np.full(int(base[-1]), -1, dtype=np.int32)
        for s in range(n):
            start, length = indptr[s], lengths[s]
            for a in range(length):
                k = indices[start + a]
                if not 0 <= k < n:
                    continue
                row = indices[indptr[k]:indptr[k + 1]].tolist()
                for b in range(length):
                    key = indices[start + b]
                    if key in row:
                        table[base[s] + a * length + b] = indptr[k] + row.index(key)
        return base, table

    cases = [workloads.configuration("c4", nx=9, ny=7),
             workloads.configuration("c3", n=300, seed=5)]
    for work in cases:
        print("pair table", work.name, flush=True)
        expected_base, expected = literal(work.indptr, work.indices)
        assert device.pair_lookup_entries(work.indptr, work.indices) == len(expected)
        base, table = device.pair_lookup_build(work.indptr, work.indices)
        np.testing.assert_array_equal(base.copy_to_host(), expected_base)
        np.testing.assert_array_equal(table.copy_to_host()[:len(expected)],
                                      expected)
        # the same table in bytes: offsets from the start of the segment
        # searched (segments of at most 127 entries)
        if np.diff(work.indptr).max() <= 127:
            lengths = np.diff(work.indptr)
            searched = np.concatenate([
                np.repeat(work.indices[work.indptr[s]:work.indptr[s + 1]],
                          lengths[s]) for s in range(work.n)])
            offsets = np.where(expected < 0, -1,
                               expected - work.indptr[searched]).astype(np.int8)
            base, table = device.pair_lookup_build(work.indptr, work.indices,
                                                   offsets=True)
            assert table.dtype == np.int8
            np.testing.assert_array_equal(base.copy_to_host(), expected_base)
            np.testing.assert_array_equal(
                table.copy_to_host()[:len(expected)], offsets)
        else:
            with pytest.raises(hip_runtime.HIPRuntimeError,
                               match="127 entries"):
                device.pair_lookup_build(work.indptr, work.indices,
                                         offsets=True)
    # an empty segment, an index beyond the segments (no segment to search)
    indptr = np.array([0, 2, 2, 5], dtype=np.int32)
    indices = np.array([0, 2, 0, 1, 7], dtype=np.int32)
    base, table = device.pair_lookup_build(indptr, indices)
    assert base.copy_to_host().tolist() == [0, 4, 4, 13]
    assert table.copy_to_host()[:13].tolist() == [
        0, 1, 2, -1,                     # segment 0: rows 0 and 2 searched
        0, -1, -1, -1, -1, -1, -1, -1, -1]   # segment 2: rows 0, 1 (empty), 7
    # more than 1024 segments: the scan of the squares runs in chunks
    work = workloads.configuration("c1")
    expected_base, expected = literal(work.indptr, work.indices)
    base, table = device.pair_lookup_build(work.indptr, work.indices)
    np.testing.assert_array_equal(base.copy_to_host(), expected_base)
    np.testing.assert_array_equal(table.copy_to_host()[:len(expected)], expected)
    assert device.pair_lookup_entries([0], np.zeros(0, dtype=np.int32)) == 0
    with pytest.raises(hip_runtime.HIPRuntimeError) as info:
        device.pair_lookup_build([0, 3, 2], [0, 1, 2])
    assert info.value.code == hip_runtime.ERR_LOOKUP_POINTER


def test_digest_is_content_sensitive(device):
    a = device.to_device(np.arange(10000, dtype=np.int32))
    b = device.to_device(np.arange(10000, dtype=np.int32))
    c_host = np.arange(10000, dtype=np.int32)
    c_host[1234] += 1
    c = device.to_device(c_host)
    assert device.digest(a) == device.digest(b)
    assert device.digest(a) != device.digest(c)


def test_inspections_reuse_device_memory_safely(device, oracle):
    """The inspector keeps its device blocks for reuse (temporaries and the
    arrays of destroyed DAGs): inspections of different structures and sizes
    one after another, with DAGs alive and destroyed in between, each match
    the oracle -- nothing depends on what an earlier one left in a block.
    Power-law rows with hundreds of predecessors (read by the whole
    wavefront) and long-range edges (the narrow sweep window) are among
    them."""
    kept = []
    for round_ in range(2):
        for name, overrides in (("c3", dict(n=40000)), ("c1", {}),
                                ("c4", dict(nx=64, ny=48)),
                                ("c3", dict(n=9000)),
                                ("c2", dict(nx=16, ny=12, nz=10))):
            work = workloads.configuration(name, **overrides)
            print("dag reuse", round_, name, overrides, flush=True)
            dag, _ = _check_dag(device, oracle, _rule_for(oracle, work),
                                work.n)
            if name == "c1":
                kept.append(dag)        # stays alive across the others
            else:
                dag.destroy()
    for dag in kept:
        work = workloads.configuration("c1")
        expected = oracle.dag_build([_rule_for(oracle, work)], work.n)
        np.testing.assert_array_equal(dag.host("level_of"), expected.level_of)
        dag.destroy()
